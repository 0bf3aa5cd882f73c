"""Stochastic sampling on the device (zr_sample, zrh_decode_step_batch_sampled)
against the oracle's restatement of sample_tokens_device_with_seeds
(runtime.rs:534-601).

Bar: the device token equals the oracle's wherever the oracle's margin (the
f64 distance from tau / top_p to the nearest cumulative boundary the decision
depends on) exceeds 1e-5.  The oracle evaluates the rule in f64; the device
sums exact integer weights round(p * 2^36) of f32 probabilities, whose error
against f64 stays near 1e-6 at 128k columns, so only decisions within that of
a boundary may differ.  Such rows are a minority for small vocabularies; at
128k columns a row's probabilities are ~1e-5 each, so the boundaries around
tau are that close and about half of the rows fall inside the margin.  argmax
rows are exact.  Tokens do not depend on the run (integer sums).
"""
import numpy as np
import pytest

import oracle as O
from mesh_amd import BackendMicrobatchExecutor, DecodeMicrobatchRequest, DeviceBuffer, DeviceContext, ModelGeometry
from mesh_amd._lib import ZR_E_INVALID, ZrError
from mesh_amd.provider import sample_device
from tests.test_gpu_model import SMALL, make
from tests.testmodels import geometry, random_weights

pytestmark = pytest.mark.gpu
MARGIN = 1e-5


def _ctx(vocab=128256):
    geo = ModelGeometry(hidden=256, num_heads=4, num_kv_heads=2, num_layers=1, vocab=vocab, ffn=64)
    return DeviceContext(geo, kv_dtype="f32", max_tokens=8, max_seqs=8, max_pages_per_seq=8)


def _params(rng, rows):
    temps = rng.choice([1.0, 0.7, 1.3, 0.3, 2.0, 0.0, -1.0], rows).astype(np.float32)
    tops = rng.choice([1.0, 0.95, 0.9, 0.5, 0.05, 1.5, 0.0], rows).astype(np.float32)
    seeds = rng.integers(0, 2 ** 63, rows, dtype=np.uint64)
    return temps, tops, seeds


def _check(x, temps, tops, seeds, got):
    compared = 0
    for r in range(x.shape[0]):
        want, margin = O.sample_token_device(x[r], float(temps[r]), float(tops[r]), int(seeds[r]))
        if margin > MARGIN:
            assert got[r] == want, (r, float(temps[r]), float(tops[r]), int(seeds[r]), got[r], want, margin)
            compared += 1
    return compared


@pytest.mark.parametrize("cols,scale", [(128256, 1.0), (128256, 4.0), (32000, 2.0), (1000, 0.5), (5, 1.0)])
def test_rows_match_oracle(cols, scale):
    ctx = _ctx(cols)
    rng = np.random.default_rng(cols)
    rows = 64
    x = (rng.standard_normal((rows, cols)) * scale).astype(np.float32)
    temps, tops, seeds = _params(rng, rows)
    got = sample_device(ctx, x, temps, tops, seeds)
    compared = _check(x, temps, tops, seeds, got)
    assert compared >= (rows - 3 if cols <= 1000 else rows // 2), compared
    assert sample_device(ctx, x, temps, tops, seeds) == got  # run to run
    ctx.close()


def test_ties_and_peaked_rows():
    ctx = _ctx(4096)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((16, 4096)).astype(np.float32)
    x[0, [7, 100, 4000]] = 9.0            # three-way tie at the top: index order
    x[1, :] = 0.0                         # uniform
    x[2, 5] = 60.0                        # one token takes all the mass
    x[3, ::2] = x[3, 1::2]                # pairs of equal probabilities
    temps = np.full(16, 1.0, np.float32)
    tops = np.full(16, 0.5, np.float32)
    tops[4:8] = 1.0
    seeds = np.arange(16, dtype=np.uint64) * 7919
    got = sample_device(ctx, x, temps, tops, seeds)
    assert _check(x, temps, tops, seeds, got) >= 14
    assert got[2] == 5
    ctx.close()


@pytest.mark.parametrize("cols", [16384, 16383])
def test_large_buckets_and_long_ties(cols):
    # rows whose crossing bucket holds more than the 8192 candidates resolved in
    # LDS: uniform (one run of equal probabilities), a narrow spread of
    # distinct logits 1.2e-5 apart (refined by the next bits), a long run of
    # ties among distinct values, and quantised logits (many ties, resolved in
    # column order)
    ctx = _ctx(cols)
    rng = np.random.default_rng(cols + 1)
    kinds = 4
    per = 24
    x = np.zeros((kinds * per, cols), np.float32)
    for r in range(per):
        x[per + r] = rng.permutation(np.linspace(0.0, 0.2, cols, dtype=np.float32))
        x[2 * per + r] = rng.standard_normal(cols).astype(np.float32)
        x[2 * per + r, rng.permutation(cols)[:12000]] = 0.25
        x[3 * per + r] = (np.round(rng.standard_normal(cols) * 2) / 2).astype(np.float32)
    rows = kinds * per
    temps = rng.choice([1.0, 0.8], rows).astype(np.float32)
    tops = rng.choice([1.0, 0.9, 0.5, 0.2], rows).astype(np.float32)
    seeds = rng.integers(0, 2 ** 63, rows, dtype=np.uint64)
    got = sample_device(ctx, x, temps, tops, seeds)
    assert _check(x, temps, tops, seeds, got) >= rows // 3
    assert sample_device(ctx, x, temps, tops, seeds) == got
    ctx.close()


def test_device_tokens_equal_host_sampler_small_vocab():
    # away from decision boundaries the device sampler returns the host
    # sampler's token (tensor_ops.rs:394-458; the reference checks the same on
    # two rows, tensor_ops.rs:641-669).  At 1000 columns the host's sequential
    # f32 sums stay within ~1e-6 of exact, far inside the margin.
    ctx = _ctx(1000)
    rng = np.random.default_rng(641)
    rows = 64
    x = (rng.standard_normal((rows, 1000)) * 2).astype(np.float32)
    temps = rng.choice([0.85, 0.7, 1.35], rows).astype(np.float32)
    tops = rng.choice([1.0, 0.72, 0.9, 0.5], rows).astype(np.float32)
    seeds = rng.integers(0, 2 ** 63, rows, dtype=np.uint64)
    got = sample_device(ctx, x, temps, tops, seeds)
    compared = 0
    for r in range(rows):
        _, margin = O.sample_token_device(x[r], float(temps[r]), float(tops[r]), int(seeds[r]))
        if margin > MARGIN:
            assert got[r] == O.sample_token(x[r], float(temps[r]), float(tops[r]), int(seeds[r])), r
            compared += 1
    assert compared >= rows - 3
    ctx.close()


def test_decode_batch_samples_its_own_logits():
    cfg = dict(SMALL)
    geo = geometry(cfg)
    ctx, _ = make(cfg, geo, random_weights(cfg, geo, seed=21), "f32", True)
    rng = np.random.default_rng(8)
    n = 12
    backends = [ctx.new_backend() for _ in range(n)]
    for b in backends:
        b.prefill(rng.integers(0, cfg["vocab"], 9).tolist())
    temps, tops, seeds = _params(rng, n)
    reqs = [DecodeMicrobatchRequest(str(i), int(rng.integers(0, cfg["vocab"])), b, temperature=float(temps[i]),
                                    top_p=float(tops[i]), sampling_seed=int(seeds[i])) for i, b in enumerate(backends)]
    outs = BackendMicrobatchExecutor.decode_step_batch(reqs, want_logits=True)
    logits = np.stack([o.logits for o in outs])
    got = [o.sampled_token for o in outs]
    assert _check(logits, temps, tops, seeds, got) >= n - 1
    for i in range(n):  # argmax rows are the step's greedy tokens
        if temps[i] <= 0 or tops[i] <= 0:
            assert got[i] == int(np.argmax(logits[i]))
    assert all(b.sequence_position() == 10 for b in backends)
    ctx.close()


def test_error_paths_launch_nothing():
    # empty (zero rows or columns) or over-wide logits are rejected before any
    # launch, with the reference's message for the empty case
    # (runtime.rs:548-552)
    ctx = _ctx(1000)
    lib = ctx.lib
    one = np.ones(1, np.float32)
    seed = np.zeros(1, np.uint64)
    f32p = O.C.POINTER(O.C.c_float)
    u64p = O.C.POINTER(O.C.c_uint64)
    d_x = DeviceBuffer(ctx, 16)
    d_out = DeviceBuffer(ctx, 16)
    args = (one.ctypes.data_as(f32p), one.ctypes.data_as(f32p), seed.ctypes.data_as(u64p), d_out.ptr)
    with pytest.raises(ZrError) as e:
        ctx.check(lib.zr_sample(ctx.h, d_x.ptr, 1, 0, *args))
    assert e.value.status == ZR_E_INVALID and "empty logits" in str(e.value)
    with pytest.raises(ZrError) as e:
        ctx.check(lib.zr_sample(ctx.h, d_x.ptr, 1, (1 << 20) + 1, *args))
    assert e.value.status == ZR_E_INVALID and "at most" in str(e.value)
    with pytest.raises(ZrError) as e:
        ctx.check(lib.zr_sample(ctx.h, d_x.ptr, 0, 4, *args))
    assert e.value.status == ZR_E_INVALID and "empty logits" in str(e.value)
    d_x.free()
    d_out.free()
    ctx.close()
