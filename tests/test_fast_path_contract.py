"""The fast-path planner, workspace staging and executor contract of the rocm
arm, through the C-ABI on the CPU (host bookkeeping, no device).

Planner and staging follow agent/src/inference/fast_path.rs; the oracle's
Python restatement (oracle.fast_path_plan_decode / fast_path_stage_decode) is
pinned by the reference's own known answers (fast_path.rs:974-1056) and the
library is checked against it.  The contract mirrors the reference's CUDA arm
(engine.rs:240-273, provider/mod.rs:88-150)."""
import glob
import os
import re

import numpy as np
import pytest

import oracle as O
from mesh_amd import FastPathPlanner, _lib, executor_contract
from mesh_amd.provider import FUSED_KERNEL_STAGES
from tests.test_cabi_host import HostBackend, host_pool

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FIELDS = ("slot_sequence_lengths", "slot_positions", "slot_block_tables", "slot_mapping")


# ------------------------------------------------------------ the oracle --
def test_oracle_staging_reproduces_the_reference_known_answers():
    # decode_workspace_lease_stages_batch_metadata_and_reuses_bucket_pool (974-1004)
    plan = O.fast_path_plan_decode(3, 5000)
    assert (plan["batch_size_ceiling"], plan["token_ceiling"]) == (4, 8192)
    out = O.fast_path_stage_decode(plan, [11, 12, 13], [(31, 7, [0]), (32, 8, [1]), (33, 9, [2])])
    assert out["token_ids"][:3].tolist() == [11, 12, 13]
    assert out["positions"][:3].tolist() == [31, 32, 33]
    assert out["slot_sequence_lengths"][:3].tolist() == [7, 8, 9]
    out = O.fast_path_stage_decode(plan, [21, 22], [(41, 3, [0]), (42, 4, [0])])  # restage resets
    assert out["token_ids"].tolist() == [21, 22, 0, 0] and out["slot_sequence_lengths"].tolist() == [3, 4, 0, 0]
    # decode_workspace_lease_preserves_real_block_table_page_ids (1022-1056)
    out = O.fast_path_stage_decode(O.fast_path_plan_decode(1, 5000), [11], [(48, 46, [9, 4, 1])])
    assert out["slot_block_tables"][:3].tolist() == [9, 4, 1]
    assert (out["slot_block_tables"][3:] == O.U32_MAX).all() and out["slot_mapping"].tolist() == [0]
    with pytest.raises(O.OracleError, match="no stable Decode bucket supports batch_size=9 token_count=10"):
        O.fast_path_plan_decode(9, 10)


def test_oracle_fnv1a64_matches_the_published_test_vectors():
    # FNV-1a 64 vectors from the algorithm's published test suite (Noll's test_fnv.c)
    assert O.fnv1a64(b"") == 0xcbf29ce484222325
    assert O.fnv1a64(b"a") == 0xaf63dc4c8601ec8c
    assert O.fnv1a64(b"foobar") == 0x85944171f73967e8
    # the layout hash is FNV-1a over the key's items in order: one reordered item changes it
    f = [("slot_sequence_lengths", 1, 4), ("slot_positions", 1, 4), ("slot_block_tables", 128, 512),
         ("slot_mapping", 1, 4)]
    assert O.fast_path_layout_hash(0, 1, 2048, f) != O.fast_path_layout_hash(0, 1, 2048, [f[1], f[0]] + f[2:])
    assert O.fast_path_layout_hash(0, 1, 2048, f) != O.fast_path_layout_hash(1, 1, 2048, f)


def test_oracle_prefill_plan_positions_and_validation_reproduce_the_reference_known_answers():
    # decode_plan_selects_smallest_supported_bucket (935-942): the fused profile replays
    assert O.fast_path_plan_decode(3, 5000)["capture_strategy"] == "replay_preferred"
    # prefill_plan_uses_explicit_single_sequence_strategy (944-955)
    plan = O.fast_path_plan_prefill(400)
    assert plan["phase"] == 1 and plan["batch_size_ceiling"] == 1 and plan["token_ceiling"] == 512
    assert plan["prefill_strategy"] == "single_sequence_buckets"
    # prefill_workspace_lease_stages_positions_and_reuses_bucket_pool (1058-1080)
    assert O.fast_path_stage_prefill_positions(plan, 64, 4)[:4].tolist() == [64, 65, 66, 67]
    again = O.fast_path_stage_prefill_positions(plan, 128, 3)
    assert again[:3].tolist() == [128, 129, 130] and not again[3:].any()  # the restage reset the buffer
    # validate_decode_contexts_rejects_provider_drift (959-972)
    plan = O.fast_path_plan_decode(1, 1024)
    cpu = dict(provider="cpu", optimization_profile="cpu_serial", model_id="llama-70b", logical_kv_tokens=1024)
    with pytest.raises(O.OracleError, match="does not match planned provider/profile"):
        O.fast_path_validate_decode_contexts(plan, [cpu])
    # the same context from the plan's own provider passes
    O.fast_path_validate_decode_contexts(plan, [dict(cpu, provider="rocm", optimization_profile="rocm_fused")])
    # a changed field no longer hashes to the plan's layout hash
    bad = dict(plan, fields=[plan["fields"][0], plan["fields"][1], ("slot_block_tables", 1, 4), plan["fields"][3]])
    with pytest.raises(O.OracleError, match="fast-path metadata drift for decode-b1-kv2048-rocm"):
        O.fast_path_validate_decode_contexts(bad, [dict(cpu, provider="rocm", optimization_profile="rocm_fused")])


# ----------------------------------------------------------- the planner --
@pytest.mark.parametrize("batch,tokens", [(1, 0), (1, 2048), (1, 2049), (3, 5000), (4, 8192), (5, 100),
                                          (8, 65536), (2, 16385)])
def test_plan_decode_matches_the_oracle(batch, tokens):
    plan = FastPathPlanner.plan_decode(batch, tokens, 2048)
    want = O.fast_path_plan_decode(batch, tokens)
    assert (plan.batch_size_ceiling, plan.token_ceiling, plan.page_slots) == (
        want["batch_size_ceiling"], want["token_ceiling"], want["page_slots"])
    assert plan.bucket_label.decode() == want["bucket_label"]
    off = 0
    for f, (_, count, stride) in enumerate(want["fields"]):
        assert plan.field_offset[f] == off and plan.field_bytes[f] == stride
        off += stride
    assert plan.metadata_bytes == off
    # workspace_requirements (869-890), fused profile: 96 B per token, 32 KiB per slot, 256 B aligned
    assert plan.workspace_bytes == off + 96 * plan.token_ceiling + 32 * 1024 * plan.batch_size_ceiling
    assert plan.workspace_alignment == 256


@pytest.mark.parametrize("batch,tokens", [(9, 1), (1, 65537), (256, 395241)])
def test_plan_decode_rejects_batches_no_bucket_holds(batch, tokens):
    # the 256-session step exceeds every bucket and runs without a plan (backend.rs:116-126)
    with pytest.raises(_lib.ZrError) as e:
        FastPathPlanner.plan_decode(batch, tokens, 8192)
    with pytest.raises(O.OracleError) as w:
        O.fast_path_plan_decode(batch, tokens)
    assert str(e.value).endswith(str(w.value))


@pytest.mark.parametrize("tokens", [0, 1, 128, 129, 400, 512, 2049, 8192, 16384])
def test_plan_prefill_matches_the_oracle(tokens):
    plan = FastPathPlanner.plan_prefill(tokens)
    want = O.fast_path_plan_prefill(tokens)
    assert (plan.phase, plan.batch_size_ceiling, plan.token_ceiling, plan.page_slots) == (
        want["phase"], want["batch_size_ceiling"], want["token_ceiling"], want["page_slots"])
    assert (plan.actual_batch_size, plan.actual_token_count, plan.max_sequence_len) == (1, tokens, tokens)
    assert plan.bucket_label.decode() == want["bucket_label"]
    assert plan.capture_strategy.decode() == "replay_preferred"
    assert plan.prefill_strategy.decode() == "single_sequence_buckets"
    assert [plan.field_bytes[f] for f in range(4)] == [stride for _, _, stride in want["fields"]]
    assert plan.workspace_bytes == want["workspace_bytes"] and plan.layout_hash == want["layout_hash"]


def test_plan_decode_carries_capture_strategy_and_layout_hash():
    for batch, tokens in ((1, 0), (3, 5000), (8, 65536)):
        plan = FastPathPlanner.plan_decode(batch, tokens, 2048)
        want = O.fast_path_plan_decode(batch, tokens)
        assert plan.phase == 0 and plan.capture_strategy.decode() == "replay_preferred"
        assert plan.prefill_strategy.decode() == "" and plan.layout_hash == want["layout_hash"]
    hashes = {FastPathPlanner.plan_decode(b, t, 1).layout_hash for b in O.DECODE_BUCKET_BATCHES
              for t in O.DECODE_BUCKET_KV_TOKENS}
    hashes |= {FastPathPlanner.plan_prefill(t).layout_hash for t in O.PREFILL_BUCKET_TOKENS}
    assert len(hashes) == 25  # every bucket has its own layout


def test_plan_prefill_rejects_prompts_no_bucket_holds():
    with pytest.raises(_lib.ZrError) as e:
        FastPathPlanner.plan_prefill(16385)
    with pytest.raises(O.OracleError) as w:
        O.fast_path_plan_prefill(16385)
    assert str(e.value).endswith(str(w.value))
    assert "no stable Prefill bucket supports batch_size=1 token_count=16385 for RocmFused" in str(e.value)


@pytest.mark.parametrize("start,count", [(64, 4), (128, 3), (0, 0), (0, 512), (4095, 400),
                                         (0xFFFFFFFF - 3, 4)])
def test_stage_prefill_positions_matches_the_oracle(start, count):
    plan = FastPathPlanner.plan_prefill(400)
    got = FastPathPlanner.stage_prefill_positions(plan, start, count)
    want = O.fast_path_stage_prefill_positions(O.fast_path_plan_prefill(400), start, count)
    np.testing.assert_array_equal(got, want[:count])


def test_stage_prefill_positions_errors_carry_the_reference_text():
    plan = FastPathPlanner.plan_prefill(400)
    for start, count in ((0, 513), (0xFFFFFFFF - 2, 4)):
        with pytest.raises(_lib.ZrError) as e:
            FastPathPlanner.stage_prefill_positions(plan, start, count)
        with pytest.raises(O.OracleError) as w:
            O.fast_path_stage_prefill_positions(O.fast_path_plan_prefill(400), start, count)
        assert str(e.value).endswith(str(w.value))
    with pytest.raises(_lib.ZrError, match="requires prefill plan"):
        FastPathPlanner.stage_prefill_positions(FastPathPlanner.plan_decode(1, 10, 10), 0, 1)


def _ctx(provider="rocm", profile="rocm_fused", model="llama-3-8b", tokens=1024):
    return dict(provider=provider, optimization_profile=profile, model_id=model, logical_kv_tokens=tokens)


@pytest.mark.parametrize("case", ["ok", "count", "primary", "mixed", "footprint", "model", "model_none", "empty"])
def test_validate_decode_contexts_matches_the_oracle(case):
    batch = 0 if case == "empty" else 3
    plan = FastPathPlanner.plan_decode(batch, 5000, 2048)
    want_plan = O.fast_path_plan_decode(batch, 5000)
    ctxs = [_ctx(), _ctx(tokens=7000), _ctx(tokens=10)]
    if case == "count":
        ctxs = ctxs[:2]
    elif case == "primary":
        ctxs[0] = _ctx("cpu", "cpu_serial")
    elif case == "mixed":
        ctxs[2] = _ctx("cuda", "cuda_fused")
    elif case == "footprint":
        ctxs[1] = _ctx(tokens=8193)
    elif case == "model":
        ctxs[2] = _ctx(model="llama-70b")
    elif case == "model_none":
        ctxs[1] = _ctx(model=None)  # a backend without a model id shares any residency
    elif case == "empty":
        ctxs = []
    if case in ("ok", "model_none", "empty"):
        FastPathPlanner.validate_decode_contexts(plan, ctxs)
        O.fast_path_validate_decode_contexts(want_plan, ctxs)
        return
    with pytest.raises(_lib.ZrError) as e:
        FastPathPlanner.validate_decode_contexts(plan, ctxs)
    with pytest.raises(O.OracleError) as w:
        O.fast_path_validate_decode_contexts(want_plan, ctxs)
    assert str(e.value).endswith(str(w.value))
    assert "fast-path capture invariant failed for decode-b4-kv8192-rocm: " in str(e.value)


def test_validate_decode_contexts_detects_metadata_drift():
    plan = FastPathPlanner.plan_decode(1, 100, 100)
    ctxs = [_ctx(tokens=100)]
    FastPathPlanner.validate_decode_contexts(plan, ctxs)
    plan.field_bytes[2] += 4  # a slot table one entry longer than the bucket's layout
    with pytest.raises(_lib.ZrError, match=f"fast-path metadata drift for decode-b1-kv2048-rocm: expected layout "
                                           f"hash {plan.layout_hash}, observed "):
        FastPathPlanner.validate_decode_contexts(plan, ctxs)


# ------------------------------------------------------------ the staging --
def _session(pool, rows, keep=None, max_seq=4096):
    b = HostBackend(pool, max_seq)
    b.reserve(rows)
    if keep is not None:
        b.retain(keep)
    return b


def _slot(b):
    lib = _lib.load()
    table, _ = b.table()
    return lib.zrh_sequence_position(b.h), b.seq_len, [p for p, _, _ in table]


def test_stage_decode_matches_the_oracle_on_live_sessions():
    pool = host_pool(4096)
    # positions / lengths of the known answer (31, 7), (32, 8), (33, 9): window trimmed to the last rows
    bs = [_session(pool, 31, 7), _session(pool, 32, 8), _session(pool, 33, 9)]
    plan = FastPathPlanner.plan_decode(3, 5000, 2048)
    got = FastPathPlanner.stage_decode(plan, bs, [11, 12, 13])
    want = O.fast_path_stage_decode(O.fast_path_plan_decode(3, 5000), [11, 12, 13], [_slot(b) for b in bs])
    assert got["positions"][:3].tolist() == [31, 32, 33]
    assert got["slot_sequence_lengths"][:3].tolist() == [7, 8, 9]
    for k in ("token_ids", "positions") + FIELDS:
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)
    # a reused-page table (forward_pass.rs:3794-3822: [1, 2, 0, 3]) and random sessions
    kat = HostBackend(pool, 48)
    kat.reserve(48)
    kat.retain(30)
    kat.reserve(18)
    rng = np.random.default_rng(5)
    rand = [_session(pool, int(rng.integers(1, 600)), None) for _ in range(6)]
    for b in rand[:3]:
        b.retain(int(rng.integers(1, b.seq_len + 1)))
    group = [kat] + rand
    plan = FastPathPlanner.plan_decode(7, 5000, 2048)
    toks = rng.integers(0, 1000, 7).tolist()
    got = FastPathPlanner.stage_decode(plan, group, toks)
    want = O.fast_path_stage_decode(O.fast_path_plan_decode(7, 5000), toks, [_slot(b) for b in group])
    S = plan.page_slots
    assert got["slot_block_tables"][:4].tolist() == [1, 2, 0, 3] and got["slot_block_tables"][4] == O.U32_MAX
    for k in ("token_ids", "positions") + FIELDS:
        np.testing.assert_array_equal(got[k], want[k], err_msg=k)
    assert (got["slot_block_tables"][7 * S:] == O.U32_MAX).all() and got["slot_mapping"][7] == O.U32_MAX
    for b in bs + group:
        b.close()
    _lib.load().zrh_pool_destroy(pool)


def test_stage_decode_capture_errors_carry_the_reference_text():
    pool = host_pool(4096)
    bs = [_session(pool, 10) for _ in range(3)]
    plan = FastPathPlanner.plan_decode(2, 100, 2048)
    with pytest.raises(_lib.ZrError, match="fast-path capture invariant failed for decode-b2-kv2048-rocm: "
                                           "runtime batch size 3 exceeds bucket ceiling 2"):
        FastPathPlanner.stage_decode(plan, bs, [1, 2, 3])
    long = _session(pool, 3000)
    plan = FastPathPlanner.plan_decode(1, 100, 2048)
    with pytest.raises(_lib.ZrError, match="slot 0 sequence length 3000 exceeds bucket token ceiling 2048"):
        FastPathPlanner.stage_decode(plan, [long], [1])
    for b in bs + [long]:
        b.close()
    _lib.load().zrh_pool_destroy(pool)


def test_fast_path_context_and_token_ceiling():
    lib = _lib.load()
    pool = host_pool(8192)
    for rows, keep, ceiling in ((5, None, 2048), (2048, None, 2048), (2049, None, 8192), (70000, 100, None)):
        b = _session(pool, rows, keep, max_seq=1 << 20)
        c = _lib.FastPathContext()
        _lib.check(lib.zrh_get_fast_path_context(b.h, c))
        # logical KV tokens: position - base position, i.e. the live window's rows
        assert c.position == rows and c.cached_tokens == b.seq_len
        assert c.logical_kv_tokens == rows - b.base
        want = next((t for t in O.DECODE_BUCKET_KV_TOKENS if c.logical_kv_tokens <= t), None)
        assert (None if c.decode_token_ceiling < 0 else c.decode_token_ceiling) == want
        if keep is None:
            assert want == ceiling
        b.close()
    lib.zrh_pool_destroy(pool)


# ------------------------------------------------------------ the contract --
def test_executor_contract_is_the_rocm_arm_and_names_real_kernels():
    c = executor_contract()
    assert c["provider"] == "rocm" and c["optimization_profile"] == "rocm_fused"
    assert c["executor_class"] == "fast_path" and c["memory_model"] == "discrete_vram"
    # the CUDA arm's stage list and flags (engine.rs:240-273), prefill microbatches aside
    assert c["fused_stages"] == ["norm_qkv", "rope_kv_write", "paged_attention", "residual_mlp", "device_sampling"]
    assert c["host_kernels"] == ["host_assisted_sampling"]
    assert c["collective_residency"] == "staged_runtime" and c["collective_tensors_per_layer"] == 2
    assert c["decode_supports_microbatch"] and c["decode_uses_device_sampling"] and c["kv_requires_paged_cache"]
    assert c["supports_device_sampling"] and c["supports_checkpoint_handoff"] and c["fast_path_eligible"]
    # FastPathPlanner::capture_strategy (fast_path.rs:831-837), as the CudaFused arm
    assert c["capture_strategy"] == "replay_preferred"
    src = "".join(open(f).read() for f in glob.glob(os.path.join(ROOT, "mesh_amd", "csrc", "*.hip")))
    defined = set(re.findall(r"__global__\s+(?:__launch_bounds__\([^)]*\)\s*)?void\s+(\w+)\s*\(", src))
    for stage, kernels in c["stage_kernels"].items():
        assert kernels and set(kernels) <= defined, (stage, set(kernels) - defined)
    assert c["stage_kernels"] == FUSED_KERNEL_STAGES
