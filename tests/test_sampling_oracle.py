"""The oracle's restatement of the batched decode path's device sampler
(sample_tokens_device_with_seeds, runtime.rs:534-601), pinned without the
reference: its two device-vs-host known answers (tensor_ops.rs:641-669), the
argmax branch, an f64 brute force of the token rule, and the distribution a
sampler must draw from (frequencies over many seeds against the renormalised
nucleus probabilities)."""
import numpy as np

import oracle as O


def test_reference_device_matches_host_examples():
    # tensor_ops.rs:641-653 and 655-669: the device sampler returns the host sampler's token
    x = [0.1, 1.3, -0.4, 2.2, 0.7]
    assert O.sample_token_device(x, 0.85, 0.72, 424242)[0] == O.sample_token(x, 0.85, 0.72, 424242)
    y = [0.5, -0.2, 0.8, 1.1, 0.0, -1.4]
    assert O.sample_token_device(y, 1.35, 1.0, 1337)[0] == O.sample_token(y, 1.35, 1.0, 1337)


def test_argmax_branch():
    x = [0.0, 7.0, 7.0, 1.0]
    for t, p in ((0.0, 0.9), (-1.0, 0.5), (0.7, 0.0)):
        assert O.sample_token_device(x, t, p, 5)[0] == 1


def _f64_rule(x, temperature, top_p, seed):
    """The token rule in f64 (the reference's ops without rounding)."""
    s = np.asarray(x, np.float64) * (np.float32(1) / np.float32(temperature) if temperature != 1.0 else 1.0)
    e = np.exp(s - s.max())
    p = e / e.sum()
    tau = float(O.sample_threshold(seed))
    if top_p >= 1.0:
        c = np.cumsum(p)
        hit = np.nonzero(c >= tau)[0]
        return int(hit[0]) if hit.size else 0
    order = sorted(range(len(p)), key=lambda i: (-p[i], i))
    ps = p[order]
    before = np.concatenate([[0.0], np.cumsum(ps)[:-1]])
    kept = ps[before < top_p]
    c = np.cumsum(kept) / kept.sum()
    hit = np.nonzero(c >= tau)[0]
    return order[int(hit[0])] if hit.size else order[0]


def test_token_rule_against_f64_brute_force():
    rng = np.random.default_rng(11)
    checked = 0
    for trial in range(400):
        n = int(rng.integers(2, 300))
        x = rng.standard_normal(n).astype(np.float32) * float(rng.choice([0.5, 2.0, 6.0]))
        t = float(rng.choice([1.0, 0.7, 1.3, 0.25]))
        p = float(rng.choice([1.0, 0.9, 0.5, 0.1, 0.999]))
        seed = int(rng.integers(0, 2 ** 63))
        tok, margin = O.sample_token_device(x, t, p, seed)
        if margin > 1e-5:
            assert tok == _f64_rule(x, t, p, seed), (trial, n, t, p, seed)
            checked += 1
    assert checked > 380


def test_draws_follow_the_nucleus_distribution():
    x = np.array([2.0, 1.0, 0.5, 0.0, -1.0, 1.5], np.float32)
    t, top_p = 0.8, 0.8
    s = x.astype(np.float64) * float(np.float32(1) / np.float32(t))
    p = np.exp(s - s.max())
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    before = np.concatenate([[0.0], np.cumsum(p[order])[:-1]])
    keep = order[before < top_p]
    want = np.zeros_like(p)
    want[keep] = p[keep] / p[keep].sum()
    draws = 40000
    counts = np.zeros(len(x))
    for seed in range(draws):
        counts[O.sample_token_device(x, t, top_p, seed)[0]] += 1
    np.testing.assert_allclose(counts / draws, want, atol=0.01)
    assert counts[want == 0].sum() == 0


def test_device_rule_equals_host_sampler_away_from_boundaries():
    # The reference asserts device == host sampling on its two examples
    # (tensor_ops.rs:641-669).  The rules differ only in rounding (x / T against
    # x * f32(1 / T), f32 sums) and in "c > tau" against "c >= tau", so on rows
    # whose decision lies away from every boundary the host sampler
    # (tensor_ops.rs:394-458) returns the same token.
    rng = np.random.default_rng(29)
    checked = 0
    for trial in range(600):
        n = int(rng.integers(2, 400))
        x = (rng.standard_normal(n) * float(rng.choice([0.5, 1.5, 4.0]))).astype(np.float32)
        t = float(rng.choice([0.85, 0.7, 1.35, 2.0]))
        p = float(rng.choice([1.0, 0.72, 0.9, 0.5, 0.2]))
        seed = int(rng.integers(0, 2 ** 63))
        tok, margin = O.sample_token_device(x, t, p, seed)
        if margin > 1e-5:
            assert tok == O.sample_token(x, t, p, seed), (trial, n, t, p, seed)
            checked += 1
    assert checked > 560
