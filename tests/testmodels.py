"""Model fixtures shared by the CPU and GPU tests.

``constant_weights`` mirrors the reference's create_test_weights
(agent/src/inference/forward_pass.rs:3163-3202); ``random_weights`` draws
bf16-valued N(0, std) weights from a seeded numpy generator.
"""
import numpy as np

from oracle import round_bf16

TEST_CONFIG = dict(hidden=64, num_heads=4, num_kv_heads=4, num_layers=2, vocab=100,
                   ffn=128, rms_norm_eps=1e-5, rope_base=10000.0)


def geometry(cfg, shard_start=0, shard_end=None, ffn_cols=None):
    shard_end = cfg["hidden"] if shard_end is None else shard_end
    d = cfg["hidden"] // cfg["num_heads"]
    qpk = cfg["num_heads"] // cfg["num_kv_heads"]
    q_cols = shard_end - shard_start
    kv_cols = (q_cols // (qpk * d)) * d
    return dict(head_dim=d, q_cols=q_cols, kv_cols=kv_cols,
                ffn_cols=cfg["ffn"] if ffn_cols is None else ffn_cols,
                shard_start=shard_start, shard_end=shard_end)


def oracle_cfg(cfg, geo):
    return dict(hidden=cfg["hidden"], num_heads=cfg["num_heads"], num_kv_heads=cfg["num_kv_heads"],
                num_layers=cfg["num_layers"], vocab=cfg["vocab"], ffn_cols=geo["ffn_cols"],
                shard_start=geo["shard_start"], shard_end=geo["shard_end"],
                rms_norm_eps=cfg["rms_norm_eps"], rope_base=cfg["rope_base"])


def constant_weights(cfg, geo):
    H, V = cfg["hidden"], cfg["vocab"]
    Q, KV, F = geo["q_cols"], geo["kv_cols"], geo["ffn_cols"]
    full = lambda r, c, x: np.full((r, c), x, np.float32)
    layers = [dict(w_q=full(H, Q, 0.1), w_k=full(H, KV, 0.2), w_v=full(H, KV, 0.3),
                   w_o=full(Q, H, 0.4), w_up=full(H, F, 0.5), w_gate=full(H, F, 0.6),
                   w_down=full(F, H, 0.7), attn_norm=np.ones(H, np.float32),
                   mlp_norm=np.ones(H, np.float32)) for _ in range(cfg["num_layers"])]
    return dict(embedding=full(V, H, 0.05), final_norm=np.ones(H, np.float32),
                lm_head=full(H, V, 0.08), layers=layers)


class NormalPool:
    """N(0, 1) values for large test tensors: windows of one 16M-value bf16-exact
    pool at random offsets (every tensor differs; generation costs a copy)."""

    SIZE = 1 << 24

    def __init__(self, rng):
        self.rng = rng
        self.pool = round_bf16(rng.standard_normal(2 * self.SIZE, dtype=np.float32))

    def take(self, shape, scale=1.0):
        n = int(np.prod(shape))
        out = np.empty(n, np.float32)
        done = 0
        while done < n:
            off = int(self.rng.integers(0, self.SIZE))
            m = min(n - done, self.SIZE)
            out[done:done + m] = self.pool[off:off + m]
            done += m
        out = out.reshape(shape)
        if scale != 1.0:
            out *= np.float32(scale)  # a power of two keeps the values bf16-exact
        return out


def random_weights(cfg, geo, seed, std=0.02, pooled=False):
    """N(0, std) weights rounded to bf16; `pooled` draws them from a NormalPool
    scaled by the power of two nearest `std` (1/64 for 0.02), for the
    full-size configurations."""
    rng = np.random.default_rng(seed)
    H, V = cfg["hidden"], cfg["vocab"]
    Q, KV, F = geo["q_cols"], geo["kv_cols"], geo["ffn_cols"]
    pool = NormalPool(rng) if pooled else None
    # pooled: the power of two nearest std, so the pool's bf16 values stay exact
    pool_scale = float(2.0 ** np.round(np.log2(std)))

    def w(r, c):
        if pool is not None:
            return pool.take((r, c), pool_scale)
        return round_bf16(rng.standard_normal((r, c), dtype=np.float32) * np.float32(std))

    layers = []
    for _ in range(cfg["num_layers"]):
        layers.append(dict(w_q=w(H, Q), w_k=w(H, KV), w_v=w(H, KV), w_o=w(Q, H),
                           w_gate=w(H, F), w_up=w(H, F), w_down=w(F, H),
                           attn_norm=np.ones(H, np.float32), mlp_norm=np.ones(H, np.float32)))
    return dict(embedding=w(V, H), final_norm=np.ones(H, np.float32), lm_head=w(H, V),
                layers=layers)
