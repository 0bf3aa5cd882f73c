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


def random_weights(cfg, geo, seed, std=0.02):
    rng = np.random.default_rng(seed)
    H, V = cfg["hidden"], cfg["vocab"]
    Q, KV, F = geo["q_cols"], geo["kv_cols"], geo["ffn_cols"]

    def w(r, c):
        return round_bf16(rng.standard_normal((r, c), dtype=np.float32) * np.float32(std))

    layers = []
    for _ in range(cfg["num_layers"]):
        layers.append(dict(w_q=w(H, Q), w_k=w(H, KV), w_v=w(H, KV), w_o=w(Q, H),
                           w_gate=w(H, F), w_up=w(H, F), w_down=w(F, H),
                           attn_norm=np.ones(H, np.float32), mlp_norm=np.ones(H, np.float32)))
    return dict(embedding=w(V, H), final_norm=np.ones(H, np.float32), lm_head=w(H, V),
                layers=layers)
