/*
 * kv_cbor.c -- CPU restatement of the KV snapshot wire format.
 *
 * TEST INFRASTRUCTURE ONLY (the test oracle for the device encoder and the host
 * decoder of the rocm provider).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it.
 *
 * KVCache::to_bytes (kv_cache.rs:880-887) is ciborium 0.2.2 `into_writer`
 * (Cargo.lock:627-629) of the serde-derived struct tree
 *   KVCache       { layers: Vec<LayerKVCache>, base_position: usize,
 *                   config: KVCacheConfig }               kv_cache.rs:664-672
 *   LayerKVCache  { keys: Option<Tensor2D>, values: Option<Tensor2D>,
 *                   seq_len: usize, layer_idx: usize }     kv_cache.rs:505-515
 *   Tensor2D      { data: Vec<f32>, rows: usize, cols: usize }
 *                                                          tensor_ops.rs:23-31
 *   KVCacheConfig { num_layers, num_heads, head_dim, max_seq_len: usize }
 *                                                          kv_cache.rs:190-200
 * as DeviceKVCache::export_snapshot builds it (forward_pass.rs:1169-1204):
 * every layer holds the same rows, layer_idx = its index, base_position is the
 * first cached position after the window trim, config is the device cache's
 * (num_heads = the model's kv heads, forward_pass.rs:1791-1796).
 *
 * serde's data model as ciborium writes it: a struct is a definite-length map
 * of (field name as text, value) pairs in declaration order; None is null,
 * Some(x) is x; usize is an unsigned integer; Vec is a definite-length array.
 * An f32 is widened to f64 (serialize_f32 -> serialize_f64) and written as the
 * narrowest IEEE float (half, single, double) whose conversion back to f64
 * gives the same bits.  RFC 8949 section 3: the head byte is major type << 5 |
 * additional info; an argument up to 23 is inline, else 1, 2, 4 or 8 bytes
 * follow in network byte order and the shortest form is used.
 *
 * NaN payloads: the half / f64 round trip of a NaN depends on the conversion
 * routine of the `half` crate (2.7.1) and the host's f32 -> f64 conversion;
 * the rule below (quiet the NaN, keep the top 10 mantissa bits) is this
 * restatement's choice and is not pinned by any reference test.
 */
#include "zip_oracle.h"

#include <math.h>
#include <string.h>

/* ---------------------------------------------------------- primitives --- */

static int put_head(uint8_t* out, int major, uint64_t v) {
    const uint8_t m = (uint8_t)(major << 5);
    if (v <= 23) {
        if (out) out[0] = (uint8_t)(m | v);
        return 1;
    }
    int n = v <= 0xffu ? 1 : v <= 0xffffu ? 2 : v <= 0xffffffffu ? 4 : 8;
    if (out) {
        out[0] = (uint8_t)(m | (n == 1 ? 24 : n == 2 ? 25 : n == 4 ? 26 : 27));
        for (int i = 0; i < n; ++i) out[1 + i] = (uint8_t)(v >> (8 * (n - 1 - i)));
    }
    return 1 + n;
}

int or_cbor_uint(int major, uint64_t v, uint8_t* out) { return put_head(out, major, v); }

/* IEEE 754 binary64 -> binary16, round to nearest, ties to even. */
static uint16_t f64_to_f16(double x) {
    uint64_t b;
    memcpy(&b, &x, 8);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const int exp = (int)((b >> 52) & 0x7ff);
    const uint64_t man = b & 0xfffffffffffffull;
    if (exp == 0x7ff) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (uint16_t)(man >> 42)); /* quiet, top 10 bits */
    }
    if (exp == 0 && man == 0) return sign;
    /* value = sig * 2^(e2), sig with the hidden bit, 53 bits */
    const uint64_t sig = exp ? (man | (1ull << 52)) : man;
    const int e2 = (exp ? exp : 1) - 1075;
    /* target: f16 quantum 2^-24 below 2^-14, else 2^(e - 10) for value in [2^e, 2^(e+1)) */
    int e = exp ? exp - 1023 : -1023;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    const int q = e < -14 ? -24 : e - 10; /* log2 of the f16 quantum at this magnitude */
    const int shift = q - e2;             /* bits of sig below the quantum */
    uint64_t k;                           /* value / 2^q, rounded */
    if (shift <= 0) {
        k = sig << (-shift);
    } else if (shift >= 64) {
        k = 0;
    } else {
        k = sig >> shift;
        const uint64_t rem = sig & ((1ull << shift) - 1), half = 1ull << (shift - 1);
        if (rem > half || (rem == half && (k & 1))) ++k;
    }
    if (q == -24) { /* subnormal range; k may round up into the normal range */
        return (uint16_t)(sign | (uint16_t)k);
    }
    /* normal: k in [2^10, 2^11]; rounding up to 2^11 bumps the exponent */
    int ee = e;
    if (k >> 11) {
        k >>= 1;
        ++ee;
    }
    if (ee > 15) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (uint16_t)((ee + 15) << 10) | (uint16_t)(k & 0x3ff));
}

static double f16_to_f64(uint16_t h) {
    const int sign = h >> 15, exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    double v;
    if (exp == 0x1f) {
        uint64_t b = ((uint64_t)sign << 63) | 0x7ff0000000000000ull | ((uint64_t)man << 42);
        if (man) b |= 0x0008000000000000ull;
        memcpy(&v, &b, 8);
        return v;
    }
    v = exp ? ldexp(1.0 + man / 1024.0, exp - 15) : ldexp(man / 1024.0, -14);
    return sign ? -v : v;
}

/* f32 -> f64 widening with the NaN quieted (x86 cvtss2sd). */
static double widen(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) {
        const uint64_t b = ((uint64_t)(u >> 31) << 63) | 0x7ff0000000000000ull |
                           ((uint64_t)((u & 0x7fffffu) | 0x400000u) << 29);
        double d;
        memcpy(&d, &b, 8);
        return d;
    }
    return (double)x;
}

int or_cbor_float(float x, uint8_t* out) {
    const double d = widen(x);
    uint64_t bd, bh;
    memcpy(&bd, &d, 8);
    const uint16_t h = f64_to_f16(d);
    const double back = f16_to_f64(h);
    memcpy(&bh, &back, 8);
    if (bh == bd) {
        if (out) {
            out[0] = 0xf9;
            out[1] = (uint8_t)(h >> 8);
            out[2] = (uint8_t)h;
        }
        return 3;
    }
    const float s = (float)d;
    const double back32 = (double)s;
    uint64_t b32;
    memcpy(&b32, &back32, 8);
    if (b32 == bd && !isnan(d)) {
        uint32_t u;
        memcpy(&u, &s, 4);
        if (out) {
            out[0] = 0xfa;
            for (int i = 0; i < 4; ++i) out[1 + i] = (uint8_t)(u >> (24 - 8 * i));
        }
        return 5;
    }
    if (out) {
        out[0] = 0xfb;
        for (int i = 0; i < 8; ++i) out[1 + i] = (uint8_t)(bd >> (56 - 8 * i));
    }
    return 9;
}

/* -------------------------------------------------------------- struct --- */

typedef struct {
    uint8_t* p; /* NULL: count only */
    int64_t n, cap;
    int overflow;
} wbuf;

static void wput(wbuf* w, const uint8_t* src, int len) {
    if (w->p && !w->overflow) {
        if (w->n + len > w->cap)
            w->overflow = 1;
        else
            memcpy(w->p + w->n, src, (size_t)len);
    }
    w->n += len;
}

static void whead(wbuf* w, int major, uint64_t v) {
    uint8_t t[9];
    wput(w, t, put_head(t, major, v));
}

static void wtext(wbuf* w, const char* s) {
    const int n = (int)strlen(s);
    whead(w, 3, (uint64_t)n);
    wput(w, (const uint8_t*)s, n);
}

static void wtensor(wbuf* w, const float* data, int rows, int cols) {
    whead(w, 5, 3);
    wtext(w, "data");
    const int64_t n = (int64_t)rows * cols;
    whead(w, 4, (uint64_t)n);
    uint8_t t[9];
    for (int64_t i = 0; i < n; ++i) wput(w, t, or_cbor_float(data[i], t));
    wtext(w, "rows");
    whead(w, 0, (uint64_t)rows);
    wtext(w, "cols");
    whead(w, 0, (uint64_t)cols);
}

int64_t or_kv_cbor_encode(const float* k, const float* v, int num_layers, int rows, int cols,
                          int64_t base_position, int cfg_num_layers, int cfg_num_heads, int cfg_head_dim,
                          int cfg_max_seq_len, uint8_t* out, int64_t capacity) {
    if (num_layers < 0 || rows < 0 || cols < 0 || base_position < 0) return -1;
    wbuf w = {out, 0, capacity, 0};
    whead(&w, 5, 3);
    wtext(&w, "layers");
    whead(&w, 4, (uint64_t)num_layers);
    const int64_t per = (int64_t)rows * cols;
    for (int l = 0; l < num_layers; ++l) {
        whead(&w, 5, 4);
        wtext(&w, "keys");
        if (rows > 0)
            wtensor(&w, k + l * per, rows, cols);
        else
            wput(&w, (const uint8_t*)"\xf6", 1);
        wtext(&w, "values");
        if (rows > 0)
            wtensor(&w, v + l * per, rows, cols);
        else
            wput(&w, (const uint8_t*)"\xf6", 1);
        wtext(&w, "seq_len");
        whead(&w, 0, (uint64_t)rows);
        wtext(&w, "layer_idx");
        whead(&w, 0, (uint64_t)l);
    }
    wtext(&w, "base_position");
    whead(&w, 0, (uint64_t)base_position);
    wtext(&w, "config");
    whead(&w, 5, 4);
    wtext(&w, "num_layers");
    whead(&w, 0, (uint64_t)cfg_num_layers);
    wtext(&w, "num_heads");
    whead(&w, 0, (uint64_t)cfg_num_heads);
    wtext(&w, "head_dim");
    whead(&w, 0, (uint64_t)cfg_head_dim);
    wtext(&w, "max_seq_len");
    whead(&w, 0, (uint64_t)cfg_max_seq_len);
    if (out && w.overflow) return -2;
    return w.n;
}
