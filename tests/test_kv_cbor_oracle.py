"""The oracle's KV snapshot encoder (oracle/kv_cbor.c), pinned without the reference.

KVCache::to_bytes (kv_cache.rs:880-887) is ciborium 0.2.2 over serde-derived
structs.  No test of the reference holds encoded bytes (kv_cache.rs:1090-1100
only round-trips), so the encoder is pinned by
* the encoded examples of RFC 8949 Appendix A (integers, half / single floats,
  text, arrays, maps, null),
* every binary16 value: numpy's IEEE binary16 says which f32 values are exact
  halves (3-byte items) and which are not (5-byte single items),
* an independent decoder written here from RFC 8949 section 3 that reads the
  oracle's document back into the serde struct tree (field names in
  declaration order: KVCache kv_cache.rs:664-672, LayerKVCache 505-515,
  Tensor2D tensor_ops.rs:23-31, KVCacheConfig kv_cache.rs:190-200) and the
  exact floats.
NaN payload encoding is not pinned (see oracle/kv_cbor.c).
"""
import struct

import numpy as np
import pytest

import oracle as O

# RFC 8949 Appendix A (value, encoding)
RFC_UINTS = [(0, "00"), (1, "01"), (10, "0a"), (23, "17"), (24, "1818"), (25, "1819"), (100, "1864"),
             (1000, "1903e8"), (1000000, "1a000f4240"), (1000000000000, "1b000000e8d4a51000"),
             (18446744073709551615, "1bffffffffffffffff")]
RFC_FLOATS = [(0.0, "f90000"), (-0.0, "f98000"), (1.0, "f93c00"), (1.5, "f93e00"), (65504.0, "f97bff"),
              (100000.0, "fa47c35000"), (3.4028234663852886e+38, "fa7f7fffff"), (5.960464477539063e-8, "f90001"),
              (0.00006103515625, "f90400"), (-4.0, "f9c400"), (float("inf"), "f97c00"),
              (float("-inf"), "f9fc00"), (float("nan"), "f97e00")]


@pytest.mark.parametrize("v,enc", RFC_UINTS)
def test_rfc8949_unsigned_integers(v, enc):
    assert O.cbor_uint(0, v).hex() == enc


def test_rfc8949_heads_of_other_major_types():
    assert O.cbor_uint(3, 4).hex() + b"IETF".hex() == "6449455446"  # "IETF"
    assert O.cbor_uint(4, 0).hex() == "80"                           # []
    assert O.cbor_uint(4, 25).hex() == "9819"                        # [1 .. 25]
    assert O.cbor_uint(5, 0).hex() == "a0"                           # {}
    assert O.cbor_uint(5, 2).hex() == "a2"


@pytest.mark.parametrize("x,enc", RFC_FLOATS)
def test_rfc8949_floats_narrowest_exact(x, enc):
    assert O.cbor_float(x).hex() == enc


def test_every_binary16_value_is_a_half_item():
    h = np.arange(1 << 16, dtype=np.uint16)
    vals = h.view(np.float16)
    finite = ~np.isnan(vals)
    for bits, v in zip(h[finite][::7], vals[finite][::7]):  # every 7th pattern keeps the test quick
        enc = O.cbor_float(np.float32(v))
        assert enc == b"\xf9" + struct.pack(">H", int(bits)), (hex(int(bits)), float(v), enc.hex())


def test_f32_values_that_are_not_halves_are_single_items():
    rng = np.random.default_rng(7)
    xs = np.concatenate([rng.standard_normal(4000).astype(np.float32),
                         (rng.standard_normal(1000) * 1e-6).astype(np.float32),   # below the half range
                         (rng.standard_normal(1000) * 1e6).astype(np.float32),    # above 65504
                         np.array([65520.0, 2.0 ** -25, 1.0 + 2.0 ** -11, 2.0 ** -126, 1e-40], np.float32)])
    for x in xs:
        with np.errstate(over="ignore"):
            half_exact = np.float32(np.float16(x)) == x and np.isfinite(np.float16(x))
        enc = O.cbor_float(x)
        if half_exact:
            assert enc == b"\xf9" + struct.pack(">e", np.float16(x)), (float(x), enc.hex())
        else:
            assert enc == b"\xfa" + struct.pack(">f", x), (float(x), enc.hex())


class Decoder:
    """RFC 8949 section 3 reader: maps keep their key order as lists of pairs."""

    def __init__(self, data):
        self.d, self.i = data, 0

    def item(self):
        b = self.d[self.i]
        self.i += 1
        major, info = b >> 5, b & 31
        if major == 7:
            if info == 22:
                return None
            size = {25: 2, 26: 4, 27: 8}[info]
            raw = self.d[self.i:self.i + size]
            self.i += size
            return ("float", size, struct.unpack({2: ">e", 4: ">f", 8: ">d"}[size], raw)[0])
        if info < 24:
            arg = info
        else:
            size = {24: 1, 25: 2, 26: 4, 27: 8}[info]
            arg = int.from_bytes(self.d[self.i:self.i + size], "big")
            shortest = {1: 24, 2: 256, 4: 65536, 8: 1 << 32}[size]
            assert arg >= shortest, "non-shortest argument"
            self.i += size
        if major == 0:
            return arg
        if major == 3:
            s = self.d[self.i:self.i + arg].decode()
            self.i += arg
            return s
        if major == 4:
            return [self.item() for _ in range(arg)]
        if major == 5:
            return [(self.item(), self.item()) for _ in range(arg)]
        raise AssertionError(f"unexpected major type {major}")


def test_document_structure_and_exact_floats():
    rng = np.random.default_rng(3)
    L, rows, cols = 3, 5, 16
    k = rng.standard_normal((L, rows, cols)).astype(np.float32)
    v = rng.standard_normal((L, rows, cols)).astype(np.float32)
    k[0, 0, :4] = [0.0, -0.0, 1.5, 65504.0]      # halves
    v[1, 2, :3] = [1e-7, 70000.0, 2.0 ** -24]   # single, single, half subnormal
    doc = O.kv_cbor_encode(k, v, base_position=40, cfg_num_layers=L, cfg_num_heads=2, cfg_head_dim=8,
                           cfg_max_seq_len=4096)
    dec = Decoder(doc)
    top = dec.item()
    assert dec.i == len(doc)
    assert [key for key, _ in top] == ["layers", "base_position", "config"]
    layers = dict(top)["layers"]
    assert dict(top)["base_position"] == 40
    assert dict(top)["config"] == [("num_layers", L), ("num_heads", 2), ("head_dim", 8), ("max_seq_len", 4096)]
    assert len(layers) == L
    for li, layer in enumerate(layers):
        assert [key for key, _ in layer] == ["keys", "values", "seq_len", "layer_idx"]
        d = dict(layer)
        assert d["seq_len"] == rows and d["layer_idx"] == li
        for name, src in (("keys", k), ("values", v)):
            t = d[name]
            assert [key for key, _ in t] == ["data", "rows", "cols"]
            td = dict(t)
            assert td["rows"] == rows and td["cols"] == cols
            got = np.array([x[2] for x in td["data"]], np.float32)
            np.testing.assert_array_equal(got.view(np.uint32), src[li].ravel().view(np.uint32))
            for x, want in zip(td["data"], src[li].ravel()):
                with np.errstate(over="ignore"):
                    assert x[1] == (2 if np.float32(np.float16(want)) == want else 4)


def test_count_only_and_capacity():
    k = np.ones((2, 3, 16), np.float32)
    doc = O.kv_cbor_encode(k, k, 0, 2, 1, 16, 4096)
    # 2 layers x 2 arrays x 48 items of 1.0 (f93c00)
    assert doc.count(b"\xf9\x3c\x00") == 2 * 2 * 48
    lib = O.lib()
    n = lib.or_kv_cbor_encode(O._f(k), O._f(k), 2, 3, 16, 0, 2, 1, 16, 4096, None, 0)
    assert n == len(doc)
    short = np.zeros(n - 1, np.uint8)
    assert lib.or_kv_cbor_encode(O._f(k), O._f(k), 2, 3, 16, 0, 2, 1, 16, 4096,
                                 short.ctypes.data_as(O.C.c_void_p), n - 1) == -2
