"""Helpers shared by the GPU tests (device buffers, staging, comparisons)."""
import ctypes as C

import numpy as np

from mesh_amd import DeviceBuffer, DeviceContext, ModelGeometry, _lib


def f32p(a):
    return a.ctypes.data_as(_lib.c_f32_p)


def i32p(a):
    return a.ctypes.data_as(_lib.c_int_p)


def u32p(a):
    return a.ctypes.data_as(_lib.c_u32_p)


def backend_ptrs(backends):
    arr = (C.c_void_p * len(backends))(*[b.h for b in backends])
    return C.cast(arr, C.POINTER(C.c_void_p)), arr


def stage_mixed(ctx, backends, q_len, tokens=None):
    """zrh_stage_mixed: reserves rows in every session, returns a zr_staged handle."""
    ptrs, keep = backend_ptrs(backends)
    ql = np.ascontiguousarray(q_len, np.int32)
    toks = None if tokens is None else np.ascontiguousarray(tokens, np.uint32)
    st = C.c_void_p()
    ctx.check(ctx.lib.zrh_stage_mixed(ptrs, len(backends), i32p(ql), None if toks is None else u32p(toks),
                                      C.byref(st)))
    return st.value


def max_rel_err_rows(got, want, width):
    """max over rows of |got - want|_inf / |want|_inf, rows of `width` values."""
    g = np.asarray(got, np.float64).reshape(-1, width)
    w = np.asarray(want, np.float64).reshape(-1, width)
    return float(np.max(np.abs(g - w).max(1) / np.maximum(np.abs(w).max(1), 1e-30)))


def margin_ok_rows(logits, thresh=1e-3):
    """Rows whose top-2 logit margin exceeds `thresh` (greedy parity is only defined there)."""
    s = np.sort(logits, axis=1)
    return (s[:, -1] - s[:, -2]) > thresh
