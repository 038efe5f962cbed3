"""ctypes binding of oracle/libkd_oracle.so.

TEST INFRASTRUCTURE ONLY: results are checked against it.  Imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
product (kandinsky.cpp_amd/).

Operands are CPU torch tensors laid out like the product binding's
(shape = ggml ``ne`` reversed); the descriptor structs mirror
include/kd_fa.h and are defined here independently of the product code.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# KD_ORACLE_LIB selects another build of the same library (the sanitized one)
LIB_PATH = os.environ.get("KD_ORACLE_LIB") or os.path.join(_HERE, "libkd_oracle.so")

TYPE_F32, TYPE_F16, TYPE_BF16 = 0, 1, 30
ROPE_NONE, ROPE_TABLE, ROPE_AXES = 0, 1, 2


class Tensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4), ("data", ctypes.c_void_p)]


class Desc(ctypes.Structure):
    _fields_ = [("q", Tensor), ("k", Tensor), ("v", Tensor), ("mask", Tensor), ("sinks", Tensor), ("dst", Tensor),
                ("scale", ctypes.c_float), ("max_bias", ctypes.c_float),
                ("logit_softcap", ctypes.c_float), ("prec", ctypes.c_int32), ("cast_type", ctypes.c_int32)]


class Rope(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("table", Tensor), ("axes_data", ctypes.c_void_p),
                ("grid", ctypes.c_int32 * 3), ("axes", ctypes.c_int32 * 3)]


_LIB = None


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER
        fp, ip, dp = P(ctypes.c_float), P(ctypes.c_int), P(ctypes.c_double)
        L.kdo_f32_to_f16.argtypes = [ctypes.c_float]
        L.kdo_f32_to_f16.restype = ctypes.c_uint16
        L.kdo_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.kdo_f16_to_f32.restype = ctypes.c_float
        L.kdo_f32_to_bf16.argtypes = [ctypes.c_float]
        L.kdo_f32_to_bf16.restype = ctypes.c_uint16
        L.kdo_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.kdo_bf16_to_f32.restype = ctypes.c_float
        for name in ("kdo_f32_to_f16_n", "kdo_f32_to_bf16_n"):
            getattr(L, name).argtypes = [fp, P(ctypes.c_uint16), ctypes.c_int64]
        for name in ("kdo_f16_to_f32_n", "kdo_bf16_to_f32_n"):
            getattr(L, name).argtypes = [P(ctypes.c_uint16), fp, ctypes.c_int64]
        L.kdo_f32_to_f16_hw_n.argtypes = [fp, P(ctypes.c_uint16), ctypes.c_int64]
        L.kdo_f16_to_f32_hw_n.argtypes = [P(ctypes.c_uint16), fp, ctypes.c_int64]
        L.kdo_f16_codec_mismatches.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int64]
        L.kdo_f16_codec_mismatches.restype = ctypes.c_int64
        L.kdo_rope_freqs.argtypes = [ctypes.c_int, ctypes.c_float, fp]
        L.kdo_rope_text_table.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, fp]
        L.kdo_rope_visual_table.argtypes = [ctypes.c_int] * 3 + [ip, fp, ctypes.c_float, fp]
        L.kdo_rope_apply_f32.argtypes = [fp] + [ctypes.c_int64] * 4 + [fp, fp]
        L.kdo_rms_norm_mul.argtypes = [fp, ctypes.c_int64, ctypes.c_int64, fp, ctypes.c_float, fp]
        L.kdo_fa_ggml.argtypes = [P(Desc), P(Rope), ctypes.c_int, P(ctypes.c_int64), ctypes.c_int64, ctypes.c_int]
        L.kdo_fa_ggml.restype = ctypes.c_int
        L.kdo_fa_f64.argtypes = [P(Desc), P(Rope), P(ctypes.c_int64), ctypes.c_int64, dp, ctypes.c_int]
        L.kdo_fa_f64.restype = ctypes.c_int
        _LIB = L
    return _LIB


def _type(dtype):
    return {torch.float32: TYPE_F32, torch.float16: TYPE_F16, torch.bfloat16: TYPE_BF16}[dtype]


def view(t) -> Tensor:
    d = Tensor()
    if t is None:
        return d
    assert t.device.type == "cpu" and t.dim() <= 4
    es = t.element_size()
    shape = list(t.shape)[::-1]
    strides = [s * es for s in list(t.stride())[::-1]]
    while len(shape) < 4:
        shape.append(1)
        strides.append(strides[-1] * shape[-2] if strides else es)
    d.type = _type(t.dtype)
    for i in range(4):
        d.ne[i] = int(shape[i])
        d.nb[i] = int(strides[i])
    d.data = t.data_ptr() if t.numel() else 0
    return d


def make_desc(q, k, v, mask=None, dst=None, scale=None, max_bias=0.0, logit_softcap=0.0):
    d = Desc()
    d._keep = (q, k, v, mask, dst)
    d.q, d.k, d.v, d.mask, d.dst = view(q), view(k), view(v), view(mask), view(dst)
    d.scale = float(1.0 / q.shape[-1] ** 0.5 if scale is None else scale)
    d.max_bias = float(max_bias)
    d.logit_softcap = float(logit_softcap)
    d.prec = 10
    return d


def rope_table(table) -> Rope:
    r = Rope()
    r.mode = ROPE_TABLE
    r.table = view(table)
    r._keep = table
    return r


def rope_axes(axes_buf, grid, axes) -> Rope:
    r = Rope()
    r.mode = ROPE_AXES
    r.axes_data = axes_buf.data_ptr()
    r._keep = axes_buf
    for i in range(3):
        r.grid[i] = int(grid[i])
        r.axes[i] = int(axes[i])
    return r


def _rows(rows):
    if rows is None:
        return None, 0, None
    arr = np.ascontiguousarray(np.asarray(rows, dtype=np.int64))
    return arr.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), len(arr), arr


def row_id(b, h, i, H, Lq):
    """Flat query-row id (ggml's ir order): i + Lq*(h + H*b)."""
    return i + Lq * (h + H * b)


def fa_ggml(q, k, v, mask=None, scale=None, rope=None, f16_vacc=True, rows=None,
            n_threads=0, max_bias=0.0, logit_softcap=0.0, dst=None):
    """ggml's per-row CPU algorithm (restated).  Returns (dst, threads):
    dst (B, Lq, H, Dv) float32 with the requested rows written."""
    if dst is None:
        dst = torch.zeros((q.shape[0], q.shape[2], q.shape[1], v.shape[3]), dtype=torch.float32)
    d = make_desc(q, k, v, mask, dst, scale, max_bias, logit_softcap)
    rp, n, _keep = _rows(rows)
    st = lib().kdo_fa_ggml(ctypes.byref(d), ctypes.byref(rope) if rope is not None else None,
                           int(bool(f16_vacc)), rp, n, int(n_threads))
    if st < 0:
        raise RuntimeError(f"kdo_fa_ggml failed: {st}")
    return dst, st


def fa_f64(q, k, v, mask=None, scale=None, rope=None, rows=None, n_threads=0,
           max_bias=0.0, logit_softcap=0.0):
    """Textbook attention in double.  Returns float64 array (n_rows, Dv);
    rows=None gives every row in row_id order."""
    Lq, H, B = q.shape[2], q.shape[1], q.shape[0]
    n = len(rows) if rows is not None else Lq * H * B
    out = np.zeros((n, v.shape[3]), dtype=np.float64)
    d = make_desc(q, k, v, mask, None, scale, max_bias, logit_softcap)
    rp, nr, _keep = _rows(rows)
    st = lib().kdo_fa_f64(ctypes.byref(d), ctypes.byref(rope) if rope is not None else None,
                          rp, nr, out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)), int(n_threads))
    if st < 0:
        raise RuntimeError(f"kdo_fa_f64 failed: {st}")
    return out


def visual_rope_table(T, Hp, Wp, axes=(32, 48, 48), scale_factor=(1.0, 2.0, 2.0), theta=10000.0):
    out = np.empty((T * Hp * Wp, sum(axes)), dtype=np.float32)
    lib().kdo_rope_visual_table(T, Hp, Wp, (ctypes.c_int * 3)(*axes),
                                (ctypes.c_float * 3)(*scale_factor), theta,
                                out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out


def text_rope_table(L, D=128, theta=10000.0):
    out = np.empty((L, D), dtype=np.float32)
    lib().kdo_rope_text_table(L, D, theta, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out


def rope_freqs(dim, theta=10000.0):
    out = np.empty(max(dim, 1), dtype=np.float32)
    lib().kdo_rope_freqs(dim, theta, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out[:dim]


def rope_apply(x, table):
    """rope::apply on x float32 (B, L, H, D) with table (L, D)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    t = np.ascontiguousarray(table, dtype=np.float32)
    B, L, H, D = x.shape
    out = np.empty_like(x)
    fp = ctypes.POINTER(ctypes.c_float)
    lib().kdo_rope_apply_f32(x.ctypes.data_as(fp), D, H, L, B, t.ctypes.data_as(fp), out.ctypes.data_as(fp))
    return out


def rms_norm(x, weight=None, eps=1e-6):
    """ops::rms_norm (ggml_rms_norm + ggml_mul by weight) over the last axis
    of float32 x; weight float32 (D,) or None."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    D = x.shape[-1]
    rows = x.size // D if D else 0
    out = np.empty_like(x)
    fp = ctypes.POINTER(ctypes.c_float)
    w = None if weight is None else np.ascontiguousarray(weight, dtype=np.float32)
    lib().kdo_rms_norm_mul(x.ctypes.data_as(fp), rows, D, None if w is None else w.ctypes.data_as(fp),
                           float(eps), out.ctypes.data_as(fp))
    return out


def f32_to_f16_bits(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().kdo_f32_to_f16_n(a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), a.size)
    return out


def f32_to_f16_bits_hw(a):
    """f32_to_f16_bits by the F16C instruction (the CPU baseline's path)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().kdo_f32_to_f16_hw_n(a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                              out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), a.size)
    return out


def f16_codec_mismatches(start, stride, count):
    """Where the F16C and software F16 conversions differ (see kd_oracle.h)."""
    return int(lib().kdo_f16_codec_mismatches(start, stride, count))


def f32_to_bf16_bits(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().kdo_f32_to_bf16_n(a.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), a.size)
    return out


def f16_bits_to_f32(a):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().kdo_f16_to_f32_n(a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), a.size)
    return out


def bf16_bits_to_f32(a):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().kdo_bf16_to_f32_n(a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                            out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), a.size)
    return out
