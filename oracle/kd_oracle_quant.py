"""CPU restatement of the linear-layer path: the weight block formats and the
GGML_OP_MUL_MAT arithmetic of ops::linear (src/core/ops.hpp:27-43).

TEST INFRASTRUCTURE ONLY: results are checked against it.  Imported by tests/, never by the
product (kandinsky.cpp_amd/).

Sources restated (numpy, vectorised):
- quantize_q8_0 / quantize_q4_0: the reference's converter,
  scripts/convert_to_gguf.py:93-143 (the files the model loader reads).
- dequantize: ggml's dequantize_row_q8_0 / dequantize_row_q4_0 [ggml
  upstream, ggml/src/ggml-quants.c; unpinned, absent here]: value = q * d
  and (nibble - 8) * d in F32, low nibble element j, high nibble j + 16 --
  the layout the converter's comments state (convert_to_gguf.py:121-123).
- quantize_row_q8_0_ggml + mul_mat_ggml: ggml's CPU GGML_OP_MUL_MAT for
  Q4_0 / Q8_0 weights [ggml upstream]: each x row is quantized to Q8_0
  (d = amax / 127, q = roundf(x / d) via x * (1 / d)), then per 32-block an
  integer dot product scaled by the two F16 scales, summed in F32 in block
  order (ggml_vec_dot_q8_0_q8_0 / _q4_0_q8_0, scalar form).  Parity with
  ggml itself is unpinned (ggml is not available); tests pin these
  functions by closed forms and invariants.
- mul_mat_f64: the exact product in float64.
"""
from __future__ import annotations

import numpy as np

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0, TYPE_BF16 = 0, 1, 2, 8, 30
BLOCK_BYTES = {TYPE_Q8_0: 34, TYPE_Q4_0: 18}


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """convert_to_gguf.py:93-113 on each row of w (N, K): uint8 (N, K/32*34).
    scale = amax / 127 (1 for an all-zero block), q = clip(round-half-even(
    x / scale), -128, 127), the scale stored as F16."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    blocks = w.reshape(N * K // 32, 32)
    amax = np.max(np.abs(blocks), axis=1)
    scales = amax / np.float32(127.0)
    scales[scales == 0] = 1.0
    q = np.clip(np.round(blocks / scales[:, None]), -128, 127).astype(np.int8)
    out = np.empty((blocks.shape[0], 34), dtype=np.uint8)
    out[:, :2] = scales.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(N, K // 32 * 34)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """convert_to_gguf.py:116-143 on each row of w (N, K): uint8 (N, K/32*18).
    d = (the block's signed value of largest magnitude) / -8; q = clip(
    trunc(x / d + 8.5), 0, 15); low nibble element j, high nibble j + 16."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    blocks = w.reshape(N * K // 32, 32)
    nbk = blocks.shape[0]
    amax = np.max(np.abs(blocks), axis=1)
    max_idx = np.argmax(np.abs(blocks), axis=1)
    max_signed = blocks[np.arange(nbk), max_idx]
    scales = max_signed / np.float32(-8.0)
    inv = np.zeros_like(scales, dtype=np.float32)
    nz = amax > 0
    inv[nz] = np.float32(1.0) / scales[nz]
    x0 = blocks[:, :16] * inv[:, None]
    x1 = blocks[:, 16:] * inv[:, None]
    q0 = np.clip((x0 + np.float32(8.5)).astype(np.int32), 0, 15).astype(np.uint8)
    q1 = np.clip((x1 + np.float32(8.5)).astype(np.int32), 0, 15).astype(np.uint8)
    out = np.empty((nbk, 18), dtype=np.uint8)
    out[:, :2] = scales.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q0 | (q1 << 4)
    return out.reshape(N, K // 32 * 18)


def block_fields(blocks: np.ndarray, qtype: int, K: int):
    """(d F32 (N, K/32), q int (N, K/32, 32)) of Q8_0 / Q4_0 rows; Q4_0 q is
    nibble - 8 in element order."""
    N = blocks.shape[0]
    bb = BLOCK_BYTES[qtype]
    b = np.ascontiguousarray(blocks).reshape(N, K // 32, bb)
    d = b[:, :, :2].copy().view(np.float16)[..., 0].astype(np.float32)
    if qtype == TYPE_Q8_0:
        q = b[:, :, 2:].view(np.int8).astype(np.int32)
    else:
        p = b[:, :, 2:].astype(np.int32)
        q = np.concatenate([(p & 15) - 8, (p >> 4) - 8], axis=2)
    return d, q


def dequantize(blocks: np.ndarray, qtype: int, K: int) -> np.ndarray:
    """ggml's dequantize_row_q8_0 / _q4_0: F32 (N, K), value = q * d."""
    d, q = block_fields(blocks, qtype, K)
    return (q.astype(np.float32) * d[:, :, None]).reshape(blocks.shape[0], K)


def round_bf16(a: np.ndarray) -> np.ndarray:
    """F32 -> BF16 (round to nearest even) -> F32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = out.copy()
        out[nan] = np.float32(np.nan)
    return out


def quantize_row_q8_0_ggml(x: np.ndarray):
    """ggml's quantize_row_q8_0_ref on each row of x (M, K): (d F32 of the
    stored F16 scale (M, K/32), q int (M, K/32, 32))."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    b = x.reshape(M, K // 32, 32)
    amax = np.max(np.abs(b), axis=2)
    d = amax / np.float32(127.0)
    idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), np.float32(0.0)).astype(np.float32)
    v = b * idv[:, :, None]
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int32)   # roundf: half away from zero
    return d.astype(np.float16).astype(np.float32), q


def mul_mat_ggml(w, qtype: int, x: np.ndarray) -> np.ndarray:
    """ggml's CPU GGML_OP_MUL_MAT for Q8_0 / Q4_0 weights (blocks uint8 rows)
    and F32 x (M, K): F32 (M, N).  Float weights: x rounded to the weight's
    type, products accumulated in float64 (the scalar ggml_vec_dot_f16)."""
    x = np.asarray(x, dtype=np.float32)
    M, K = x.shape
    if qtype in BLOCK_BYTES:
        dw, qw = block_fields(w, qtype, K)                 # (N, nb), (N, nb, 32)
        dx, qx = quantize_row_q8_0_ggml(x)                 # (M, nb), (M, nb, 32)
        sumi = np.einsum("mbj,nbj->mnb", qx, qw, dtype=np.int64).astype(np.float32)
        if qtype == TYPE_Q8_0:
            terms = sumi * (dx[:, None, :] * dw[None, :, :])
        else:
            terms = (sumi * dw[None, :, :]) * dx[:, None, :]
        acc = np.zeros((M, w.shape[0]), dtype=np.float32)
        for ib in range(terms.shape[2]):                   # F32 sum in block order
            acc = (acc + terms[:, :, ib]).astype(np.float32)
        return acc
    wf = np.asarray(w, dtype=np.float32)
    if qtype == TYPE_F16:
        xr = x.astype(np.float16).astype(np.float64)
    elif qtype == TYPE_BF16:
        xr = round_bf16(x).astype(np.float64)
    else:
        xr = x.astype(np.float64)
    return (xr @ wf.astype(np.float64).T).astype(np.float32)


def mul_mat_f64(w_f32: np.ndarray, x: np.ndarray, bias=None) -> np.ndarray:
    """sum_k w[n][k] x[m][k] (+ bias[n]) in float64: (M, N)."""
    r = np.asarray(x, dtype=np.float64) @ np.asarray(w_f32, dtype=np.float64).T
    if bias is not None:
        r = r + np.asarray(bias, dtype=np.float64)[None, :]
    return r


def abs_product_sum(w_f32: np.ndarray, x: np.ndarray) -> np.ndarray:
    """sum_k |w[n][k] x[m][k]| (M, N): the scale of a sum's rounding error."""
    return np.abs(np.asarray(x, dtype=np.float64)) @ np.abs(np.asarray(w_f32, dtype=np.float64)).T
