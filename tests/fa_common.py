"""Shared helpers for the flash-attention tests: seeded inputs, the CrossDiT
workload shapes, row sampling and the parity metrics."""
from __future__ import annotations

import numpy as np
import torch

D = 128
# Parity gate against a float64 CPU result on the same rounded operands.
TOL_MAX_ABS = 2e-2
TOL_COS = 0.9995

# CrossDiT Pro constants (src/models/crossdit.hpp:67-75): head_dim 128 =
# 32 + 48 + 48 (t/h/w), 32 heads, RoPE theta 10000, scale_factor (1, 2, 2).
AXES = (32, 48, 48)
SCALE_FACTOR = (1.0, 2.0, 2.0)
THETA = 10000.0
HEADS = 32


def randn(shape, dtype, seed, device="cpu"):
    """N(0, 1) float32 from a seeded generator, rounded to dtype."""
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32, device=device).to(dtype)


def qkv(B, H, Lq, Lk, dtype, seed, device="cpu", Hkv=None, Bk=None, q_dtype=None):
    """q (B, H, Lq, D), k/v (Bk, Hkv, Lk, D): ggml [D, L, H, B] views."""
    Hkv = H if Hkv is None else Hkv
    Bk = B if Bk is None else Bk
    q = randn((B, H, Lq, D), q_dtype or dtype, seed, device)
    k = randn((Bk, Hkv, Lk, D), dtype, seed + 1000, device)
    v = randn((Bk, Hkv, Lk, D), dtype, seed + 2000, device)
    return q, k, v


def padding_mask(B, Lq, Lk, valid, device="cpu", pad_rows=0):
    """F16 mask (B, 1, Lq+pad_rows, Lk): 0 for keys j < valid[b], -inf after
    (a per-batch text padding mask broadcast over heads)."""
    m = torch.full((B, 1, Lq + pad_rows, Lk), float("-inf"), dtype=torch.float16, device=device)
    for b in range(B):
        m[b, :, :, : valid[b]] = 0.0
    return m


def sample_rows(B, H, Lq, per_head, seed):
    """Row ids i + Lq*(h + H*b) with `per_head` query rows per (b, h),
    always including the first and last row."""
    rng = np.random.default_rng(seed)
    rows = []
    for b in range(B):
        for h in range(H):
            if per_head >= Lq:
                idx = np.arange(Lq)
            else:
                idx = rng.choice(Lq, size=per_head, replace=False)
                idx[0], idx[-1] = 0, Lq - 1
                idx = np.unique(idx)
            rows.append(idx + Lq * (h + H * b))
    return np.concatenate(rows).astype(np.int64)


def gather_rows(dst, rows, H, Lq):
    """dst (B, Lq, H, Dv) -> (n_rows, Dv) float64 in the order of rows."""
    rows = np.asarray(rows)
    i = rows % Lq
    h = (rows // Lq) % H
    b = rows // (Lq * H)
    d = dst.detach().to("cpu", torch.float64).numpy()
    return d[b, i, h, :]


def metrics(got, ref):
    got = np.asarray(got, dtype=np.float64).reshape(-1, np.shape(ref)[-1])
    ref = np.asarray(ref, dtype=np.float64).reshape(got.shape)
    err = float(np.max(np.abs(got - ref))) if got.size else 0.0
    num = float(np.sum(got * ref))
    den = float(np.sqrt(np.sum(got * got) * np.sum(ref * ref)))
    cos = num / den if den > 0 else (1.0 if np.allclose(got, ref) else 0.0)
    rn = np.sqrt(np.sum(got * got, axis=1) * np.sum(ref * ref, axis=1))
    rc = np.where(rn > 0, np.sum(got * ref, axis=1) / np.where(rn > 0, rn, 1), 1.0)
    return {"max_abs": err, "cos": cos, "min_row_cos": float(rc.min()) if rc.size else 1.0,
            "finite": bool(np.isfinite(got).all())}


def assert_parity(got, ref, what=""):
    m = metrics(got, ref)
    assert m["finite"], f"{what}: non-finite output"
    assert m["max_abs"] <= TOL_MAX_ABS, f"{what}: max_abs {m['max_abs']:.3e} > {TOL_MAX_ABS} ({m})"
    assert m["cos"] >= TOL_COS, f"{what}: cosine {m['cos']:.6f} < {TOL_COS} ({m})"
    return m


def grid_tokens(T, Hp, Wp):
    return T * Hp * Wp
