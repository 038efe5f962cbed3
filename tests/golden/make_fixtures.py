#!/usr/bin/env python3
"""Writes the golden attention fixtures in this directory.

The reference ships no golden vectors, and its CPU kernel (ggml) is not
available, so the expected outputs here come from an independent
implementation: torch's float64 scaled_dot_product_attention on CPU, with
RoPE applied as complex multiplication (x[2i] + i*x[2i+1]) * e^{i*angle} in
float64 and angles from the closed form of src/rope.hpp:23-102.  Inputs are
stored as float32 arrays holding exactly the values of the stated storage
type (f16 / bf16), so the oracle can rebuild the typed tensors bit for bit.

Run from the repository root:  python tests/golden/make_fixtures.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
D = 128


def typed(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def angles_visual(T, Hp, Wp, axes, sf, theta):
    """float64 angles [L, D/2] of compute_visual_rope (rope.hpp:56-102)."""
    rows = []
    for t in range(T):
        for h in range(Hp):
            for w in range(Wp):
                ang = []
                for pos, a, s in zip((t, h, w), axes, sf):
                    n = a // 2
                    f = np.exp(-np.log(theta) * np.arange(n) / n)
                    ang.append(pos * f / s)
                rows.append(np.concatenate(ang))
    return np.array(rows)


def rope_f64(x, ang):
    """x (B, H, L, D) float64 rotated pairwise by ang (L, D/2)."""
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * np.exp(1j * ang)[None, None]
    out = np.empty_like(x)
    out[..., 0::2] = z.real
    out[..., 1::2] = z.imag
    return out


def sdpa(q, k, v, mask, scale):
    """q (B,H,Lq,D) f64, k/v (B,Hkv,Lk,D), mask (B or 1, 1, Lq, Lk) -> (B, Lq, H, D).
    Fully masked rows give zeros (ggml's S == 0 convention)."""
    H, Hkv = q.shape[1], k.shape[1]
    k = k.repeat_interleave(H // Hkv, dim=1)
    v = v.repeat_interleave(H // Hkv, dim=1)
    s = (q @ k.transpose(-1, -2)) * scale
    if mask is not None:
        s = s + mask
    mx = s.amax(dim=-1, keepdim=True)
    dead = torch.isinf(mx) & (mx < 0)
    p = torch.exp(s - torch.where(dead, torch.zeros_like(mx), mx))
    den = p.sum(dim=-1, keepdim=True)
    o = torch.where(den > 0, (p @ v) / torch.where(den > 0, den, torch.ones_like(den)), torch.zeros_like(den))
    # cross-check the live rows against torch's own SDPA
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale)
    live = ~dead.expand_as(o)
    assert torch.allclose(o[live], ref[live], atol=1e-12, rtol=1e-12)
    return o.permute(0, 2, 1, 3).contiguous()


def case(name, B, H, Hkv, Lq, Lk, dt, mask_kind=None, rope=None, seed=0):
    q = typed((B, H, Lq, D), dt, seed)
    k = typed((B, Hkv, Lk, D), dt, seed + 1)
    v = typed((B, Hkv, Lk, D), dt, seed + 2)
    scale = float(np.float32(1.0 / np.sqrt(D)))   # op params are F32
    mask = None
    if mask_kind == "pad":
        mask = torch.full((B, 1, Lq, Lk), float("-inf"), dtype=torch.float16)
        for b in range(B):
            mask[b, :, :, : max(1, Lk // (2 + b))] = 0.0
        mask[0, :, 1, :] = float("-inf")      # one fully masked query row
    elif mask_kind == "rand":
        g = torch.Generator().manual_seed(seed + 3)
        mask = (torch.randn((B, 1, Lq, Lk), generator=g) * 1.5).to(torch.float16)
    qd, kd, vd = q.double(), k.double(), v.double()
    extra = {}
    if rope is not None:
        T, Hp, Wp = rope
        ang = angles_visual(T, Hp, Wp, (32, 48, 48), (1.0, 2.0, 2.0), 10000.0)
        # rotated operands are rounded to the K type, as the fused op defines
        qd = torch.from_numpy(rope_f64(qd.numpy(), ang[:Lq])).to(dt).double()
        kd = torch.from_numpy(rope_f64(kd.numpy(), ang[:Lk])).to(dt).double()
        extra["rope_grid"] = np.array(rope, dtype=np.int64)
    o = sdpa(qd, kd, vd, None if mask is None else mask.double(), scale)
    np.savez_compressed(
        os.path.join(HERE, f"{name}.npz"),
        q=q.float().numpy(), k=k.float().numpy(), v=v.float().numpy(),
        mask=(mask.float().numpy() if mask is not None else np.zeros(0, np.float32)),
        dtype=np.array(str(dt).split(".")[-1]), scale=np.array(scale, dtype=np.float32),
        out=o.numpy(), **extra)
    print(name, tuple(o.shape))


def main():
    case("attn_bf16_plain", 1, 2, 2, 9, 13, torch.bfloat16, seed=100)
    case("attn_f16_gqa_padmask", 2, 4, 2, 7, 11, torch.float16, mask_kind="pad", seed=200)
    case("attn_bf16_randmask", 1, 2, 1, 6, 40, torch.bfloat16, mask_kind="rand", seed=300)
    case("attn_f16_rope_2x2x3", 1, 2, 2, 12, 12, torch.float16, rope=(2, 2, 3), seed=400)


if __name__ == "__main__":
    main()
