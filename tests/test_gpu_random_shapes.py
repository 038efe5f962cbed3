"""Seeded random shapes through every kernel choice.

Each case draws a shape (ragged Lq and Lk from 1 to 1,500 keys, grouped-query
and batch broadcast of K/V), the operand types (K/V F16 or BF16, Q F32 or in
K's type), a mask (none, a per-batch padding mask, or random finite values
with -inf holes), and a scale (positive or negative), then runs the node
under each routing choice of kd_fa_set_routing: as routed, with the 64-row
and long-prompt kernels out, with the short-key kernel out, with the 64-row
kernel taking the short unmasked key sets too, with all specialised
kernels out, and with the persistent 32-row long-prompt kernel in place of
the 64-row one.  Every
kernel computes each query row with the same arithmetic, so all outputs must
be bitwise equal; the routed one must also match the float64 oracle on every
row.  Odd seeds give the mask rows whole 8-key chunks (ggml pads them; the
values past Lk must not count), which lets masked key sets of up to 256 keys
reach the short-key kernel, and every case also runs kd_fa_run_ws (the mask
summary), which must give the same bits.  The cases are fixed by their seeds
(no draw differs between runs).
"""
import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import D, assert_parity, gather_rows, randn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ROUTES = [kd_fa.ROUTE_DEFAULT, kd_fa.ROUTE_NO_W64, kd_fa.ROUTE_NO_XRES, kd_fa.ROUTE_W64_SHORT,
          kd_fa.ROUTE_NO_W64 | kd_fa.ROUTE_NO_XRES, kd_fa.ROUTE_NO_XLONG64]


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _case(seed):
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.choice([1, 2]))
    Bk = int(rng.choice([b for b in (1, 2) if B % b == 0]))
    H = int(rng.choice([1, 2, 4]))
    Hkv = int(rng.choice([h for h in (1, 2, 4) if H % h == 0]))
    Lq = int(rng.integers(1, 301))
    # key counts in each kernel's range: < 64, the short-key kernel's, the
    # long-prompt kernel's (unmasked) and the 64-row kernel's
    bins = [(1, 64), (64, 257), (257, 1025), (1025, 1501)]
    lo, hi = bins[seed % 4]
    Lk = int(rng.integers(lo, hi))
    kv = [torch.float16, torch.bfloat16][int(rng.integers(2))]
    qt = [torch.float32, kv][int(rng.integers(2))]
    mask = ["none", "pad", "rand"][(seed // 4) % 3]
    scale = float(rng.uniform(0.03, 0.2)) * (-1 if seed % 5 == 4 else 1)
    return B, Bk, H, Hkv, Lq, Lk, kv, qt, mask, scale


def _mask(kind, B, Lq, Lk, seed, ne0=None):
    if kind == "none":
        return None
    ne0 = Lk if ne0 is None else ne0
    g = torch.Generator().manual_seed(seed)
    if kind == "pad":
        m = torch.full((B, 1, Lq, ne0), float("-inf"), dtype=torch.float16)
        for b in range(B):
            m[b, :, :, : int(torch.randint(1, Lk + 1, (1,), generator=g))] = 0.0
    else:
        m = (torch.randn((B, 1, Lq, ne0), generator=g) * 2).to(torch.float16)
        m[torch.rand((B, 1, Lq, ne0), generator=g) < 0.3] = float("-inf")
    m[..., Lk:] = 3.0       # padding past Lk: never read as a key
    return m


@pytest.mark.parametrize("seed", range(24))
def test_random_shape_all_routes_bitwise_and_oracle(seed):
    _need_gpu()
    B, Bk, H, Hkv, Lq, Lk, kv, qt, mk, scale = _case(seed)
    what = f"seed {seed}: B{B} Bk{Bk} H{H} Hkv{Hkv} Lq{Lq} Lk{Lk} {kv} q{qt} mask {mk} scale {scale:.4f}"
    print(f"[case] {what}", flush=True)
    q = randn((B, H, Lq, D), qt, 50 + seed)
    k = randn((Bk, Hkv, Lk, D), kv, 150 + seed)
    v = randn((Bk, Hkv, Lk, D), kv, 250 + seed)
    mask = _mask(mk, B, Lq, Lk, 350 + seed, ne0=(Lk + 7) // 8 * 8 if seed % 2 else None)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    mg = None if mask is None else mask.to(DEV)
    outs = []
    for route in ROUTES:
        with kd_fa.routing(route):
            outs.append(kd_fa.flash_attn_ext(qg, kg, vg, mask=mg, scale=scale))
    # kd_fa_run_ws: the mask summary where the short-key kernel runs
    out_ws = torch.empty_like(outs[0])
    d = kd_fa.make_desc(qg, kg, vg, mg, out_ws, scale)
    ws = torch.empty(max(kd_fa.workspace_size_full(d), 16), dtype=torch.uint8, device=DEV).fill_(0x5A)
    with kd_fa.routing(kd_fa.ROUTE_SUMMARY):     # (these shapes are below the summary's row threshold)
        assert kd_fa.run_desc(d, workspace=ws) == kd_fa.OK
    torch.cuda.synchronize()
    for route, out in zip(ROUTES[1:], outs[1:]):
        assert torch.equal(out, outs[0]), f"{what}: route {route} differs from the routed output"
    assert torch.equal(out_ws, outs[0]), f"{what}: kd_fa_run_ws differs from kd_fa_run"
    ref = orc.fa_f64(q, k, v, mask=mask, scale=scale)
    got = gather_rows(outs[0], np.arange(B * H * Lq), H, Lq)
    assert_parity(got, ref, what)
