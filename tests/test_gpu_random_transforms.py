"""Seeded random shapes through the transformed-operand entry points.

Each case draws a self-attention shape (ragged token counts from 1 to 2,600,
grouped-query and batch broadcast of K/V), the operand types (K/V F16 or
BF16, Q F32 or in K's type) and a scale (positive or negative), with RoPE
from a random table, and runs it:
- kd_fa_rope_run without a workspace (K rotated staged or on load) and
  kd_fa_rope_run_ws (K rotated once into the workspace), each under every
  routing choice of kd_fa_set_routing -- all bitwise equal, since every
  kernel computes each query row with the same arithmetic;
- on odd seeds, kd_fa_dit_run with query/key RMSNorm too, with and without a
  workspace (bitwise equal);
- with a 16-bit dst (bitwise the F32 result rounded);
and the routed F32 result must match the float64 oracle (rope::apply by the
oracle, rounded to K's type, then the attention) on sampled rows.  The
cases are fixed by their seeds.
"""
import ctypes

import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import D, assert_parity, gather_rows, randn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ROUTES = [kd_fa.ROUTE_DEFAULT, kd_fa.ROUTE_NO_W64, kd_fa.ROUTE_W64_SHORT, kd_fa.ROUTE_STAGED]


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _case(seed):
    rng = np.random.default_rng(4000 + seed)
    B = int(rng.choice([1, 2]))
    Bk = int(rng.choice([b for b in (1, 2) if B % b == 0]))
    H = int(rng.choice([1, 2, 4, 8]))
    Hkv = int(rng.choice([h for h in (1, 2, 4, 8) if H % h == 0]))
    L = int(rng.integers(1, 2601))
    kv = [torch.float16, torch.bfloat16][int(rng.integers(2))]
    qt = [torch.float32, kv][int(rng.integers(2))]
    scale = float(rng.uniform(0.03, 0.2)) * (-1 if seed % 5 == 4 else 1)
    return B, Bk, H, Hkv, L, kv, qt, scale


def _rot(x, table, dtype):
    """rope::apply in F32 by the oracle, rounded to dtype: x (B, H, L, D)."""
    xb = x.float().permute(0, 2, 1, 3).contiguous().numpy()
    r = orc.rope_apply(xb, table[: x.shape[2]])
    return torch.from_numpy(r).permute(0, 2, 1, 3).contiguous().to(dtype)


def _dit_run(desc, rope, norm, ws):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if ws is None:
        return kd_fa.lib().kd_fa_dit_run(ctypes.byref(desc), ctypes.byref(rope), ctypes.byref(norm), None, 0, stream)
    return kd_fa.run_desc(desc, rope, None, ws, norm)


@pytest.mark.parametrize("seed", range(16))
def test_random_rope_norm_routes_bitwise_and_oracle(seed):
    _need_gpu()
    B, Bk, H, Hkv, L, kv, qt, scale = _case(seed)
    what = f"seed {seed}: B{B} Bk{Bk} H{H} Hkv{Hkv} L{L} {kv} q{qt} scale {scale:.4f}"
    print(f"[case] {what}", flush=True)
    q = randn((B, H, L, D), qt, 60 + seed)
    k = randn((Bk, Hkv, L, D), kv, 160 + seed)
    v = randn((Bk, Hkv, L, D), kv, 260 + seed)
    table = np.random.default_rng(seed).uniform(-1.0, 1.0, (L, D)).astype(np.float32)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))

    outs = []
    for route in ROUTES:
        for use_ws in (False, True):
            o = torch.empty((B, L, H, D), device=DEV)
            d = kd_fa.make_desc(qg, kg, vg, None, o, scale)
            ws = None
            if use_ws:
                ws = torch.empty(max(kd_fa.workspace_size_full(d, rope), 16), dtype=torch.uint8, device=DEV)
                ws.fill_(0x5A)
            with kd_fa.routing(route):
                assert kd_fa.run_desc(d, rope, None, ws) == kd_fa.OK, (what, route, use_ws)
            outs.append(((route, use_ws), o))
    odt = [torch.bfloat16, torch.float16][seed % 2]
    o16 = torch.empty((B, L, H, D), device=DEV, dtype=odt)
    assert kd_fa.run_desc(kd_fa.make_desc(qg, kg, vg, None, o16, scale), rope) == kd_fa.OK
    if seed % 2:
        wq = (randn((D,), torch.float32, 900 + seed) * 0.3 + 1.0).to(DEV)
        wk = (randn((D,), torch.float32, 901 + seed) * 0.3 + 1.0).to(DEV)
        norm = kd_fa.qk_norm(wq, wk, 1e-6)
        on = []
        for use_ws in (False, True):
            o = torch.empty((B, L, H, D), device=DEV)
            d = kd_fa.make_desc(qg, kg, vg, None, o, scale)
            ws = None
            if use_ws:
                ws = torch.empty(max(kd_fa.workspace_size_full(d, rope, norm), 16), dtype=torch.uint8, device=DEV)
            assert _dit_run(d, rope, norm, ws) == kd_fa.OK, (what, "norm", use_ws)
            on.append(o)
    torch.cuda.synchronize()
    for key, o in outs[1:]:
        assert torch.equal(o, outs[0][1]), f"{what}: {key} differs from the routed call without a workspace"
    assert torch.equal(o16, outs[0][1].to(odt)), f"{what}: 16-bit dst is not the rounded F32 result"
    if seed % 2:
        assert torch.isfinite(on[0]).all(), what
        assert torch.equal(on[0], on[1]), f"{what}: kd_fa_dit_run with and without a workspace differ"
    rows = np.sort(np.random.default_rng(seed).choice(B * H * L, size=min(32, B * H * L), replace=False))
    ref = orc.fa_f64(_rot(q, table, kv), _rot(k, table, kv), v, scale=scale, rows=rows)
    assert_parity(gather_rows(outs[0][1], rows, H, L), ref, what)
