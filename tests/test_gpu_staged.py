"""GPU checks of the staged one-call path: kd_fa_rope_run / kd_fa_dit_run
without a workspace, whose transformed K is written into output rows that a
later head group overwrites, group by group on the 64-row kernel, with the
last group rotating K on load.

The result is defined to be kd_fa_run on the transformed operands, and the
workspace path computes exactly that; the staged path must equal it bitwise.
The shapes walk the group schedule: many groups across two and three
batches (groups never straddle a batch), a single tail head (fewer than 16
head pairs), F32 output (a group may hold twice the next group's heads) and
16-bit output (as many), TABLE and AXES RoPE, and the query/key RMSNorm; the
32-row kernel routed in its place (K rotated on load everywhere) must give
the same bits too.  Full-size: the 31,744-token self-attention, bitwise
against the workspace path and sampled rows against the float64 oracle.
"""
import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import AXES, D, HEADS, SCALE_FACTOR, THETA, assert_parity, gather_rows, qkv, randn, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _rope(mode, T, Hp, Wp):
    if mode == "table":
        tab = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
        return kd_fa.rope_table(torch.from_numpy(tab).to(DEV))
    ax = kd_fa.axes_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    return kd_fa.rope_axes(torch.from_numpy(ax).to(DEV), (T, Hp, Wp), AXES)


CASES = [
    # B, H, (T, Hp, Wp), K/V dtype, Q dtype, dst dtype, rope mode
    (2, 8, (4, 8, 8), torch.bfloat16, torch.bfloat16, torch.float32, "table"),
    (1, 5, (5, 8, 8), torch.float16, torch.float32, torch.float32, "axes"),
    (3, 3, (3, 8, 8), torch.bfloat16, torch.float32, torch.bfloat16, "table"),
    (2, 16, (2, 8, 16), torch.float16, torch.float16, torch.float16, "axes"),
    (1, 32, (2, 16, 16), torch.bfloat16, torch.float32, torch.float32, "table"),
    # token counts that are not multiples of 64 (a partial last key tile)
    (2, 8, (3, 5, 7), torch.bfloat16, torch.float32, torch.float32, "table"),
    (1, 6, (5, 9, 16), torch.float16, torch.float16, torch.bfloat16, "axes"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}L{c[2][0] * c[2][1] * c[2][2]}"
                                                        f"{str(c[3])[-4:]}o{str(c[5])[-4:]}{c[6]}")
def test_staged_equals_workspace(case):
    _need_gpu()
    B, H, (T, Hp, Wp), kt, qt, ot, mode = case
    L = T * Hp * Wp
    _announce(f"staged vs workspace {case}")
    q, k, v = (t.to(DEV) for t in qkv(B, H, L, L, kt, seed=B * 100 + H, q_dtype=qt))
    rope = _rope(mode, T, Hp, Wp)
    ws = torch.empty(k.numel(), dtype=kt, device=DEV)
    # these shapes fit one round of workgroups, where the default choice is
    # one launch rotating K on load; ROUTE_STAGED stages them anyway
    with kd_fa.routing(kd_fa.ROUTE_STAGED):
        staged = kd_fa.flash_attn_ext(q, k, v, rope=rope, out_dtype=ot)
    default = kd_fa.flash_attn_ext(q, k, v, rope=rope, out_dtype=ot)
    viaws = kd_fa.flash_attn_ext(q, k, v, rope=rope, workspace=ws, out_dtype=ot)
    with kd_fa.routing(kd_fa.ROUTE_NO_W64):
        onload = kd_fa.flash_attn_ext(q, k, v, rope=rope, out_dtype=ot)
    torch.cuda.synchronize()
    assert torch.equal(staged, viaws)
    assert torch.equal(staged, onload)
    assert torch.equal(default, viaws)
    if mode == "table":
        tab = torch.from_numpy(kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA))
        rows = sample_rows(B, H, L, 40, seed=H)
        ref = orc.fa_f64(q.cpu(), k.cpu(), v.cpu(), rope=orc.rope_table(tab), rows=rows)
        assert_parity(gather_rows(staged.float(), rows, H, L), ref, f"staged {case}")


def test_staged_norm_and_rope_equals_workspace():
    """kd_fa_dit_run without a workspace (query/key RMSNorm, RoPE) equals it
    with one."""
    _need_gpu()
    _announce("staged dit norm+rope")
    B, H, T, Hp, Wp = 2, 6, 4, 8, 8
    L = T * Hp * Wp
    q, k, v = (t.to(DEV) for t in qkv(B, H, L, L, torch.bfloat16, seed=9, q_dtype=torch.float32))
    wq = (randn((D,), torch.float32, 10) * 0.3 + 1.0).to(DEV)
    wk = (randn((D,), torch.float32, 11) * 0.3 + 1.0).to(DEV)
    norm = kd_fa.qk_norm(wq, wk, 1e-6)
    rope = _rope("table", T, Hp, Wp)
    ws = torch.empty(k.numel(), dtype=k.dtype, device=DEV)
    with kd_fa.routing(kd_fa.ROUTE_STAGED):
        a = kd_fa.flash_attn_ext(q, k, v, rope=rope, norm=norm)
    a1 = kd_fa.flash_attn_ext(q, k, v, rope=rope, norm=norm)   # one launch, K on load
    b = kd_fa.flash_attn_ext(q, k, v, rope=rope, norm=norm, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(a1, b)


def test_staged_production_shape():
    """kd_fa_rope_run at the 31,744-token shape (bf16, batch 2, 32 heads):
    bitwise the workspace path's result; 32 sampled rows per (b, h) against
    the oracle."""
    _need_gpu()
    B, T = 2, 31
    L = T * 32 * 32
    _announce(f"staged production [128,{L},32,{B}] bf16 rope")
    g = torch.Generator(device=DEV).manual_seed(3)
    q, k, v = (torch.randn((B, HEADS, L, D), generator=g, device=DEV).to(torch.bfloat16) for _ in range(3))
    tab = kd_fa.visual_rope_table(T, 32, 32, AXES, SCALE_FACTOR, THETA)
    rope = kd_fa.rope_table(torch.from_numpy(tab).to(DEV))
    staged = kd_fa.flash_attn_ext(q, k, v, rope=rope)
    ws = torch.empty(k.numel(), dtype=k.dtype, device=DEV)
    viaws = kd_fa.flash_attn_ext(q, k, v, rope=rope, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(staged, viaws)
    rows = sample_rows(B, HEADS, L, 32, seed=5)
    ref = orc.fa_f64(q.cpu(), k.cpu(), v.cpu(), rope=orc.rope_table(torch.from_numpy(tab)), rows=rows)
    m = assert_parity(gather_rows(staged, rows, HEADS, L), ref, "staged production")
    print(f"[staged production] {m}", flush=True)
