"""GPU checks of the 64-rows-per-wave kernel (fa_fwd_w64), which takes the
unmasked calls whose K is read as stored and that have more than 896 keys
(shorter key sets run on the 32-row kernel's 4-wave workgroups unless the
routing flag KD_FA_ROUTE_W64_SHORT sends them here too).

Each case runs twice through the C ABI: once on the 64-row kernel
(kd_fa_set_routing(KD_FA_ROUTE_W64_SHORT)) and once with it routed out
(KD_FA_ROUTE_NO_W64: the 32-row kernel, fa_fwd_d128), and the two outputs
must be bitwise equal -- both kernels perform the same arithmetic per query
row.
Parity against the float64 oracle completes each case.  The shapes walk the
loop's control paths: 1 key tile (last step only), 2 (one step + last), 3
(a step pair + last), 4 (pair + step + last) and many; ragged Lq; GQA and
batch broadcast; strided activation views; F16 and BF16; scales that force
the running-max rescale in later tiles.
"""
import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import AXES, D, SCALE_FACTOR, THETA, assert_parity, gather_rows, qkv, randn, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _both(fn):
    """(64-row kernel output, 32-row kernel output) of fn()."""
    with kd_fa.routing(kd_fa.ROUTE_NO_W64):
        ref = fn()
        torch.cuda.synchronize()
    with kd_fa.routing(kd_fa.ROUTE_W64_SHORT):
        out = fn()
        torch.cuda.synchronize()
    return out, ref


CASES = [
    # B, H, Hkv, Bk, Lq, Lk, dtype
    (1, 2, 2, 1, 256, 64, torch.bfloat16),
    (2, 2, 1, 1, 300, 128, torch.bfloat16),
    (1, 3, 3, 1, 77, 192, torch.float16),
    (2, 4, 2, 2, 513, 256, torch.bfloat16),
    (1, 2, 2, 1, 1000, 1280, torch.float16),
    (1, 1, 1, 1, 260, 4096, torch.bfloat16),
    # Lk not a multiple of 64: the partial last tile (1 .. 63 keys) in the
    # loop after 1 .. many whole tiles
    (1, 2, 2, 1, 256, 65, torch.bfloat16),
    (2, 3, 1, 1, 130, 127, torch.float16),
    (1, 2, 2, 1, 300, 200, torch.bfloat16),
    (2, 4, 2, 2, 513, 333, torch.float16),
    (1, 2, 2, 1, 1000, 1337, torch.bfloat16),
    (1, 1, 1, 1, 77, 4095, torch.float16),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}kv{c[2]}Bk{c[3]}q{c[4]}k{c[5]}{str(c[6])[-4:]}")
def test_w64_equals_w32(case):
    _need_gpu()
    B, H, Hkv, Bk, Lq, Lk, dt = case
    _announce(f"w64 vs w32 {case}")
    q, k, v = qkv(B, H, Lq, Lk, dt, seed=Lq + Lk, Hkv=Hkv, Bk=Bk)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg))
    assert torch.equal(out, ref)
    rows = sample_rows(B, H, Lq, 48, seed=Lk)
    assert_parity(gather_rows(out, rows, H, Lq), orc.fa_f64(q, k, v, rows=rows), f"w64 {case}")


@pytest.mark.parametrize("Lk", [640, 650])
@pytest.mark.parametrize("scale", [-0.0883883, 0.0, 0.5, 4.0], ids=["neg", "zero", "large", "huge"])
def test_w64_scales_and_rescale(scale, Lk):
    """Keys that grow tile by tile move the running max again and again
    (the out-of-line rescale of O in the accumulation registers; with
    Lk = 650 the partial last tile's rescale too)."""
    _need_gpu()
    _announce(f"w64 scale {scale} Lk {Lk}")
    B, H, Lq = 1, 2, 200
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=31)
    growth = torch.linspace(0.2, 3.0, Lk).view(1, 1, Lk, 1)
    k = (k.float() * growth).to(torch.bfloat16)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, scale=scale))
    assert torch.equal(out, ref)
    assert_parity(gather_rows(out, np.arange(B * H * Lq), H, Lq), orc.fa_f64(q, k, v, scale=scale), "w64 scale")


def test_w64_strided_views_and_16bit_out():
    _need_gpu()
    _announce("w64 strided views, bf16 out")
    L, H = 320, 4
    g = torch.Generator().manual_seed(41)
    act = [torch.randn((1, L, H, D), generator=g).to(torch.bfloat16) for _ in range(3)]
    q, k, v = [a.permute(0, 2, 1, 3) for a in act]
    qg, kg, vg = [a.to(DEV).permute(0, 2, 1, 3) for a in act]
    for odt in (None, torch.bfloat16):
        out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, out_dtype=odt))
        assert torch.equal(out, ref)
    out32 = kd_fa.flash_attn_ext(qg, kg, vg)
    torch.cuda.synchronize()
    assert_parity(gather_rows(out32, np.arange(H * L), H, L),
                  orc.fa_f64(q.contiguous(), k.contiguous(), v.contiguous()), "w64 strided")


@pytest.mark.parametrize("mode", ["table", "axes"])
def test_w64_rope_workspace(mode):
    """kd_fa_rope_run_ws: K rotated into the workspace by the pre-pass, Q on
    load -- fa_fwd_w64 -- equals the fused one-kernel form (K rotated on
    load by fa_fwd_d128) bitwise."""
    _need_gpu()
    _announce(f"w64 rope ws {mode}")
    T, Hp, Wp = 2, 8, 8
    L = T * Hp * Wp
    B, H, Hkv = 2, 4, 2
    q, k, v = qkv(B, H, L, L, torch.bfloat16, seed=53, Hkv=Hkv, Bk=1)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    if mode == "table":
        rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
    else:
        axes = torch.from_numpy(kd_fa.axes_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)).to(DEV)
        rope = kd_fa.rope_axes(axes, (T, Hp, Wp), AXES)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    ws = torch.empty(k.numel(), dtype=k.dtype, device=DEV)
    viaws = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, workspace=ws)
    fused = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope)
    torch.cuda.synchronize()
    assert torch.equal(viaws, fused)


def test_w64_production_shape_sampled():
    """One head pair at the 31,744-token shape (496 key tiles)."""
    _need_gpu()
    _announce("w64 31744 tokens, 2 heads")
    B, H, L = 1, 2, 31744
    q, k, v = qkv(B, H, L, L, torch.bfloat16, seed=61)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg))
    assert torch.equal(out, ref)
    rows = sample_rows(B, H, L, 16, seed=62)
    assert_parity(gather_rows(out, rows, H, L), orc.fa_f64(q, k, v, rows=rows), "w64 31744")


def test_w64_ragged_production_shape_sampled():
    """A token count that is not a multiple of 64 at production length:
    768x432, 121 frames -> latent 31 x 54 x 96, patch (1, 2, 2) -> 31 x 27 x 48
    = 40,176 tokens (627 whole tiles and 48 keys), one head pair."""
    _need_gpu()
    B, H, L = 1, 2, 31 * 27 * 48
    _announce(f"w64 ragged {L} tokens, 2 heads")
    q, k, v = qkv(B, H, L, L, torch.bfloat16, seed=63)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg))
    assert torch.equal(out, ref)
    rows = sample_rows(B, H, L, 16, seed=64)
    assert_parity(gather_rows(out, rows, H, L), orc.fa_f64(q, k, v, rows=rows), "w64 ragged 40176")
