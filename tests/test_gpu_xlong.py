"""GPU checks of the persistent long-prompt kernels, which take the unmasked
calls with more than 256 keys whose K is read as stored and whose Q is
neither rotated nor normalised -- the text cross-attention of a long prompt
(src/models/crossdit.hpp:198, no mask; up to 512 prompt tokens,
src/models/qwen_tokenizer.hpp:128,183-186): fa_fwd_xlong64 (the 64-row
loop, any number of keys; F32 Q, or Q in K's type with a scale >= 0) and
fa_fwd_xlong (up to 1,024 keys: 16-bit Q with a negative scale, and scale 0
with a partial last tile).

Each case runs through the C ABI as routed and with the kernels routed out
(kd_fa_set_routing): KD_FA_ROUTE_NO_XLONG64 (fa_fwd_xlong, or fa_fwd_w64
past 1,024 keys) and KD_FA_ROUTE_NO_XLONG (the 32-row kernel fa_fwd_d128, or
fa_fwd_w64 past 896 keys); the outputs must be bitwise equal, since the
kernels perform the same arithmetic per query row.
Parity against the float64 oracle completes each case.  The shapes walk the kernel's structure: 5 to 16 key
tiles (an odd or even count, with or without a partial last tile: Lk = 257,
300, 320, 448, 512, 513, 640, 896, 1,000, 1,024), Q in F32 (four 128-byte pieces per row
brought in during a unit's first steps) or in K's type (two), workgroups
that walk one unit or many (the 31,744-row reference-form call: 31 units
each), units whose last rows lie past Lq (their O stores are then not all
issued, and the next unit waits for them), workgroups with no unit, GQA and
batch broadcast of K/V, strided Q views, negative / zero / large scales,
16-bit outputs, and F32 K/V cast by the workspace pre-pass.
"""

import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import D, assert_parity, gather_rows, qkv, randn, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _both(fn):
    """(routed output, 32-row kernel output) of fn(); the persistent 32-row
    kernel's output (KD_FA_ROUTE_NO_XLONG64) must equal the routed one."""
    with kd_fa.routing(kd_fa.ROUTE_NO_XLONG):
        ref = fn()
        torch.cuda.synchronize()
    with kd_fa.routing(kd_fa.ROUTE_NO_XLONG64):
        mid = fn()
        torch.cuda.synchronize()
    out = fn()
    torch.cuda.synchronize()
    assert torch.equal(out, mid)
    return out, ref


CASES = [
    # B, H, Hkv, Bk, Lq, Lk, kv dtype, q dtype
    (2, 4, 4, 2, 1000, 300, torch.bfloat16, torch.float32),    # 5 tiles, last partial; last unit partial
    (1, 2, 2, 1, 771, 257, torch.float16, torch.float32),      # one key in the last tile
    (2, 4, 2, 1, 2000, 320, torch.float16, torch.float16),     # 5 full tiles, GQA, batch broadcast
    (1, 3, 3, 1, 1500, 448, torch.bfloat16, torch.bfloat16),   # 7 tiles (odd)
    (2, 8, 8, 2, 4096, 512, torch.float16, torch.float32),     # the reference form, whole units
    (1, 2, 2, 1, 300, 513, torch.bfloat16, torch.float32),     # 9 tiles, one key in the last
    (1, 4, 4, 1, 5000, 896, torch.bfloat16, torch.float32),    # 14 tiles
    (1, 2, 2, 1, 1200, 1000, torch.float16, torch.float32),    # 16 tiles, the last partial
    (1, 2, 2, 1, 900, 1024, torch.bfloat16, torch.bfloat16),   # 16 tiles, fa_fwd_xlong's largest key set
    (1, 1, 1, 1, 100, 640, torch.float16, torch.float32),      # one unit in all
    (1, 5, 5, 1, 3000, 384, torch.float16, torch.float16),     # 60 units: XCD ranges of 8, the last short
    (1, 2, 1, 1, 20, 600, torch.bfloat16, torch.float32),      # fewer rows than one wave's 32
    (1, 2, 2, 1, 700, 1500, torch.float16, torch.float32),     # past 1,024 keys: F32 Q only
    (2, 2, 1, 1, 333, 2113, torch.bfloat16, torch.float32),    # 34 tiles, GQA
    (1, 3, 3, 1, 600, 1600, torch.float16, torch.float16),     # past 1,024 keys, Q in K's type
]


def _id(c):
    kt = "bf16" if c[6] == torch.bfloat16 else "f16"
    qt = {torch.float32: "q32", torch.float16: "q16", torch.bfloat16: "qbf"}[c[7]]
    return f"B{c[0]}H{c[1]}kv{c[2]}Bk{c[3]}q{c[4]}k{c[5]}{kt}{qt}"


@pytest.mark.parametrize("case", CASES, ids=_id)
def test_xlong_equals_w32(case):
    _need_gpu()
    B, H, Hkv, Bk, Lq, Lk, kt, qt = case
    _announce(f"xlong vs w32 {case}")
    q, k, v = qkv(B, H, Lq, Lk, kt, seed=Lq + 7 * Lk, Hkv=Hkv, Bk=Bk, q_dtype=qt)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg))
    assert torch.equal(out, ref)
    rows = sample_rows(B, H, Lq, 64, seed=Lk)
    assert_parity(gather_rows(out, rows, H, Lq), orc.fa_f64(q, k, v, rows=rows), f"xlong {case}")


def test_xlong_reference_form_full_size():
    """The unmasked long-prompt cross-attention as ops::attention hands it
    over: Q F32 [128, 31744, 32, 2] as a strided view of the projection
    ([D, H, L, B] permuted), K/V F16 with 512 keys; 7,936 units, 31 per
    workgroup."""
    _need_gpu()
    B, H, L, Lk = 2, 32, 31744, 512
    _announce(f"xlong reference form B={B} H={H} Lq={L} Lk={Lk}")
    qp = randn((B, L, H, D), torch.float32, 61, device=DEV)
    q = qp.permute(0, 2, 1, 3)   # (B, H, L, D) view: row stride H * D
    k = randn((B, H, Lk, D), torch.float16, 62, device=DEV)
    v = randn((B, H, Lk, D), torch.float16, 63, device=DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(q, k, v))
    assert torch.equal(out, ref)
    rows = sample_rows(B, H, L, 24, seed=64)
    qc, kc, vc = q.contiguous().cpu(), k.cpu(), v.cpu()
    assert_parity(gather_rows(out, rows, H, L), orc.fa_f64(qc, kc, vc, rows=rows), "xlong reference form")


@pytest.mark.parametrize("scale", [-0.0883883, 0.0, 2.0], ids=["neg", "zero", "large"])
@pytest.mark.parametrize("qt", [torch.float32, torch.float16], ids=["q32", "q16"])
def test_xlong_scales(scale, qt):
    """Scores that grow key by key move the running max from tile to tile;
    with scale 0 the keys of the partial tile must still get weight 0.  A
    negative scale negates Q: F32 Q in the 64-row kernel's conversion,
    16-bit Q on the 32-row kernel (the 64-row one DMAs 16-bit Q as stored)."""
    _need_gpu()
    _announce(f"xlong scale {scale} q {qt}")
    B, H, Lq, Lk = 1, 2, 700, 330
    q, k, v = qkv(B, H, Lq, Lk, torch.float16, seed=9, q_dtype=qt)
    k = (k.float() * torch.linspace(0.2, 3.0, Lk).view(1, 1, Lk, 1)).to(torch.float16)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, scale=scale))
    assert torch.equal(out, ref)
    assert_parity(gather_rows(out, np.arange(B * H * Lq), H, Lq), orc.fa_f64(q, k, v, scale=scale),
                  f"xlong scale {scale}")


@pytest.mark.parametrize("qt", [torch.float32, torch.bfloat16], ids=["q32", "q16"])
@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_xlong_sixteen_bit_output(odt, qt):
    """16-bit dst: 16 store instructions per wave and unit (the count the
    next unit's first wait leaves outstanding), equal to the F32 result
    rounded."""
    _need_gpu()
    _announce(f"xlong 16-bit dst {odt} q {qt}")
    B, H, Lq, Lk = 2, 4, 1024, 450
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=17, q_dtype=qt)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    f32 = kd_fa.flash_attn_ext(qg, kg, vg)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, out_dtype=odt))
    assert torch.equal(out, ref)
    assert torch.equal(out, f32.to(odt))


def test_xlong_f32_k_v_cast_by_the_workspace():
    """The node exactly as ops::attention receives it (Q, K, V F32), through
    kd_fa_dit_run without norm weights: the pre-pass rounds K and V to F16
    into the workspace, and this kernel reads them there -- bitwise the call
    on the rounded operands."""
    _need_gpu()
    _announce("xlong F32 K/V through the workspace")
    B, H, Lq, Lk = 2, 4, 1300, 512
    q = randn((B, H, Lq, D), torch.float32, 71)
    k = randn((B, H, Lk, D), torch.float32, 72)
    v = randn((B, H, Lk, D), torch.float32, 73)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    ws = torch.empty(2 * k.numel() * 2 + 256, dtype=torch.uint8, device=DEV)
    out = kd_fa.flash_attn_ext(qg, kg, vg, norm=kd_fa.qk_norm(None, None, 1e-6), workspace=ws)
    torch.cuda.synchronize()
    k16, v16 = k.to(torch.float16), v.to(torch.float16)
    plain = kd_fa.flash_attn_ext(qg, k16.to(DEV), v16.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    rows = sample_rows(B, H, Lq, 48, seed=74)
    assert_parity(gather_rows(out, rows, H, Lq), orc.fa_f64(q, k16, v16, rows=rows), "xlong F32 K/V")
