"""GPU checks of F32 K and V in the workspace forms: the projection outputs as
ops::attention receives them (src/core/ops.hpp:122-169: Q F32, K and V F32
cast by ggml_cast to F16 before the node), with the cast done by the
pre-pass that writes the transformed K (kd_fa_dit_run, kd_fa_rope_run_ws).

The definition is checked bitwise: the call with F32 K / V equals the same
call on K and V rounded to the operand type by the oracle's codecs
(round-to-nearest-even, all 65,536 patterns pinned in the CPU suite); the
workspace holds exactly those rounded values; and the oracle gate (float64
textbook attention on the rounded operands) holds at the 1,280-token shape
on every row and at the 31,744-token shape on 64 sampled rows per (b, h).
"""
import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import AXES, D, HEADS, SCALE_FACTOR, THETA, assert_parity, gather_rows, metrics, randn, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6
SCALE = 1.0 / D ** 0.5


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _round(x, dtype):
    """F32 tensor rounded to dtype by the oracle's codec (RNE)."""
    a = np.ascontiguousarray(x.detach().to("cpu", torch.float32).numpy())
    bits = orc.f32_to_bf16_bits(a) if dtype == torch.bfloat16 else orc.f32_to_f16_bits(a)
    return torch.from_numpy(np.asarray(bits, dtype=np.uint16).view(np.int16)).view(dtype)


def _norm(x, w):
    return torch.from_numpy(orc.rms_norm(x.float().numpy(), w.numpy(), EPS))


def _rot_f32(x, table):
    """rope::apply in F32 by the oracle over x (B, H, L, D)."""
    xb = x.float().permute(0, 2, 1, 3).contiguous().numpy()
    r = orc.rope_apply(xb, table[: x.shape[2]])
    return torch.from_numpy(r).permute(0, 2, 1, 3).contiguous()


def _dev_rand(shape, seed, dtype=torch.float32):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=g, device=DEV, dtype=torch.float32).to(dtype)


@pytest.mark.parametrize("kv", ["k32_v32", "k16_v32", "k32_v16"])
@pytest.mark.parametrize("cast", [torch.float16, torch.bfloat16])
def test_cast_bitwise_equals_rounded_operands(kv, cast):
    """RMSNorm + 3-D RoPE + attention from F32 projections, GQA and batch
    broadcast, ragged tiles: the output equals the same call on the
    oracle-rounded K and V, and the workspace holds them."""
    _need_gpu()
    _announce(f"F32 operands {kv}, cast {cast}")
    T, Hp, Wp = 3, 5, 7
    L = T * Hp * Wp
    B, H, Hkv = 2, 4, 2
    q = randn((B, H, L, D), torch.float32, 501)
    k32 = randn((1, Hkv, L, D), torch.float32, 502) * 2.0
    v32 = randn((1, Hkv, L, D), torch.float32, 503)
    g = torch.Generator().manual_seed(504)
    wq = (torch.randn(D, generator=g) * 0.3 + 1.0).float()
    wk = (torch.randn(D, generator=g) * 0.3 + 1.0).float()
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
    norm = kd_fa.qk_norm(wq.to(DEV), wk.to(DEV), EPS)
    k_in = k32 if kv.startswith("k32") else _round(k32, cast)
    v_in = v32 if kv.endswith("v32") else _round(v32, cast)
    ct = kd_fa.TYPE_BF16 if cast == torch.bfloat16 else kd_fa.TYPE_F16
    qg, kg, vg = q.to(DEV), k_in.to(DEV), v_in.to(DEV)
    out = torch.full((B, L, H, D), float("nan"), device=DEV)
    desc = kd_fa.make_desc(qg, kg, vg, None, out, SCALE, cast_type=ct)
    ws = torch.empty(kd_fa.workspace_size_full(desc, rope, norm), dtype=torch.uint8, device=DEV)
    assert kd_fa.run_desc(desc, rope, None, ws, norm) == kd_fa.OK
    torch.cuda.synchronize()
    # the operands as ggml_cast would hand them over: K normalised and
    # rotated in F32, then rounded; V rounded
    k2 = _round(_rot_f32(_norm(k_in.float(), wk), table), cast)
    v2 = _round(v_in.float(), cast)
    kb = k2.numel() * 2
    assert torch.equal(ws[:kb].view(cast).view(k2.shape).cpu(), k2)
    if kv.endswith("v32"):
        v_off = (kb + 255) // 256 * 256
        assert torch.equal(ws[v_off:v_off + v2.numel() * 2].view(cast).view(v2.shape).cpu(), v2)
    # the node on the final operands
    plain = kd_fa.flash_attn_ext(_round(_rot_f32(_norm(q, wq), table), cast).to(DEV), k2.to(DEV), v2.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    if kv.endswith("v32"):
        # the same call with V already rounded by the oracle (16-bit V)
        out16 = torch.full_like(out, float("nan"))
        d16 = kd_fa.make_desc(qg, kg, v2.to(DEV), None, out16, SCALE, cast_type=ct)
        ws16 = torch.empty(max(kd_fa.workspace_size_full(d16, rope, norm), 16), dtype=torch.uint8, device=DEV)
        assert kd_fa.run_desc(d16, rope, None, ws16, norm) == kd_fa.OK
        torch.cuda.synchronize()
        assert torch.equal(out, out16)
    q2 = _round(_rot_f32(_norm(q, wq), table), cast)
    assert_parity(gather_rows(out, np.arange(B * H * L), H, L), orc.fa_f64(q2, k2, v2), f"F32 {kv} {cast}")


def test_cast_k_and_v_with_different_heads():
    """K with 2 heads and V with 4 (each a divisor of H = 4): the pre-pass
    runs as two launches, K's then V's; same definition."""
    _need_gpu()
    _announce("F32 K (2 heads) and V (4 heads), two pre-pass launches")
    B, H, L = 1, 4, 130
    q = randn((B, H, L, D), torch.float32, 511)
    k32 = randn((B, 2, L, D), torch.float32, 512)
    v32 = randn((B, 4, L, D), torch.float32, 513)
    out = kd_fa.flash_attn_ext(q.to(DEV), k32.to(DEV), v32.to(DEV), norm=kd_fa.qk_norm(None, None, EPS),
                               workspace=torch.empty(2 * 6 * L * D * 2 + 256, dtype=torch.uint8, device=DEV))
    torch.cuda.synchronize()
    k2, v2 = _round(k32, torch.float16), _round(v32, torch.float16)
    plain = kd_fa.flash_attn_ext(q.to(DEV), k2.to(DEV), v2.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    assert_parity(gather_rows(out, np.arange(B * H * L), H, L), orc.fa_f64(_round(q, torch.float16), k2, v2),
                  "F32 K/V, different heads")


def test_c1_all_f32_every_row():
    """The 1,280-token self-attention in the form ops::attention receives it
    after rope::apply: Q, K, V F32 [128, 1280, 32, 1], RoPE grid 5x16x16 fused,
    K and V cast to F16 (ggml_cast) by the pre-pass: bitwise the call on
    the oracle-rounded V, and the oracle gate on every row."""
    _need_gpu()
    _announce("C1 all-F32 via kd_fa_rope_run_ws: [128,1280,32,1], cast F16, every row")
    T, Hp, Wp = 5, 16, 16
    L = T * Hp * Wp
    q = _dev_rand((1, HEADS, L, D), 1)
    k = _dev_rand((1, HEADS, L, D), 1001)
    v = _dev_rand((1, HEADS, L, D), 2001)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
    out = torch.empty((1, L, HEADS, D), device=DEV)
    d = kd_fa.make_desc(q, k, v, None, out, SCALE)
    ws = torch.empty(kd_fa.workspace_size(d), dtype=torch.uint8, device=DEV)
    assert kd_fa.run_desc(d, rope, None, ws) == kd_fa.OK
    # the same with V already rounded by the oracle (16-bit V): bitwise
    v16 = _round(v, torch.float16).to(DEV)
    out2 = torch.empty_like(out)
    d2 = kd_fa.make_desc(q, k, v16, None, out2, SCALE)
    ws2 = torch.empty(kd_fa.workspace_size(d2), dtype=torch.uint8, device=DEV)
    assert kd_fa.run_desc(d2, rope, None, ws2) == kd_fa.OK
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    qc, kc = q.cpu(), k.cpu()
    k2 = _round(_rot_f32(kc, table), torch.float16)
    q2 = _round(_rot_f32(qc, table), torch.float16)
    v2 = v16.cpu()
    ref = orc.fa_f64(q2, k2, v2)
    m = assert_parity(gather_rows(out, np.arange(HEADS * L), HEADS, L), ref, "C1 all-F32")
    print(f"[C1 all-F32] vs f64: {m}", flush=True)
    ggml, _ = orc.fa_ggml(q2, k2, v2, f16_vacc=True)
    mg = metrics(out.cpu().double().numpy(), ggml.double().numpy())
    print(f"[C1 all-F32] vs ggml restatement: {mg}", flush=True)
    assert mg["max_abs"] <= 2e-2 and mg["cos"] >= 0.9995, mg


def test_c3_all_f32_sampled():
    """The 31,744-token self-attention from F32 operands: Q, K, V F32
    [128, 31744, 32, 2], RoPE grid 31x32x32, cast to F16; 64 sampled rows per
    (b, h) against the oracle, and the cast V in the workspace on sampled
    heads."""
    _need_gpu()
    _announce("C3 all-F32 via kd_fa_rope_run_ws: [128,31744,32,2], cast F16, 64 rows per (b,h)")
    B, T = 2, 31
    L = T * 32 * 32
    q = _dev_rand((B, HEADS, L, D), 3)
    k = _dev_rand((B, HEADS, L, D), 1003)
    v = _dev_rand((B, HEADS, L, D), 2003)
    table = kd_fa.visual_rope_table(T, 32, 32, AXES, SCALE_FACTOR, THETA)
    rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
    out = torch.empty((B, L, HEADS, D), device=DEV)
    d = kd_fa.make_desc(q, k, v, None, out, SCALE)
    ws = torch.empty(kd_fa.workspace_size(d), dtype=torch.uint8, device=DEV)
    assert kd_fa.run_desc(d, rope, None, ws) == kd_fa.OK
    torch.cuda.synchronize()
    kb = B * HEADS * L * D * 2
    v_ws = ws[kb:kb + kb].view(torch.float16).view(B, HEADS, L, D)
    for b, h in ((0, 0), (1, 31), (0, 17)):
        assert torch.equal(v_ws[b, h].cpu(), _round(v[b, h], torch.float16)), (b, h)
    rows = sample_rows(B, HEADS, L, 64, seed=3)
    q2 = _round(_rot_f32(q.cpu(), table), torch.float16)
    k2 = _round(_rot_f32(k.cpu(), table), torch.float16)
    v2 = _round(v.cpu(), torch.float16)
    ref = orc.fa_f64(q2, k2, v2, rows=rows)
    m = assert_parity(gather_rows(out, rows, HEADS, L), ref, "C3 all-F32")
    print(f"[C3 all-F32] {m}", flush=True)


@pytest.mark.parametrize("cast", [torch.float16, torch.bfloat16])
def test_masked_cross_attention_from_f32_projections(cast):
    """The cross-attention of DiTCrossAttention from its projections: Q, K, V
    F32, the key norm, a padding mask, 256 keys and 2,048 query rows per head
    (65,536 in all, so the mask summary runs): the workspace holds K, then V,
    then the summary, and the result is the call on the oracle-rounded
    operands, bitwise, and within the oracle gate on every row."""
    _need_gpu()
    _announce(f"masked cross-attention from F32 projections, cast {cast}")
    B, H, Lq, Lk = 2, 16, 2048, 256
    q = randn((B, H, Lq, D), torch.float32, 521)
    k = randn((B, H, Lk, D), torch.float32, 522) * 1.5
    v = randn((B, H, Lk, D), torch.float32, 523)
    from fa_common import padding_mask
    m = padding_mask(B, Lq, Lk, (200, 37))
    g = torch.Generator().manual_seed(524)
    wq = (torch.randn(D, generator=g) * 0.3 + 1.0).float()
    wk = (torch.randn(D, generator=g) * 0.3 + 1.0).float()
    norm = kd_fa.qk_norm(wq.to(DEV), wk.to(DEV), EPS)
    ct = kd_fa.TYPE_BF16 if cast == torch.bfloat16 else kd_fa.TYPE_F16
    qg, kg, vg, mg = q.to(DEV), k.to(DEV), v.to(DEV), m.to(DEV)
    out = torch.full((B, Lq, H, D), float("nan"), device=DEV)
    d = kd_fa.make_desc(qg, kg, vg, mg, out, SCALE, cast_type=ct)
    n_ws = kd_fa.workspace_size_full(d, None, norm)
    kb = B * H * Lk * D * 2
    assert n_ws == 2 * kb + 4 * B * ((Lq + 31) // 32)      # K, V, then one word per batch and 32 rows
    ws = torch.full((n_ws,), 0xAB, dtype=torch.uint8, device=DEV)
    assert kd_fa.run_desc(d, None, None, ws, norm) == kd_fa.OK
    torch.cuda.synchronize()
    k2 = _round(_norm(k, wk), cast)
    v2 = _round(v, cast)
    assert torch.equal(ws[:kb].view(cast).view(k2.shape).cpu(), k2)
    assert torch.equal(ws[kb:2 * kb].view(cast).view(v2.shape).cpu(), v2)
    q2 = _round(_norm(q, wq), cast)
    plain = kd_fa.flash_attn_ext(q2.to(DEV), k2.to(DEV), v2.to(DEV), mask=mg)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    rows = np.arange(B * H * Lq)
    assert_parity(gather_rows(out, rows, H, Lq), orc.fa_f64(q2, k2, v2, mask=m), f"masked cross F32 {cast}")
