"""GPU checks of kd_fa_dit_run (RMSNorm of the Q and K head rows, then RoPE,
then the attention node: src/models/crossdit.hpp:134-150, 191-199) and of
16-bit outputs, through the C ABI.

The definition is checked bitwise: kd_fa_dit_run on (q, k, v) equals
kd_fa_run on q' = round(rot(rms(q) * wq)), k' = round(rot(rms(k) * wk)),
with q', k' computed by the oracle's restatements of ops::rms_norm and
rope::apply; the workspace and on-load forms agree bitwise, and the
workspace holds the oracle's k'.  Parity against the float64 oracle on the
transformed operands completes each case.
"""
import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import AXES, D, SCALE_FACTOR, THETA, assert_parity, gather_rows, padding_mask, qkv, randn, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _weights(seed):
    g = torch.Generator().manual_seed(seed)
    wq = (torch.randn(D, generator=g) * 0.3 + 1.0).float()
    wk = (torch.randn(D, generator=g) * 0.3 + 1.0).float()
    return wq, wk


def _norm(x, w):
    """ops::rms_norm by the oracle over the head rows of x (B, H, L, D), F32."""
    return torch.from_numpy(orc.rms_norm(x.float().numpy(), w.numpy(), EPS))


def _rot(x, table, dtype):
    """rope::apply in F32 by the oracle, rounded to dtype: x (B, H, L, D)."""
    xb = x.float().permute(0, 2, 1, 3).contiguous().numpy()
    r = orc.rope_apply(xb, table[: x.shape[2]])
    return torch.from_numpy(r).permute(0, 2, 1, 3).contiguous().to(dtype)


def _plain(q, k, v, mask=None):
    out = kd_fa.flash_attn_ext(q.to(DEV), k.to(DEV), v.to(DEV), mask=None if mask is None else mask.to(DEV))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_self_attention_norm_rope(dt):
    """RMSNorm + 3-D RoPE + attention, GQA and batch broadcast, partial tile."""
    _need_gpu()
    _announce(f"dit self-attention norm+rope {dt}")
    T, Hp, Wp = 3, 5, 7
    L = T * Hp * Wp
    B, H, Hkv = 2, 4, 2
    q, k, v = qkv(B, H, L, L, dt, seed=71, Hkv=Hkv, Bk=1, q_dtype=torch.float32)
    wq, wk = _weights(72)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    tab_g = torch.from_numpy(table).to(DEV)
    norm = kd_fa.qk_norm(wq.to(DEV), wk.to(DEV), EPS)
    rope = kd_fa.rope_table(tab_g)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    fused = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, norm=norm)
    ws = torch.empty(k.numel(), dtype=dt, device=DEV)
    viaws = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, norm=norm, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(fused, viaws)
    q2 = _rot(_norm(q, wq), table, dt)
    k2 = _rot(_norm(k, wk), table, dt)
    assert torch.equal(ws.view(k.shape).cpu(), k2)
    assert torch.equal(fused, _plain(q2, k2, v))
    ref = orc.fa_f64(q2, k2, v)
    assert_parity(gather_rows(fused, np.arange(B * H * L), H, L), ref, "dit self-attention")


@pytest.mark.parametrize("L", [77, 256, 300])
def test_text_block_self_attention(L):
    """TextBlock self-attention (src/models/crossdit.hpp:234-275): the same
    DiTSelfAttention with the 1-D text RoPE table (rope::compute_text_rope,
    src/rope.hpp:36-49, built at crossdit.hpp:562) over the prompt tokens,
    CFG batch 2, 32 heads; fused and workspace forms bitwise equal, both equal
    to the plain node on the oracle-transformed operands."""
    _need_gpu()
    _announce(f"text block self-attention L={L}")
    B, H = 2, 32
    q, k, v = qkv(B, H, L, L, torch.bfloat16, seed=L, q_dtype=torch.float32)
    wq, wk = _weights(L + 1)
    table = kd_fa.text_rope_table(L, D)
    norm = kd_fa.qk_norm(wq.to(DEV), wk.to(DEV), EPS)
    rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    fused = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, norm=norm)
    ws = torch.empty(k.numel(), dtype=torch.bfloat16, device=DEV)
    viaws = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, norm=norm, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(fused, viaws)
    q2 = _rot(_norm(q, wq), table, torch.bfloat16)
    k2 = _rot(_norm(k, wk), table, torch.bfloat16)
    assert torch.equal(fused, _plain(q2, k2, v))
    rows = sample_rows(B, H, L, 32, seed=L + 2)
    assert_parity(gather_rows(fused, rows, H, L), orc.fa_f64(q2, k2, v, rows=rows), "text block")


def test_self_attention_f32_k_through_workspace():
    """K given as the F32 projection output: normalised and rotated in F32,
    rounded once into the workspace (the reference's cast after RoPE)."""
    _need_gpu()
    _announce("dit self-attention F32 K via workspace")
    T, Hp, Wp = 2, 6, 8
    L = T * Hp * Wp
    B, H = 1, 4
    q = randn((B, H, L, D), torch.float32, 81)
    k = randn((B, H, L, D), torch.float32, 82) * 3.0
    v = randn((B, H, L, D), torch.bfloat16, 83)
    wq, wk = _weights(84)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
    norm = kd_fa.qk_norm(wq.to(DEV), wk.to(DEV), EPS)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    ws = torch.empty(k.numel(), dtype=torch.bfloat16, device=DEV)
    out = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, norm=norm, workspace=ws)
    torch.cuda.synchronize()
    k2 = _rot(_norm(k, wk), table, torch.bfloat16)
    q2 = _rot(_norm(q, wq), table, torch.bfloat16)
    assert torch.equal(ws.view(k.shape).cpu(), k2)
    assert torch.equal(out, _plain(q2, k2, v))
    # an F32 K needs the workspace (the on-load path works in the operand type):
    # without one the call names the missing buffer
    with pytest.raises(kd_fa.KdFaError) as e:
        kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, norm=norm)
    assert e.value.status == kd_fa.ERR_NULL
    assert_parity(gather_rows(out, np.arange(B * H * L), H, L), orc.fa_f64(q2, k2, v), "dit F32 K")


@pytest.mark.parametrize("use_ws", [False, True])
def test_cross_attention_norm_mask(use_ws):
    """Text cross-attention: RMSNorm on Q and K, no RoPE, padding mask."""
    _need_gpu()
    _announce(f"dit cross-attention norm, workspace={use_ws}")
    B, H, Lq, Lk = 2, 4, 200, 77
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=91, q_dtype=torch.float32)
    m = padding_mask(B, Lq, Lk, (77, 30))
    wq, wk = _weights(92)
    norm = kd_fa.qk_norm(wq.to(DEV), wk.to(DEV), EPS)
    qg, kg, vg, mg = q.to(DEV), k.to(DEV), v.to(DEV), m.to(DEV)
    ws = torch.empty(k.numel(), dtype=torch.bfloat16, device=DEV) if use_ws else None
    out = kd_fa.flash_attn_ext(qg, kg, vg, mask=mg, norm=norm, workspace=ws)
    torch.cuda.synchronize()
    q2 = _norm(q, wq).to(torch.bfloat16)
    k2 = _norm(k, wk).to(torch.bfloat16)
    if use_ws:
        assert torch.equal(ws.view(k.shape).cpu(), k2)
    assert torch.equal(out, _plain(q2, k2, v, m))
    assert_parity(gather_rows(out, np.arange(B * H * Lq), H, Lq), orc.fa_f64(q2, k2, v, mask=m), "dit cross")


@pytest.mark.parametrize("q_dtype,masked", [(torch.bfloat16, True), (torch.bfloat16, False),
                                             (torch.float32, True), (torch.float32, False)])
def test_cross_attention_norm_several_blocks_per_wave(q_dtype, masked):
    """Short key set with the query norm, 256 (b, h) pairs and 10 query
    blocks of 32 rows each: one range per pair, so waves 0 and 1 of every
    workgroup run a second block after storing their first one's O (the
    query-norm weights are reloaded between the two).  Bitwise equal to the
    node on the pre-normalised operands, and the oracle on sampled rows."""
    _need_gpu()
    _announce(f"dit cross-attention norm, 2 blocks per wave, q {q_dtype}, mask {masked}")
    B, H, Lq, Lk = 1, 256, 300, 77
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=93, q_dtype=q_dtype)
    m = padding_mask(B, Lq, Lk, (61,)) if masked else None
    wq, wk = _weights(94)
    norm = kd_fa.qk_norm(wq.to(DEV), wk.to(DEV), EPS)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    mg = None if m is None else m.to(DEV)
    ws = torch.empty(k.numel(), dtype=torch.bfloat16, device=DEV)
    out = kd_fa.flash_attn_ext(qg, kg, vg, mask=mg, norm=norm, workspace=ws)
    o16 = kd_fa.flash_attn_ext(qg, kg, vg, mask=mg, norm=norm, workspace=ws, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    q2 = _norm(q, wq).to(torch.bfloat16)
    k2 = _norm(k, wk).to(torch.bfloat16)
    assert torch.equal(out, _plain(q2, k2, v, m))
    assert torch.equal(o16, out.to(torch.bfloat16))
    rows = sample_rows(B, H, Lq, 2, 95)   # row 299 of each head: block 9, wave 1's second
    assert_parity(gather_rows(out, rows, H, Lq), orc.fa_f64(q2, k2, v, mask=m, rows=rows), "dit cross, 2 blocks per wave")


def test_norm_of_one_side_only():
    """A NULL weight leaves that side as it is."""
    _need_gpu()
    _announce("dit norm of Q only")
    B, H, L = 1, 2, 70
    q, k, v = qkv(B, H, L, L, torch.float16, seed=95, q_dtype=torch.float32)
    wq, _ = _weights(96)
    out = kd_fa.flash_attn_ext(q.to(DEV), k.to(DEV), v.to(DEV), norm=kd_fa.qk_norm(wq.to(DEV), None, EPS))
    torch.cuda.synchronize()
    assert torch.equal(out, _plain(_norm(q, wq).to(torch.float16), k, v))


@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float16])
def test_sixteen_bit_output_is_rounded_f32(odt):
    """dst BF16 / F16: the F32 result rounded to nearest even, bitwise."""
    _need_gpu()
    _announce(f"16-bit dst {odt}")
    B, H, Lq, Lk = 2, 3, 150, 90
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=97)
    m = padding_mask(B, Lq, Lk, (90, 41))
    for mask in (None, m):
        qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
        mg = None if mask is None else mask.to(DEV)
        f32 = kd_fa.flash_attn_ext(qg, kg, vg, mask=mg)
        o16 = kd_fa.flash_attn_ext(qg, kg, vg, mask=mg, out_dtype=odt)
        torch.cuda.synchronize()
        assert o16.dtype == odt
        assert torch.equal(o16, f32.to(odt))
