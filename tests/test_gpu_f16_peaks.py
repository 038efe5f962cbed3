"""F16 operands with peaked logits, unmasked: the reference's own operand
form for the DiT attention (ops.hpp:122-169: Q stays F32, K and V are cast to
F16; crossdit.hpp:198,611 pass no mask).

The unmasked kernels take the exponents against a running max that is
refreshed only when a row's weight sum over a 64-key tile leaves
[0, cap].  The weights are rounded to the operand type for the PV product,
so the cap must keep every rounded weight finite: for F16 (largest finite
value 65504) a key whose logit exceeds the running max by more than about
11 nats would otherwise round to +inf.  These cases plant such keys: for a
subset of the query rows of every wave -- not all of them -- one key beyond
the first 64-key tile gets a logit 12 to 40 nats above that row's maximum
over the first tile.  Every output must be finite and within the parity
gate of the float64 oracle, through each kernel that takes unmasked calls:
the 64-row kernel (with and without a partial last tile), the 32-row kernel
routed in its place, and the short-key kernel (Lk <= 256).
"""
import math

import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import D, HEADS, assert_parity, gather_rows, qkv, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
SCALE = 1.0 / math.sqrt(D)


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def spiked(B, H, Lq, Lk, kv_dtype, seed, q_dtype=torch.float32, every=5, rows=None, gaps=(12.0, 40.0)):
    """q, k, v (N(0, 1)) plus, for every `every`-th query row of each (b, h)
    (or the given rows), one key in tiles 1.. set to c * q_row so that the
    row's logit to it is m0 + gap nats, m0 = the row's max over keys 0..63
    and gap spread over `gaps`.  Returns (q, k, v, planted) with planted a
    list of (b, h, row, key, gap) measured on the rounded operands."""
    q, k, v = qkv(B, H, Lq, Lk, kv_dtype, seed, q_dtype=q_dtype)
    rng = np.random.default_rng(seed)
    kf = k.float().clone()
    qd = q.to(kv_dtype).float()          # Q as the kernels convert it (to K's type)
    planted = []
    sel = np.arange(0, Lq, every) if rows is None else np.asarray(rows)
    for b in range(B):
        for h in range(H):
            keys = rng.choice(np.arange(64, Lk), size=min(len(sel), Lk - 64), replace=False)
            for n, (r, j) in enumerate(zip(sel, keys)):
                gap = gaps[0] + (gaps[1] - gaps[0]) * (n % 7) / 6.0
                qr = qd[b, h, r]
                m0 = SCALE * float((kf[b, h, :64] @ qr).max())
                c = (m0 + gap) / (SCALE * float(qr @ qr))
                kf[b, h, j] = c * qr
    k = kf.to(kv_dtype)
    # the gaps as the rounded operands give them (the tests assert the range)
    kd = k.float()
    for b in range(B):
        for h in range(H):
            s = SCALE * (qd[b, h, sel] @ kd[b, h].T)
            m0 = s[:, :64].max(dim=1).values
            later = s[:, 64:].max(dim=1)
            for i, r in enumerate(sel):
                planted.append((b, h, int(r), int(later.indices[i]) + 64, float(later.values[i] - m0[i])))
    return q, k, v, planted


def _check(out, q, k, v, rows, H, Lq, what):
    got = gather_rows(out, rows, H, Lq)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    return assert_parity(got, orc.fa_f64(q, k, v, rows=rows), what)


def _planted_rows(planted, H, Lq):
    return np.array(sorted({r + Lq * (h + H * b) for b, h, r, _, _ in planted}), dtype=np.int64)


@pytest.mark.parametrize("kv", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("qt", [torch.float32, "kv"], ids=["q32", "qkv"])
def test_peaks_w64_and_w32(kv, qt):
    """Lk a multiple of 64: the 64-row kernel, and the 32-row kernel routed
    in its place -- bitwise equal, finite, within the gate."""
    _need_gpu()
    _announce(f"peaks w64/w32 kv={kv} q={qt}")
    B, H, Lq, Lk = 1, 2, 300, 1024
    q, k, v, planted = spiked(B, H, Lq, Lk, kv, seed=71, q_dtype=kv if qt == "kv" else qt)
    gaps = [g for *_, g in planted]
    assert min(gaps) >= 11.5 and max(gaps) <= 41.0, (min(gaps), max(gaps))
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out = kd_fa.flash_attn_ext(qg, kg, vg)
    with kd_fa.routing(kd_fa.ROUTE_NO_W64):
        ref = kd_fa.flash_attn_ext(qg, kg, vg)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    _check(out, q, k, v, np.arange(B * H * Lq), H, Lq, f"w64 peaks {kv}")


@pytest.mark.parametrize("Lk", [333, 1000])
def test_peaks_ragged_keys(Lk):
    """A ragged Lk: the 64-row kernel with its partial last tile in the
    loop, and the 32-row kernel routed in its place -- bitwise equal,
    finite, within the gate."""
    _need_gpu()
    _announce(f"peaks ragged Lk={Lk} f16")
    B, H, Lq = 2, 2, 257
    q, k, v, planted = spiked(B, H, Lq, Lk, torch.float16, seed=Lk)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    with kd_fa.routing(kd_fa.ROUTE_W64_SHORT):
        out = kd_fa.flash_attn_ext(qg, kg, vg)
    with kd_fa.routing(kd_fa.ROUTE_NO_W64):
        ref = kd_fa.flash_attn_ext(qg, kg, vg)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    _check(out, q, k, v, np.arange(B * H * Lq), H, Lq, f"ragged peaks Lk={Lk}")


@pytest.mark.parametrize("Lk", [77, 256])
def test_peaks_short_keys(Lk):
    """Lk <= 256: the short-key kernel, and the 32-row kernel routed in its
    place -- bitwise equal, finite, within the gate."""
    _need_gpu()
    _announce(f"peaks xres Lk={Lk} f16")
    B, H, Lq = 2, 4, 1000
    q, k, v, planted = spiked(B, H, Lq, Lk, torch.float16, seed=90 + Lk, every=3)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    out = kd_fa.flash_attn_ext(qg, kg, vg)
    with kd_fa.routing(kd_fa.ROUTE_NO_XRES):
        ref = kd_fa.flash_attn_ext(qg, kg, vg)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    _check(out, q, k, v, np.arange(B * H * Lq), H, Lq, f"xres peaks Lk={Lk}")


@pytest.mark.parametrize("Lk,route", [(77, kd_fa.ROUTE_DEFAULT), (77, kd_fa.ROUTE_NO_XRES),
                                      (1024, kd_fa.ROUTE_DEFAULT), (1024, kd_fa.ROUTE_NO_W64),
                                      (333, kd_fa.ROUTE_DEFAULT), (333, kd_fa.ROUTE_W64_SHORT)],
                         ids=["short", "short-w32-4w", "w64", "w32-8w", "ragged-w32-4w", "ragged-w64"])
def test_rows_independent_of_wave_mates(Lk, route):
    """A row's result depends on its own scores only: the query rows in a
    random order give the same rows bitwise.  The planted keys also lift
    the logits of other rows (their Q correlates with the planted row's), so
    many rows see a tile max well above their running max without their own
    weight sum leaving the cap -- the rows whose wave-mates overflow must not
    move their max because of it."""
    _need_gpu()
    _announce(f"row independence Lk={Lk} route={route}")
    B, H, Lq = 1, 2, 1000
    q, k, v, _ = spiked(B, H, Lq, Lk, torch.float16, seed=400 + Lk, every=3)
    perm = torch.from_numpy(np.random.default_rng(Lk).permutation(Lq))
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    with kd_fa.routing(route):
        out = kd_fa.flash_attn_ext(qg, kg, vg)
        outp = kd_fa.flash_attn_ext(qg[:, :, perm.to(DEV)].contiguous(), kg, vg)
    torch.cuda.synchronize()
    # dst [B, Lq, H, D]: rows along dim 1
    assert torch.equal(outp, out[:, perm.to(DEV)])


def test_peaks_with_rope_workspace_and_16bit_out():
    """The self-attention path with RoPE through the K workspace and an F16
    output: the planted peaks survive the rotation's redistribution of the
    logits only approximately, so the rows are checked, not the gaps."""
    _need_gpu()
    _announce("peaks rope ws f16 out")
    T, Hp, Wp = 4, 8, 8
    L = T * Hp * Wp
    B, H = 1, 4
    q, k, v, _ = spiked(B, H, L, L, torch.float16, seed=5, every=4)
    table = kd_fa.visual_rope_table(T, Hp, Wp, (32, 48, 48), (1.0, 2.0, 2.0), 10000.0)
    rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    ws = torch.empty(k.numel(), dtype=k.dtype, device=DEV)
    out32 = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, workspace=ws)
    out16 = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, workspace=ws, out_dtype=torch.float16)
    torch.cuda.synchronize()
    assert torch.equal(out16, out32.to(torch.float16))
    ref = orc.fa_f64(q, k, v, rope=orc.rope_table(torch.from_numpy(table)))
    got = gather_rows(out32, np.arange(B * H * L), H, L)
    assert np.isfinite(got).all()
    assert_parity(got, ref, "rope ws peaks")


def test_peaks_reference_operand_form_production_shape():
    """The reference's operand form at the production shape: Q F32
    [128, 31744, 32], K/V F16, no mask (kd_fa_run -> the 64-row kernel),
    with peaks planted for 64 rows of every head; those rows and 64 sampled
    ones per head are checked."""
    _need_gpu()
    B, H, L = 1, HEADS, 31744
    _announce(f"peaks production: Q F32 [128,{L},{H}], K/V F16")
    rng = np.random.default_rng(3)
    prow = np.sort(rng.choice(L, 64, replace=False))
    q, k, v, planted = spiked(B, H, L, L, torch.float16, seed=77, rows=prow)
    gaps = [g for *_, g in planted]
    assert min(gaps) >= 11.5, min(gaps)
    out = kd_fa.flash_attn_ext(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    rows = np.union1d(_planted_rows(planted, H, L), sample_rows(B, H, L, 64, seed=78))
    m = _check(out, q, k, v, rows, H, L, "production peaks")
    print(f"[peaks production] {m}", flush=True)


@pytest.mark.parametrize("Lk", [300, 512])
def test_cross_attention_reference_form_long_prompt(Lk):
    """The text cross-attention as the reference builds it for a long prompt
    (Lk up to 512 after the tokenizer's crop, qwen_tokenizer.hpp:129,183):
    Q F32 [128, 31744, 32], K/V F16 [128, Lk, 32], no mask; 64 sampled rows
    per head, with peaks planted for every 97th row."""
    _need_gpu()
    B, H, L = 1, HEADS, 31744
    _announce(f"cross-attn reference form: Q F32 [128,{L},{H}], K/V F16 Lk={Lk}, unmasked")
    q, k, v, planted = spiked(B, H, L, Lk, torch.float16, seed=Lk + 7, every=97)
    out = kd_fa.flash_attn_ext(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    rows = np.union1d(sample_rows(B, H, L, 64, seed=Lk), _planted_rows(planted, H, L)[::8])
    m = _check(out, q, k, v, rows, H, L, f"cross Lk={Lk}")
    print(f"[cross Lk={Lk}] {m}", flush=True)
