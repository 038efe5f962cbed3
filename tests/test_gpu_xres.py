"""GPU checks of the short-key kernel (fa_fwd_xres), which takes the calls
with Lk <= 256 whose K is read as stored and whose Q is not rotated -- the
text cross-attention (src/models/crossdit.hpp:174-200).

Each case runs twice through the C ABI: once as routed (fa_fwd_xres) and
once with the short-key kernel routed out (kd_fa_set_routing: the 32-row
kernel, fa_fwd_d128); the outputs must be
bitwise equal, since both kernels perform the same arithmetic per query row.
Parity against the float64 oracle completes each case.  The shapes walk the
kernel's structure: 1..4 key tiles held in LDS with ragged last tiles
(Lk = 1, 40, 64, 77, 130, 200, 256), query ranges shorter than the four
waves of a workgroup (Lq < 128) and ragged last blocks, GQA and batch
broadcast, masks shared by all heads or per head, tiles that are -inf for
every row (skipped) and rows that see no key, F32 Q (the reference's
operand type), the query/key RMSNorm path, negative / zero scales, and
16-bit outputs.
"""

import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import D, assert_parity, gather_rows, padding_mask, qkv, randn, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _both(fn):
    """(routed output, 32-row kernel output) of fn()."""
    with kd_fa.routing(kd_fa.ROUTE_NO_XRES):
        ref = fn()
        torch.cuda.synchronize()
    out = fn()
    torch.cuda.synchronize()
    return out, ref


def _mask(kind, B, H, Lq, Lk, seed):
    if kind is None:
        return None
    if kind == "pad":
        return padding_mask(B, Lq, Lk, [max(1, (Lk * (b + 1)) // (B + 2)) for b in range(B)], pad_rows=5)
    g = torch.Generator().manual_seed(seed)
    hm = H if kind == "rand_per_head" else 1
    m = (torch.randn((B, hm, Lq, Lk), generator=g) * 2).to(torch.float16)
    m[torch.rand((B, hm, Lq, Lk), generator=g) < 0.3] = float("-inf")
    return m


CASES = [
    # B, H, Hkv, Bk, Lq, Lk, kv dtype, q dtype, mask
    (2, 4, 4, 2, 1000, 256, torch.bfloat16, torch.bfloat16, "pad"),
    (2, 4, 4, 2, 1000, 256, torch.bfloat16, torch.bfloat16, None),
    (1, 2, 2, 1, 77, 1, torch.float16, torch.float32, None),
    (1, 3, 3, 1, 100, 40, torch.float16, torch.float32, "pad"),
    (2, 4, 2, 1, 333, 64, torch.bfloat16, torch.bfloat16, "rand"),
    (1, 2, 1, 1, 129, 77, torch.float16, torch.float16, None),
    (2, 2, 2, 2, 257, 130, torch.bfloat16, torch.float32, "rand_per_head"),
    (1, 4, 4, 1, 31, 200, torch.float16, torch.float16, "pad"),
    (2, 8, 8, 2, 4096, 200, torch.bfloat16, torch.float32, None),
    (2, 8, 8, 2, 4096, 256, torch.float16, torch.float32, "pad"),
    # the largest key set with a partial last chunk (no mask: this kernel),
    # and a masked one whose mask rows stop at Lk (the 32-row kernel)
    (1, 2, 2, 1, 70, 255, torch.bfloat16, torch.float32, None),
    (1, 2, 2, 1, 64, 129, torch.float16, torch.bfloat16, "rand"),
]


def _id(c):
    kt = "bf16" if c[6] == torch.bfloat16 else "f16"
    qt = {torch.float32: "q32", torch.float16: "q16", torch.bfloat16: "qbf"}[c[7]]
    return f"B{c[0]}H{c[1]}kv{c[2]}Bk{c[3]}q{c[4]}k{c[5]}{kt}{qt}{c[8] or 'nomask'}"


@pytest.mark.parametrize("case", CASES, ids=_id)
def test_xres_equals_w32(case):
    _need_gpu()
    B, H, Hkv, Bk, Lq, Lk, kt, qt, mk = case
    _announce(f"xres vs w32 {case}")
    q, k, v = qkv(B, H, Lq, Lk, kt, seed=Lq + 7 * Lk, Hkv=Hkv, Bk=Bk, q_dtype=qt)
    mask = _mask(mk, B, H, Lq, Lk, seed=Lq + Lk)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    mg = None if mask is None else mask.to(DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, mask=mg))
    assert torch.equal(out, ref)
    rows = sample_rows(B, H, Lq, 64, seed=Lk)
    assert_parity(gather_rows(out, rows, H, Lq), orc.fa_f64(q, k, v, mask=mask, rows=rows), f"xres {case}")


def test_xres_rows_without_keys_and_dead_tiles():
    """Every third query row is masked entirely (written as zeros); keys
    128..255 are -inf for every row (two tiles skipped)."""
    _need_gpu()
    _announce("xres rows without keys")
    B, H, Lq, Lk = 1, 2, 200, 256
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=5)
    mask = torch.zeros((1, 1, Lq, Lk), dtype=torch.float16)
    mask[:, :, :, 128:] = float("-inf")
    mask[:, :, ::3, :] = float("-inf")
    qg, kg, vg, mg = q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV)
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, mask=mg))
    assert torch.equal(out, ref)
    assert torch.count_nonzero(out[:, ::3]) == 0
    assert_parity(gather_rows(out, np.arange(B * H * Lq), H, Lq), orc.fa_f64(q, k, v, mask=mask), "xres dead")


@pytest.mark.parametrize("scale", [-0.0883883, 0.0, 2.0], ids=["neg", "zero", "large"])
def test_xres_scales(scale):
    """Scores that grow key by key move the running max from tile to tile."""
    _need_gpu()
    _announce(f"xres scale {scale}")
    B, H, Lq, Lk = 1, 2, 150, 250
    q, k, v = qkv(B, H, Lq, Lk, torch.float16, seed=9)
    k = (k.float() * torch.linspace(0.2, 3.0, Lk).view(1, 1, Lk, 1)).to(torch.float16)
    qg, kg, vg = q.to(DEV), k.to(DEV), v.to(DEV)
    for mk in (None, "pad"):
        mask = _mask(mk, B, H, Lq, Lk, seed=3)
        mg = None if mask is None else mask.to(DEV)
        out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, mask=mg, scale=scale))
        assert torch.equal(out, ref)
        assert_parity(gather_rows(out, np.arange(B * H * Lq), H, Lq),
                      orc.fa_f64(q, k, v, mask=mask, scale=scale), f"xres scale {mk}")


@pytest.mark.parametrize("use_ws", [False, True], ids=["k_on_load", "k_workspace"])
def test_xres_cross_attention_norm(use_ws):
    """kd_fa_dit_run on the cross-attention: Q normalised on load by this
    kernel (weights staged in LDS); K normalised by the workspace pre-pass
    (routed here) or on load (the 32-row kernel)."""
    _need_gpu()
    _announce(f"xres norm ws={use_ws}")
    B, H, Lq, Lk = 2, 4, 300, 256
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=13, q_dtype=torch.float32)
    wq = randn((D,), torch.float32, 14) * 0.5 + 1.0
    wk = randn((D,), torch.float32, 15) * 0.5 + 1.0
    mask = padding_mask(B, Lq, Lk, [120, 40])
    qg, kg, vg, mg = q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV)
    norm = kd_fa.qk_norm(wq.to(DEV), wk.to(DEV), EPS)
    ws = torch.empty(k.numel(), dtype=k.dtype, device=DEV) if use_ws else None
    out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, mask=mg, norm=norm, workspace=ws))
    assert torch.equal(out, ref)
    qn = torch.from_numpy(orc.rms_norm(q.float().numpy(), wq.numpy(), EPS)).to(torch.bfloat16)
    kn = torch.from_numpy(orc.rms_norm(k.float().numpy(), wk.numpy(), EPS)).to(torch.bfloat16)
    rows = sample_rows(B, H, Lq, 48, seed=16)
    assert_parity(gather_rows(out, rows, H, Lq), orc.fa_f64(qn, kn, v, mask=mask, rows=rows), "xres norm")


def test_xres_sixteen_bit_output():
    _need_gpu()
    _announce("xres 16-bit dst")
    B, H, Lq, Lk = 2, 2, 130, 120
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=17)
    mask = _mask("pad", B, H, Lq, Lk, seed=0)
    qg, kg, vg, mg = q.to(DEV), k.to(DEV), v.to(DEV), mask.to(DEV)
    f32 = kd_fa.flash_attn_ext(qg, kg, vg, mask=mg)
    for odt in (torch.bfloat16, torch.float16):
        out, ref = _both(lambda: kd_fa.flash_attn_ext(qg, kg, vg, mask=mg, out_dtype=odt))
        assert torch.equal(out, ref)
        assert torch.equal(out, f32.to(odt))
