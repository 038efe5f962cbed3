"""GPU parity of the D = 512 node: the single-head attention of the 2-D VAE's
attention block (src/models/vae.hpp:60-101 -> ops::attention with one head,
D = channels = 512; Q F32, K/V F16 as ops.hpp:122-169 prepares them).

Parity is against the oracle's float64 textbook attention on the same rounded
operands (max-abs <= 2e-2 and cosine >= 0.9995), every row for small cases
and sampled rows at the 64x64-latent size.  The shapes walk the kernel's
32-key tiles (Lk < 32, ragged last tile), its 32-row query tiles (ragged
Lq), GQA and batch broadcast, negative / zero / large scales, and 16-bit
outputs (the F32 result rounded, bitwise).
"""
import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import assert_parity, gather_rows, randn, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = 512


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _qkv(B, H, Lq, Lk, kt, seed, Hkv=None, Bk=None, qt=torch.float32):
    Hkv = H if Hkv is None else Hkv
    Bk = B if Bk is None else Bk
    q = randn((B, H, Lq, D), qt, seed)
    k = randn((Bk, Hkv, Lk, D), kt, seed + 1)
    v = randn((Bk, Hkv, Lk, D), kt, seed + 2)
    return q, k, v


def _run(q, k, v, **kw):
    out = kd_fa.flash_attn_ext(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    torch.cuda.synchronize()
    return out


CASES = [
    # B, H, Hkv, Bk, Lq, Lk, K/V type
    (1, 1, 1, 1, 1024, 1024, torch.float16),   # 32x32 latent
    (1, 1, 1, 1, 77, 45, torch.bfloat16),
    (1, 1, 1, 1, 40, 5, torch.float16),
    (2, 2, 1, 1, 100, 200, torch.float16),
    (2, 1, 1, 2, 33, 96, torch.bfloat16),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}kv{c[2]}q{c[4]}k{c[5]}{'bf16' if c[6] == torch.bfloat16 else 'f16'}")
def test_d512_parity(case):
    _need_gpu()
    B, H, Hkv, Bk, Lq, Lk, kt = case
    _announce(f"d512 {case}")
    q, k, v = _qkv(B, H, Lq, Lk, kt, seed=Lq + 3 * Lk, Hkv=Hkv, Bk=Bk)
    scale = D ** -0.5
    out = _run(q, k, v, scale=scale)
    ref = orc.fa_f64(q, k, v, scale=scale)
    assert_parity(gather_rows(out, np.arange(B * H * Lq), H, Lq), ref, f"d512 {case}")
    again = _run(q, k, v, scale=scale)
    assert torch.equal(out, again)


@pytest.mark.parametrize("scale", [-0.0441941738, 0.0, 0.25], ids=["neg", "zero", "large"])
def test_d512_scales(scale):
    _need_gpu()
    _announce(f"d512 scale {scale}")
    q, k, v = _qkv(1, 1, 96, 130, torch.float16, seed=11)
    out = _run(q, k, v, scale=scale)
    assert_parity(gather_rows(out, np.arange(96), 1, 96), orc.fa_f64(q, k, v, scale=scale), "d512 scale")


def test_d512_sixteen_bit_output():
    _need_gpu()
    _announce("d512 16-bit dst")
    q, k, v = _qkv(1, 1, 70, 90, torch.bfloat16, seed=21)
    f32 = _run(q, k, v, scale=D ** -0.5)
    for odt in (torch.bfloat16, torch.float16):
        o16 = _run(q, k, v, scale=D ** -0.5, out_dtype=odt)
        assert torch.equal(o16, f32.to(odt))


def test_d512_vae_64x64_sampled():
    """The mid-block attention at a 64x64 latent (512-pixel images): 4,096
    tokens, sampled query rows."""
    _need_gpu()
    _announce("d512 4096 tokens")
    L = 4096
    q, k, v = _qkv(1, 1, L, L, torch.float16, seed=31)
    out = _run(q, k, v, scale=D ** -0.5)
    rows = sample_rows(1, 1, L, 64, seed=32)
    assert_parity(gather_rows(out, rows, 1, L), orc.fa_f64(q, k, v, scale=D ** -0.5, rows=rows), "d512 4096")


def _run_rows32(q, k, v, **kw):
    """The same call with 32 query rows per workgroup forced."""
    with kd_fa.routing(kd_fa.ROUTE_D512_R1):
        return _run(q, k, v, **kw)


ROWS64_CASES = [
    # B, H, Hkv, Bk, Lq, Lk, K/V type: >= 256 workgroups of 64 rows, so the
    # 64-row kernel runs; ragged query blocks (Lq % 64) and key tiles
    (4, 64, 64, 4, 100, 45, torch.float16),
    (2, 128, 32, 1, 64, 97, torch.bfloat16),
    (1, 256, 256, 1, 33, 32, torch.float16),
]


@pytest.mark.parametrize("case", ROWS64_CASES, ids=lambda c: f"B{c[0]}H{c[1]}kv{c[2]}q{c[4]}k{c[5]}")
def test_d512_64_rows_equal_32_rows(case):
    """Two 32-row blocks per wave (the key stream shared by 64 rows) give
    bitwise the 32-row kernel's result; both agree with the oracle."""
    _need_gpu()
    B, H, Hkv, Bk, Lq, Lk, kt = case
    _announce(f"d512 64 rows {case}")
    q, k, v = _qkv(B, H, Lq, Lk, kt, seed=Lq + Lk + H, Hkv=Hkv, Bk=Bk)
    scale = D ** -0.5
    out = _run(q, k, v, scale=scale)
    assert torch.equal(out, _run_rows32(q, k, v, scale=scale))
    rows = sample_rows(B, H, Lq, 48, seed=Lk)
    assert_parity(gather_rows(out, rows, H, Lq), orc.fa_f64(q, k, v, scale=scale, rows=rows), f"d512 64 rows {case}")


def test_d512_vae_128x128_sampled():
    """The mid-block attention at a 128x128 latent (1024-pixel images):
    16,384 tokens, one head -- 256 workgroups of 64 rows; bitwise the 32-row
    kernel's result, sampled rows against the oracle."""
    _need_gpu()
    _announce("d512 16384 tokens")
    L = 16384
    q, k, v = _qkv(1, 1, L, L, torch.float16, seed=41)
    out = _run(q, k, v, scale=D ** -0.5)
    assert torch.equal(out, _run_rows32(q, k, v, scale=D ** -0.5))
    rows = sample_rows(1, 1, L, 32, seed=42)
    assert_parity(gather_rows(out, rows, 1, L), orc.fa_f64(q, k, v, scale=D ** -0.5, rows=rows), "d512 16384")
