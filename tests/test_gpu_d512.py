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


def _split_ranges(Lq, Lk, H, B):
    """(ranges, keys per range) of the key split kd_fa_run_ws takes for a
    D = 512 node: fewer than 512 blocks of 32 query rows (two workgroups per
    CU) and at least four key tiles, at most 8 ranges of whole 32-key tiles,
    at least two."""
    nb = (Lq + 31) // 32 * H * B
    tiles = (Lk + 31) // 32
    if nb >= 512 or tiles < 4:
        return 1, 0
    S = min(8, 512 // nb, tiles)
    if S < 2:
        return 1, 0
    per = (tiles + S - 1) // S
    S = (tiles + per - 1) // per
    return (S, per * 32) if S >= 2 else (1, 0)


SPLIT_CASES = [
    # B, H, Hkv, Bk, Lq, Lk, K/V type, dst type
    (1, 1, 1, 1, 4096, 4096, torch.float16, torch.float32),    # 64x64 latent: four key ranges
    (1, 1, 1, 1, 8192, 2048, torch.bfloat16, torch.float32),   # 256 blocks: two ranges
    (1, 1, 1, 1, 1024, 1024, torch.float16, torch.float32),    # 32x32 latent: eight ranges
    (1, 1, 1, 1, 300, 1000, torch.bfloat16, torch.float32),    # ragged last tile and range
    (2, 2, 1, 1, 100, 200, torch.float16, torch.bfloat16),     # GQA and batch broadcast, 16-bit dst
    (1, 1, 1, 1, 64, 130, torch.float16, torch.float32),       # five tiles: five ranges of one tile
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=lambda c: f"B{c[0]}H{c[1]}q{c[4]}k{c[5]}{str(c[7])[-4:]}")
def test_d512_key_split(case):
    """kd_fa_run_ws on a D = 512 node with few query rows: the keys of every
    row are split into ranges computed side by side and merged through the
    workspace.  Parity against the oracle, determinism, the workspace size
    rule, and with the split routed out the call is bitwise kd_fa_run."""
    _need_gpu()
    B, H, Hkv, Bk, Lq, Lk, kt, ot = case
    _announce(f"d512 key split {case}")
    q, k, v = _qkv(B, H, Lq, Lk, kt, seed=Lq + Lk + 7, Hkv=Hkv, Bk=Bk)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    scale = D ** -0.5
    outs = [torch.empty((B, Lq, H, D), dtype=ot, device=DEV) for _ in range(4)]
    descs = [kd_fa.make_desc(q, k, v, None, o, scale) for o in outs]
    S, _ = _split_ranges(Lq, Lk, H, B)
    need = kd_fa.workspace_size_full(descs[0])
    assert S >= 2 and need == S * B * H * Lq * (D * 4 + 8)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV).fill_(0x7F)
    assert kd_fa.run_desc(descs[0], workspace=ws) == kd_fa.OK
    assert kd_fa.run_desc(descs[1], workspace=ws) == kd_fa.OK
    assert kd_fa.run_desc(descs[2]) == kd_fa.OK
    with kd_fa.routing(kd_fa.ROUTE_NO_SPLIT):
        assert kd_fa.run_desc(descs[3], workspace=ws) == kd_fa.OK
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(outs[2], outs[3])
    # each range rounds its weights to the operand type against its own
    # running max (the unsplit call: against the row's), and the ranges'
    # sums are merged in another order: the difference is that rounding
    diff = (outs[0].float() - outs[2].float()).abs().max().item()
    tol = 1e-2 if ot != torch.float32 else (2e-3 if kt == torch.bfloat16 else 2e-4)
    assert diff <= tol, diff
    rows = np.arange(B * H * Lq) if Lq <= 1024 else sample_rows(B, H, Lq, 64, seed=5)
    ref = orc.fa_f64(q.cpu(), k.cpu(), v.cpu(), scale=scale, rows=rows)
    assert_parity(gather_rows(outs[0].float(), rows, H, Lq), ref, f"d512 key split {case}")


def test_d512_key_split_in_static_scratch():
    """kd_fa_dit_run_static on the VAE node keeps the key split's partial
    results in the library's static scratch: bitwise kd_fa_run_ws with a
    caller workspace."""
    _need_gpu()
    _announce("d512 key split in the static scratch")
    L = 2048
    q, k, v = _qkv(1, 1, L, L, torch.float16, seed=51)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = [torch.empty((1, L, 1, D), dtype=torch.float32, device=DEV) for _ in range(2)]
    descs = [kd_fa.make_desc(q, k, v, None, o, D ** -0.5) for o in outs]
    ws = torch.empty(kd_fa.workspace_size_full(descs[0]), dtype=torch.uint8, device=DEV)
    assert kd_fa.run_desc(descs[0], workspace=ws) == kd_fa.OK
    assert kd_fa.run_static(descs[1]) == kd_fa.OK
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
