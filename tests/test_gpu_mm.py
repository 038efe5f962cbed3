"""GPU parity of the linear-layer product (include/kd_mm.h): ops::linear
(src/core/ops.hpp:27-43) with Q4_0 / Q8_0 / BF16 / F16 / F32 weights.

- kd_mm_dequant is bitwise the oracle's dequantization rounded to BF16.
- kd_mm_run against the float64 product of the same BF16-rounded operands
  (the arithmetic the header states): every output within 1e-4 of
  sum_k |w_k x_k| -- the F32 accumulation's error scale; a dropped or
  doubled 32-k block would be off by ~1% of it.
- Against the exact product of the unrounded dequantized weights and F32 x,
  and against the oracle's restatement of ggml's CPU path (x rounded to
  Q8_0): reported and bounded (cosine >= 0.9999).
The shapes walk the 256 x 256 tiles and 32-k stages: M and N below, at and
past a tile, K of one to many stages, both tile orders (output tiles a
multiple of 4 or not), x as F32 and BF16, 3-D x, bias on and off, and the
31,744-token DiT projection shape with sampled rows.
"""
import numpy as np
import pytest
import torch

import kd_mm
import kd_oracle_quant as oq

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
QT = {"q8_0": oq.TYPE_Q8_0, "q4_0": oq.TYPE_Q4_0}


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _weight(kind, N, K, seed):
    """(device weight for kd_mm, F32 dequantized values (N, K))."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    if kind in QT:
        b = oq.quantize_q8_0(w) if kind == "q8_0" else oq.quantize_q4_0(w)
        return kd_mm.QuantWeight(torch.from_numpy(b).to(DEV), QT[kind], K), oq.dequantize(b, QT[kind], K)
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[kind]
    t = torch.from_numpy(w).to(dt)
    return t.to(DEV), t.float().numpy()


def _check(got, wd, x32, bias, what, exact_too=True):
    """got (M, N) vs the float64 product of BF16-rounded operands."""
    g = got.detach().cpu().double().numpy().reshape(-1, wd.shape[0])
    wr, xr = oq.round_bf16(wd), oq.round_bf16(x32)
    ref = oq.mul_mat_f64(wr, xr, bias)
    scale = oq.abs_product_sum(wr, xr)
    err = np.abs(g - ref)
    assert np.all(np.isfinite(g)), what
    assert np.all(err <= 1e-4 * scale + 1e-6), f"{what}: worst {np.max(err / (scale + 1e-30)):.3e} of sum|wx|"
    if exact_too:
        ex = oq.mul_mat_f64(wd, x32, bias)
        cos = np.sum(g * ex) / np.sqrt(np.sum(g * g) * np.sum(ex * ex))
        assert cos >= 0.9999, f"{what}: cosine to the exact product {cos}"


CASES = [
    # M, N, K, weight, x dtype, bias
    (1, 4, 32, "q8_0", torch.float32, False),
    (37, 100, 64, "q4_0", torch.float32, True),
    (256, 256, 256, "q8_0", torch.bfloat16, True),
    (300, 260, 96, "bf16", torch.float32, False),
    (513, 516, 4096, "q8_0", torch.float32, True),
    (257, 1024, 512, "q4_0", torch.bfloat16, False),
    (64, 128, 160, "f16", torch.bfloat16, True),
    (100, 36, 1024, "f32", torch.float32, True),
    # output tiles a multiple of 4 (the column-grouped tile order) with
    # partial last tiles in both directions
    (600, 2000, 128, "bf16", torch.bfloat16, True),
    (70, 1000, 224, "q8_0", torch.float32, False),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"M{c[0]}N{c[1]}K{c[2]}{c[3]}x{str(c[4])[-4:]}{'b' if c[5] else ''}")
def test_mm_parity(case):
    _need_gpu()
    M, N, K, kind, xdt, has_bias = case
    _announce(f"mm {case}")
    w, wd = _weight(kind, N, K, seed=M + N + K)
    rng = np.random.default_rng(K)
    x32 = rng.standard_normal((M, K)).astype(np.float32)
    x = torch.from_numpy(x32).to(xdt)
    xval = x.float().numpy()
    bias = (rng.standard_normal(N) * 0.1).astype(np.float32) if has_bias else None
    out = kd_mm.linear(x.to(DEV), w, None if bias is None else torch.from_numpy(bias).to(DEV))
    torch.cuda.synchronize()
    _check(out, wd, xval, bias, f"mm {case}")
    again = kd_mm.linear(x.to(DEV), w, None if bias is None else torch.from_numpy(bias).to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(out, again)


@pytest.mark.parametrize("kind", ["q8_0", "q4_0", "bf16", "f16", "f32"])
def test_dequant_bitwise(kind):
    _need_gpu()
    _announce(f"dequant {kind}")
    N, K = 70, 320
    w, wd = _weight(kind, N, K, seed=11)
    got = kd_mm.dequant(w)
    torch.cuda.synchronize()
    expect = torch.from_numpy(oq.round_bf16(wd)).to(torch.bfloat16)
    assert torch.equal(got.cpu(), expect)


def test_bf16_weight_direct_equals_workspace_path():
    """A BF16 weight is multiplied as stored; the same values given as F32
    go through the workspace expansion: bitwise the same product."""
    _need_gpu()
    _announce("bf16 direct vs f32 through workspace")
    M, N, K = 200, 300, 384
    wb, _ = _weight("bf16", N, K, seed=3)
    x = torch.randn((M, K), generator=torch.Generator().manual_seed(4)).to(DEV)
    direct = kd_mm.linear(x, wb)
    via_ws = kd_mm.linear(x, wb.float())
    torch.cuda.synchronize()
    assert torch.equal(direct, via_ws)


def test_three_d_activations_and_ggml_path():
    """x (B, L, K) flattened as ops::linear's reshape; the oracle's
    restatement of ggml's CPU path (x rounded to Q8_0) stays close."""
    _need_gpu()
    _announce("3-D x vs ggml path")
    B, L, N, K = 2, 150, 260, 512
    w, wd = _weight("q4_0", N, K, seed=21)
    x = torch.randn((B, L, K), generator=torch.Generator().manual_seed(22))
    out = kd_mm.linear(x.to(DEV), w)
    torch.cuda.synchronize()
    assert out.shape == (B, L, N)
    x32 = x.numpy().reshape(B * L, K)
    _check(out, wd, x32, None, "3-D")
    gg = oq.mul_mat_ggml(w.blocks.cpu().numpy(), oq.TYPE_Q4_0, x32).astype(np.float64)
    g = out.cpu().double().numpy().reshape(B * L, N)
    cos = np.sum(g * gg) / np.sqrt(np.sum(g * g) * np.sum(gg * gg))
    assert cos >= 0.9999, f"cosine to the ggml path {cos}"


def test_workspace_errors():
    _need_gpu()
    _announce("workspace errors")
    w, _ = _weight("q8_0", 64, 64, seed=1)
    x = torch.randn((8, 64), device=DEV)
    dst = torch.empty((8, 64), device=DEV)
    d = kd_mm.make_desc(w, x, None, dst)
    assert kd_mm.workspace_size(d) == 64 * 64 * 2
    assert kd_mm.run_desc(d, None) == -1          # KD_FA_ERR_NULL
    small = torch.empty(64 * 64 * 2 - 16, dtype=torch.uint8, device=DEV)
    assert kd_mm.run_desc(d, small) == -4         # KD_FA_ERR_LAYOUT
    torch.cuda.synchronize()


def test_dit_projection_shape_sampled():
    """to_query at the 31,744-token shape: x F32 (31744, 4096), Q8_0 weight
    4096 x 4096, bias; 24 sampled rows against float64."""
    _need_gpu()
    _announce("DiT projection 31744 x 4096 x 4096 q8_0")
    M, N, K = 31744, 4096, 4096
    w, wd = _weight("q8_0", N, K, seed=31)
    g = torch.Generator(device=DEV).manual_seed(32)
    x = torch.randn((M, K), generator=g, device=DEV)
    bias = torch.randn(N, generator=g, device=DEV) * 0.1
    out = kd_mm.linear(x, w, bias)
    torch.cuda.synchronize()
    rows = np.concatenate([[0, M - 1], np.random.default_rng(33).choice(M, 22, replace=False)])
    ri = torch.from_numpy(rows).to(DEV)
    _check(out[ri], wd, x[ri].cpu().numpy(), bias.cpu().numpy(), "DiT shape", exact_too=True)
