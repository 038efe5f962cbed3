"""Pins the oracle's linear-layer restatement (oracle/kd_oracle_quant.py):
the converter's Q8_0 / Q4_0 quantizers (scripts/convert_to_gguf.py:93-143),
ggml's dequantization and ggml's CPU mul_mat path, by closed forms, exact
special cases and error bounds chosen so that a plausible slip (round-half
rule, scale sign, nibble order, a dropped block, F16 scale not used) fails.
"""
import numpy as np
import pytest

import kd_oracle_quant as oq


def _blocks(rows):
    return np.asarray(rows, dtype=np.float32)


def test_q8_0_ramp_closed_form():
    w = _blocks([np.arange(32, dtype=np.float32)])
    b = oq.quantize_q8_0(w)
    assert b.shape == (1, 34)
    d = np.frombuffer(b[0, :2].tobytes(), dtype=np.float16)[0]
    assert d == np.float16(np.float32(31) / np.float32(127))
    q = b[0, 2:].view(np.int8).astype(int)
    scale = np.float32(31) / np.float32(127)
    expect = [int(np.round(np.float32(j) / scale)) for j in range(32)]   # half to even
    assert q.tolist() == expect
    assert q[31] == 127 and q[0] == 0


def test_q8_0_zero_and_constant_blocks():
    w = _blocks([[0.0] * 32 + [-3.0] * 32])
    b = oq.quantize_q8_0(w)
    d0 = np.frombuffer(b[0, :2].tobytes(), dtype=np.float16)[0]
    assert d0 == np.float16(1.0)                     # all-zero block: scale 1
    assert np.all(b[0, 2:34] == 0)
    q1 = b[0, 36:68].view(np.int8)
    assert np.all(q1 == -127)
    d1 = np.frombuffer(b[0, 34:36].tobytes(), dtype=np.float16)[0]
    assert d1 == np.float16(np.float32(3) / np.float32(127))


def test_q8_0_round_half_even_differs_from_roundf():
    # x / scale = 2.5 exactly: the converter's np.round gives 2, C roundf 3
    w = np.zeros((1, 32), dtype=np.float32)
    w[0, 0] = 127.0
    w[0, 1] = 2.5
    q = oq.quantize_q8_0(w)[0, 2:].view(np.int8)
    assert q[0] == 127 and q[1] == 2
    d, qg = oq.quantize_row_q8_0_ggml(w)
    assert d[0, 0] == 1.0 and qg[0, 0, 1] == 3 and qg[0, 0, 0] == 127


def test_q4_0_closed_form_and_nibble_order():
    v = np.arange(32, dtype=np.float32) - 16.0          # -16 .. 15; max magnitude -16 at j = 0
    b = oq.quantize_q4_0(v[None, :])
    d = np.frombuffer(b[0, :2].tobytes(), dtype=np.float16)[0]
    assert d == np.float16(2.0)                          # max_signed / -8
    packed = b[0, 2:]
    lo = (packed & 15).astype(int)
    hi = (packed >> 4).astype(int)
    expect = [min(15, int(np.float32(x) * np.float32(0.5) + np.float32(8.5))) for x in v]
    assert lo.tolist() == expect[:16]                    # low nibble: element j
    assert hi.tolist() == expect[16:]                    # high nibble: element j + 16
    deq = oq.dequantize(b, oq.TYPE_Q4_0, 32)[0]
    assert deq[0] == -16.0                               # the extreme maps exactly
    assert deq[31] == 14.0                               # 15 clips to nibble 15: (15 - 8) * 2


def test_q4_0_zero_block():
    b = oq.quantize_q4_0(np.zeros((1, 32), dtype=np.float32))
    assert np.all(oq.dequantize(b, oq.TYPE_Q4_0, 32) == 0.0)


@pytest.mark.parametrize("qtype", [oq.TYPE_Q8_0, oq.TYPE_Q4_0])
def test_round_trip_error_bounds(qtype):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((16, 256)) * np.exp(rng.uniform(-6, 6, (16, 1)))).astype(np.float32)
    b = oq.quantize_q8_0(w) if qtype == oq.TYPE_Q8_0 else oq.quantize_q4_0(w)
    deq = oq.dequantize(b, qtype, 256)
    d, _ = oq.block_fields(b, qtype, 256)
    err = np.abs(deq - w).reshape(16, 8, 32).max(axis=2)
    bound = np.abs(d) * (0.5 + 127 * 2.0 ** -11 + 1e-6) if qtype == oq.TYPE_Q8_0 else np.abs(d) * (1.0 + 8 * 2.0 ** -10)
    assert np.all(err <= bound)
    # the F16 scale is the one that multiplies: dequantizing with it is exact
    _, q = oq.block_fields(b, qtype, 256)
    assert np.array_equal(deq, (q.astype(np.float32) * d[:, :, None]).reshape(16, 256))


def test_mul_mat_ggml_exact_on_integer_operands():
    """Integers with block maxima 127 are exactly representable in Q8_0 (d =
    1), so ggml's path is exact integer arithmetic there."""
    rng = np.random.default_rng(5)
    K, N, M = 128, 8, 6
    w = rng.integers(-127, 128, (N, K)).astype(np.float32)
    x = rng.integers(-127, 128, (M, K)).astype(np.float32)
    w.reshape(N, K // 32, 32)[:, :, 0] = 127
    x.reshape(M, K // 32, 32)[:, :, 0] = -127
    b = oq.quantize_q8_0(w)
    assert np.array_equal(oq.dequantize(b, oq.TYPE_Q8_0, K), w)
    got = oq.mul_mat_ggml(b, oq.TYPE_Q8_0, x)
    assert np.array_equal(got, (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32))


@pytest.mark.parametrize("qtype", [oq.TYPE_Q8_0, oq.TYPE_Q4_0])
def test_mul_mat_ggml_within_activation_quantization(qtype):
    """ggml's path differs from the exact product of the dequantized weights
    only by the Q8_0 rounding of x: |err| <= sum_k |w_k| * d_x(block)/2."""
    rng = np.random.default_rng(7)
    K, N, M = 256, 12, 5
    w = rng.standard_normal((N, K)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    b = oq.quantize_q8_0(w) if qtype == oq.TYPE_Q8_0 else oq.quantize_q4_0(w)
    wd = oq.dequantize(b, qtype, K)
    got = oq.mul_mat_ggml(b, qtype, x).astype(np.float64)
    exact = oq.mul_mat_f64(wd, x)
    dx, _ = oq.quantize_row_q8_0_ggml(x)
    bound = np.einsum("nbj,mb->mn", np.abs(wd).reshape(N, K // 32, 32), dx.astype(np.float64) * 0.5 * 1.01)
    bound += 1e-5 * oq.abs_product_sum(wd, x)
    assert np.all(np.abs(got - exact) <= bound)
    # and the bound is not vacuous: a product that drops the last block fails it
    wd_drop = wd.copy()
    wd_drop[:, -32:] = 0
    assert np.any(np.abs(oq.mul_mat_f64(wd_drop, x) - exact) > bound)


def test_round_bf16():
    bf16_max = np.uint32(0x7F7F0000).view(np.float32)
    a = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.0 ** 100, np.inf, 3.4e38, bf16_max],
                 dtype=np.float32)
    r = oq.round_bf16(a)
    assert r[0] == 1.0
    assert r[1] == 1.0                      # tie to even (mantissa ...0)
    assert r[2] == 1.0 + 4 * 2 ** -8        # tie to even (mantissa ...1 -> up)
    assert r[3] == -2.0 ** 100
    assert np.isinf(r[4]) and np.isinf(r[5])   # past the largest BF16: infinity
    assert r[6] == bf16_max
