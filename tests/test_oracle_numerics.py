"""Pins the oracle's number formats and RoPE against independent sources:
numpy / torch conversions, float64 closed forms, complex multiplication,
and the invariants RoPE must satisfy (src/rope.hpp:23-155)."""
import numpy as np
import pytest
import torch

import kd_oracle as orc
from fa_common import AXES, SCALE_FACTOR, THETA

# ----------------------------------------------------------------------------
# conversions
# ----------------------------------------------------------------------------


def test_f16_decode_all_patterns():
    bits = np.arange(65536, dtype=np.uint16)
    got = orc.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _probe_floats(seed=0):
    rng = np.random.default_rng(seed)
    x = [rng.standard_normal(20000).astype(np.float32),
         (rng.standard_normal(20000) * 1e-5).astype(np.float32),      # f16 subnormal range
         (rng.standard_normal(20000) * 3e4).astype(np.float32),       # near f16 overflow
         np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, 1e-8, -1e-8,
                   6.103515625e-05, 5.960464477539063e-08, 2.98e-08], dtype=np.float32)]
    # exact halfway points between neighbouring f16 values (ties to even)
    h = np.arange(0x0400, 0x7bff, 37, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt = (np.arange(0x0400, 0x7bff, 37, dtype=np.uint16) + 1).view(np.float16).astype(np.float64)
    x.append(((h + nxt) / 2).astype(np.float32))
    return np.concatenate(x)


def test_f32_to_f16_round_to_nearest_even():
    x = _probe_floats()
    got = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f16c_conversions_equal_software_codec():
    """The F16C path of the CPU baseline's F16 accumulator: every F16
    pattern decoded and every positive F32 pattern from 2^-26 (below half
    the smallest F16 subnormal) to 2^17 (beyond the F16 overflow) encoded,
    bit for bit equal to the software codec; negatives, NaN payloads,
    infinities and the rest of the range on strided sweeps."""
    lo, hi = 0x32800000, 0x48000000                 # 2^-26 .. 2^17
    assert orc.f16_codec_mismatches(lo, 1, hi - lo) == 0
    assert orc.f16_codec_mismatches(0x80000000 | lo, 1, (hi - lo) // 7 + 1) == 0
    assert orc.f16_codec_mismatches(0, 4099, (1 << 32) // 4099) == 0
    assert orc.f16_codec_mismatches(0x7f800000, 1, 1 << 16) == 0      # +inf, NaNs
    assert orc.f16_codec_mismatches(0xff800000, 1, 1 << 16) == 0
    x = _probe_floats(3)
    with np.errstate(over="ignore"):
        assert np.array_equal(orc.f32_to_f16_bits_hw(x), x.astype(np.float16).view(np.uint16))


def test_f32_to_bf16_round_to_nearest_even():
    x = _probe_floats(1)
    rng = np.random.default_rng(2)
    u = rng.integers(0, 2**32, 50000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    u = u[np.isfinite(u)]
    x = np.concatenate([x, u])
    got = orc.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    back = orc.bf16_bits_to_f32(got)
    assert np.array_equal(back, torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float().numpy())


# ----------------------------------------------------------------------------
# RoPE tables (rope.hpp:23-102)
# ----------------------------------------------------------------------------


def test_freqs_closed_form():
    for n in (16, 24, 64):
        f = orc.rope_freqs(n, THETA)
        ref = np.exp(-np.log(THETA) * np.arange(n) / n)
        assert f[0] == 1.0
        # float expf/logf of an argument up to ln(1e4) ~ 9.2: a few ulp of the argument
        assert np.allclose(f, ref, rtol=3e-6, atol=0)
        assert np.all(np.diff(f) < 0)


def _angles_f64(T, Hp, Wp, axes, sf, theta):
    out = []
    for t in range(T):
        for h in range(Hp):
            for w in range(Wp):
                row = []
                for pos, a, s in zip((t, h, w), axes, sf):
                    n = a // 2
                    row.append(pos * np.exp(-np.log(theta) * np.arange(n) / n) / s)
                out.append(np.concatenate(row))
    return np.array(out)


def test_visual_table_closed_form_and_kats():
    T, Hp, Wp = 4, 6, 5
    tab = orc.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    assert tab.shape == (T * Hp * Wp, 128)
    ang = _angles_f64(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    assert np.allclose(tab[:, 0::2], np.cos(ang), atol=2e-6)
    assert np.allclose(tab[:, 1::2], np.sin(ang), atol=2e-6)
    # position (0,0,0): identity rotation in every column
    assert np.all(tab[0, 0::2] == 1.0) and np.all(tab[0, 1::2] == 0.0)
    # row index (t*Hp + h)*Wp + w; first pair of each block has frequency 1
    t, h, w = 3, 5, 2
    row = tab[(t * Hp + h) * Wp + w]
    assert np.isclose(row[0], np.cos(t), atol=1e-6) and np.isclose(row[1], np.sin(t), atol=1e-6)
    # the h and w angles are divided by scale_factor 2; blocks start at 32 / 80
    assert np.isclose(row[32], np.cos(h / 2), atol=1e-6) and np.isclose(row[33], np.sin(h / 2), atol=1e-6)
    assert np.isclose(row[80], np.cos(w / 2), atol=1e-6) and np.isclose(row[81], np.sin(w / 2), atol=1e-6)
    # 16 / 24 / 24 frequencies per block: the pair after each block restarts at frequency 1
    assert not np.isclose(row[30], np.cos(t), atol=1e-3)


def test_visual_table_scale_factor_one():
    tab = orc.visual_rope_table(2, 3, 3, AXES, (1.0, 1.0, 1.0), THETA)
    row = tab[(1 * 3 + 2) * 3 + 1]
    assert np.isclose(row[32], np.cos(2.0), atol=1e-6) and np.isclose(row[80], np.cos(1.0), atol=1e-6)


def test_product_tables_equal_oracle_tables():
    """libkd_fa's host table helpers give the oracle's values bit for bit,
    and the factorised per-axis table holds exactly the table's columns."""
    import kd_fa
    T, Hp, Wp = 5, 16, 16
    a = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    b = orc.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    ax = kd_fa.axes_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    t_tab = ax[: T * 32].reshape(T, 32)
    h_tab = ax[T * 32: T * 32 + Hp * 48].reshape(Hp, 48)
    w_tab = ax[T * 32 + Hp * 48:].reshape(Wp, 48)
    idx = np.arange(T * Hp * Wp)
    t, h, w = idx // (Hp * Wp), (idx // Wp) % Hp, idx % Wp
    rebuilt = np.concatenate([t_tab[t], h_tab[h], w_tab[w]], axis=1)
    assert np.array_equal(rebuilt.view(np.uint32), a.view(np.uint32))
    tt = kd_fa.text_rope_table(37, 128)
    assert np.array_equal(tt.view(np.uint32), orc.text_rope_table(37, 128).view(np.uint32))


def test_text_table_closed_form():
    tab = orc.text_rope_table(50, 128)
    ang = np.arange(50)[:, None] * np.exp(-np.log(THETA) * np.arange(64) / 64)[None, :]
    assert np.allclose(tab[:, 0::2], np.cos(ang), atol=3e-6)
    assert np.allclose(tab[:, 1::2], np.sin(ang), atol=3e-6)


# ----------------------------------------------------------------------------
# rope::apply (rope.hpp:109-155)
# ----------------------------------------------------------------------------


def _x(B, L, H, seed):
    return np.random.default_rng(seed).standard_normal((B, L, H, 128)).astype(np.float32)


def test_apply_is_complex_multiplication():
    B, L, H = 2, 60, 3
    tab = orc.visual_rope_table(3, 4, 5, AXES, SCALE_FACTOR, THETA)
    x = _x(B, L, H, 0)
    got = orc.rope_apply(x, tab)
    z = (x[..., 0::2] + 1j * x[..., 1::2]).astype(np.complex128)
    e = (tab[:, 0::2] + 1j * tab[:, 1::2]).astype(np.complex128)[None, :, None, :]
    ref = z * e
    assert np.allclose(got[..., 0::2], ref.real, atol=2e-6)
    assert np.allclose(got[..., 1::2], ref.imag, atol=2e-6)
    # the same (cos, sin) row serves every head
    assert np.allclose(got[:, :, 0, :], orc.rope_apply(x[:, :, :1, :], tab)[:, :, 0, :], atol=0)


def test_apply_rounds_each_op_separately():
    """out0 = fl(fl(x0*c) - fl(x1*s)): no fused multiply-add."""
    B, L, H = 1, 30, 2
    tab = orc.visual_rope_table(2, 3, 5, AXES, SCALE_FACTOR, THETA)
    x = _x(B, L, H, 1)
    got = orc.rope_apply(x, tab)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    c, s = tab[None, :, None, 0::2], tab[None, :, None, 1::2]
    r0 = (x0 * c).astype(np.float32) - (x1 * s).astype(np.float32)
    r1 = (x0 * s).astype(np.float32) + (x1 * c).astype(np.float32)
    assert np.array_equal(got[..., 0::2], r0) and np.array_equal(got[..., 1::2], r1)


def test_apply_invariants():
    B, L, H = 1, 64, 2
    tab = orc.text_rope_table(L + 20, 128)
    x = _x(B, L, H, 2)
    y = orc.rope_apply(x, tab[:L])
    # per-pair norm preserved
    n0 = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    n1 = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    assert np.allclose(n0, n1, rtol=2e-5, atol=1e-6)
    # identity at position 0
    assert np.array_equal(y[:, 0], x[:, 0])
    # <R(p) q, R(p+d) k> depends only on d
    q = _x(1, 1, 1, 3)[0, 0, 0]
    k = _x(1, 1, 1, 4)[0, 0, 0]
    pos = np.stack([np.broadcast_to(q, (L + 20, 128)), np.broadcast_to(k, (L + 20, 128))], 0)[:, :, None, :]
    r = orc.rope_apply(np.ascontiguousarray(pos), tab)
    d = 7
    dots = [float(np.dot(r[0, p, 0].astype(np.float64), r[1, p + d, 0].astype(np.float64))) for p in range(0, 40, 5)]
    assert np.allclose(dots, dots[0], rtol=1e-4, atol=1e-4)
    # a rotation the other way (sign error) would not satisfy the complex form
    wrong = x.copy()
    wrong[..., 0::2] = x[..., 0::2] * tab[None, :L, None, 0::2] + x[..., 1::2] * tab[None, :L, None, 1::2]
    assert not np.allclose(wrong[:, 1:], y[:, 1:], atol=1e-3)


@pytest.mark.parametrize("neox", [True])
def test_apply_is_not_half_split(neox):
    """Pairs are interleaved (x[2i], x[2i+1]), not NeoX halves (x[i], x[i+D/2])."""
    tab = orc.text_rope_table(8, 128)
    x = _x(1, 8, 1, 5)
    y = orc.rope_apply(x, tab)
    half = x.copy()
    c, s = tab[None, :, None, 0::2], tab[None, :, None, 1::2]
    half[..., :64] = x[..., :64] * c - x[..., 64:] * s
    half[..., 64:] = x[..., :64] * s + x[..., 64:] * c
    assert not np.allclose(half[:, 1:], y[:, 1:], atol=1e-3)
