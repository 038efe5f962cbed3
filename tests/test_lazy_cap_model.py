"""The lazy running max of the unmasked kernels, modelled on the CPU.

The kernels take a 64-key tile's exponents against the row's running max m
and recompute the exact max only when the tile's weight sum leaves
[0, cap]; the weights are then rounded to the operand type for the PV
product.  Every weight is at most the sum, so a cap below the type's
round-to-infinity threshold keeps every rounded weight finite.  These tests
read the caps from the sources (the device header and the generator of the
hand-scheduled loop), check them against that threshold, and run the rule
on a row with a key 12 nats above its first-tile max: numpy's float16
rounding turns that weight into +inf under the BF16 cap (2^64) and keeps it
finite under the F16 one.
"""
import importlib.util
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "kandinsky.cpp_amd", "csrc")
F16_INF_THRESHOLD = 65520.0     # float16 rounds x >= 65520 to +inf (RNE)


def _header_caps():
    with open(os.path.join(CSRC, "kd_fa_device.h")) as f:
        text = f.read()
    caps = {}
    for t, name in (("__bf16", "bf16"), ("_Float16", "f16")):
        m = re.search(r"struct Elem<%s>\s*\{.*?kSumCap\s*=\s*([0-9.e+]+)f;" % re.escape(t), text, re.S)
        assert m, t
        caps[name] = float(m.group(1))
    return caps


def _generator_caps():
    spec = importlib.util.spec_from_file_location("gen_w64_loop", os.path.join(CSRC, "gen_w64_loop.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return {t: float(np.array([int(h, 16)], dtype=np.uint32).view(np.float32)[0]) for t, h in mod.SUM_CAP.items()}


def test_caps_agree_and_fit_the_types():
    hc, gc = _header_caps(), _generator_caps()
    assert hc == gc
    assert hc["f16"] < F16_INF_THRESHOLD
    assert np.isfinite(np.float16(hc["f16"]))
    assert hc["bf16"] == 2.0 ** 64


def _lazy_row(s_log2, cap, rnd):
    """Per 64-key tile: weights against m; if the row's own sum leaves
    [0, cap], m moves to the tile max and the weights are redone (the
    kernels' rule, decided per row); returns the rounded weights of every
    tile."""
    m = -np.inf
    out = []
    for t in range(0, len(s_log2), 64):
        s = s_log2[t:t + 64]
        with np.errstate(over="ignore", invalid="ignore"):
            p = np.exp2(s - m)
            total = p.sum()
        if not total <= cap:
            m = max(m, s.max())
            p = np.exp2(s - m)
        with np.errstate(over="ignore"):
            out.append(rnd(p))
    return np.concatenate(out)


def _planted_row(gap_nats, seed=0):
    rng = np.random.default_rng(seed)
    s = rng.standard_normal(256)                    # logits in nats
    s[100] = s[:64].max() + gap_nats               # tile 1, above the tile-0 max
    return s * np.log2(np.e)


def test_f16_cap_keeps_rounded_weights_finite():
    caps = _header_caps()
    f16 = lambda p: p.astype(np.float16)
    for gap in (11.5, 12.0, 20.0, 40.0):
        s = _planted_row(gap)
        assert np.isfinite(_lazy_row(s, caps["f16"], f16)).all(), gap
        # the same row under the BF16 cap would overflow an F16 weight:
        # the planted inputs discriminate the two caps
        assert not np.isfinite(_lazy_row(s, caps["bf16"], f16)).all(), gap


def test_bf16_cap_with_bf16_rounding_is_finite():
    caps = _header_caps()

    def bf16(p):
        u = p.astype(np.float32).view(np.uint32)
        u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        return u.astype(np.uint32).view(np.float32)

    for gap in (12.0, 40.0):
        assert np.isfinite(_lazy_row(_planted_row(gap), caps["bf16"], bf16)).all()
