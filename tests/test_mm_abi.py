"""Host-side checks of the linear-layer C ABI (include/kd_mm.h), no GPU:
every declared symbol is exported, kd_mm_supports accepts the node as
ops::linear (src/core/ops.hpp:27-43) builds it for each weight format and
rejects what the kernels cannot run with the documented reason, and the
workspace size rule."""
import ctypes

import numpy as np
import pytest
import torch

import kd_fa
import kd_mm
import kd_oracle_quant as oq


def test_library_exports_every_kd_mm_symbol():
    syms = kd_mm.header_symbols()
    assert set(syms) == {"kd_mm_supports", "kd_mm_workspace_size", "kd_mm_dequant", "kd_mm_run"}
    lib = kd_fa.lib()
    for s in syms:
        assert hasattr(lib, s), s


def test_desc_is_four_tensor_views():
    assert ctypes.sizeof(kd_mm.KdMmDesc) == 4 * ctypes.sizeof(kd_fa.KdFaTensor)


def _qw(kind, N, K):
    w = np.random.default_rng(0).standard_normal((N, K)).astype(np.float32)
    if kind == "q8_0":
        return kd_mm.QuantWeight(torch.from_numpy(oq.quantize_q8_0(w)), kd_mm.TYPE_Q8_0, K)
    if kind == "q4_0":
        return kd_mm.QuantWeight(torch.from_numpy(oq.quantize_q4_0(w)), kd_mm.TYPE_Q4_0, K)
    return torch.from_numpy(w).to({"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[kind])


@pytest.mark.parametrize("kind", ["q8_0", "q4_0", "bf16", "f16", "f32"])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_accepts_linear_node(kind, xdt):
    w = _qw(kind, 64, 96)
    x = torch.zeros((3, 5, 96), dtype=xdt)
    ok, reason = kd_mm.supports(w, x, torch.zeros(64))
    assert ok, reason
    dst = torch.empty((3, 5, 64))
    d = kd_mm.make_desc(w, x, None, dst)
    assert kd_mm.workspace_size(d) == (0 if kind == "bf16" else 64 * 96 * 2)


def test_rejections_carry_reason():
    w = _qw("q8_0", 64, 96)
    assert kd_mm.supports(w, torch.zeros((4, 96), dtype=torch.float16)) == (False, kd_fa.ERR_TYPE)
    assert kd_mm.supports(w, torch.zeros((4, 64))) == (False, kd_fa.ERR_SHAPE)          # K mismatch
    w60 = _qw("f32", 62, 96)
    assert kd_mm.supports(w60, torch.zeros((4, 96))) == (False, kd_fa.ERR_SHAPE)        # N % 4
    assert kd_mm.supports(w, torch.zeros((4, 96)), torch.zeros(63)) == (False, kd_fa.ERR_SHAPE)
    xs = torch.zeros((4, 98))[:, :96]                                                   # row stride 392 B
    assert kd_mm.supports(w, xs) == (False, kd_fa.ERR_LAYOUT)
    wt = torch.zeros((96, 64)).t()                                                      # K not contiguous
    assert kd_mm.supports(wt, torch.zeros((4, 96))) == (False, kd_fa.ERR_LAYOUT)


def test_k_must_be_whole_blocks():
    w = torch.zeros((8, 40))
    ok, reason = kd_mm.supports(w, torch.zeros((2, 40)))
    assert not ok and reason == kd_fa.ERR_SHAPE


def test_run_validates_before_touching_the_device():
    w = _qw("q8_0", 64, 96)
    d = kd_mm.make_desc(w, torch.zeros((4, 96), dtype=torch.float16), None, torch.empty((4, 64)))
    assert kd_mm._lib().kd_mm_run(ctypes.byref(d), None, 0, None) == kd_fa.ERR_TYPE
    t = kd_mm.w_view(w)
    assert kd_mm._lib().kd_mm_dequant(ctypes.byref(t), None, 0, None) == kd_fa.ERR_NULL


def test_python_type_ids_equal_the_header():
    """The KD_MM_TYPE_* ids of include/kd_mm.h are kd_mm.TYPE_* (the ctypes mirror)."""
    import re
    text = open(kd_mm.HEADER_PATH).read()
    ids = {m.group(1): int(m.group(2)) for m in re.finditer(r"\bKD_MM_(TYPE_[A-Z0-9_]+)\s*=\s*(-?\d+)", text)}
    assert len(ids) == 5
    for name, value in ids.items():
        assert getattr(kd_mm, name) == value, name
