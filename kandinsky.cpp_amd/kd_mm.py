"""ctypes binding of the linear-layer product (include/kd_mm.h) in
libkd_fa.so: ops::linear (src/core/ops.hpp:27-43) = ggml_mul_mat(w, x) plus
the Linear bias (src/core/module.hpp:87-110), with w in the formats the
reference's converter writes (scripts/convert_to_gguf.py:90-146).

Weights are torch tensors (N, K) of float32 / float16 / bfloat16, or
QuantWeight: the raw Q4_0 / Q8_0 blocks of each row as a uint8 tensor
(N, K/32 * block_bytes).  x is (..., K) float32 or bfloat16; the result is
(..., N) float32.  There is no fallback path: the library must be built.
"""
from __future__ import annotations

import ctypes
import os
import re

import kd_fa

HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "kd_mm.h")

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q4_0 = 2
TYPE_Q8_0 = 8
TYPE_BF16 = 30
BLOCK_BYTES = {TYPE_Q8_0: 34, TYPE_Q4_0: 18}


class KdMmDesc(ctypes.Structure):
    """struct kd_mm_desc: the GGML_OP_MUL_MAT node plus its bias."""

    _fields_ = [
        ("w", kd_fa.KdFaTensor),
        ("x", kd_fa.KdFaTensor),
        ("bias", kd_fa.KdFaTensor),
        ("dst", kd_fa.KdFaTensor),
    ]


class QuantWeight:
    """Q4_0 / Q8_0 weight rows: `blocks` uint8 (N, K/32 * block_bytes)."""

    def __init__(self, blocks, qtype: int, K: int):
        if qtype not in BLOCK_BYTES:
            raise ValueError(f"not a block format: {qtype}")
        if K % 32 or blocks.dim() != 2 or blocks.shape[1] != K // 32 * BLOCK_BYTES[qtype]:
            raise ValueError("blocks must be (N, K/32 * block_bytes)")
        self.blocks, self.type, self.K, self.N = blocks, qtype, K, blocks.shape[0]

    def to(self, device):
        return QuantWeight(self.blocks.to(device), self.type, self.K)


_BOUND = False


def _lib():
    global _BOUND
    lib = kd_fa.lib()
    if not _BOUND:
        P = ctypes.POINTER
        lib.kd_mm_supports.argtypes = [P(KdMmDesc), P(ctypes.c_int)]
        lib.kd_mm_supports.restype = ctypes.c_int
        lib.kd_mm_workspace_size.argtypes = [P(KdMmDesc)]
        lib.kd_mm_workspace_size.restype = ctypes.c_size_t
        lib.kd_mm_dequant.argtypes = [P(kd_fa.KdFaTensor), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.kd_mm_dequant.restype = ctypes.c_int
        lib.kd_mm_run.argtypes = [P(KdMmDesc), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.kd_mm_run.restype = ctypes.c_int
        _BOUND = True
    return lib


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Function names declared in include/kd_mm.h."""
    with open(path) as f:
        text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    return sorted(set(re.findall(r"\b(kd_mm_\w+)\s*\(", text)))


def w_view(w) -> kd_fa.KdFaTensor:
    """ggml view [K, N] of a weight."""
    if isinstance(w, QuantWeight):
        t = kd_fa.KdFaTensor()
        t.type = w.type
        bb = BLOCK_BYTES[w.type]
        t.ne[0], t.ne[1], t.ne[2], t.ne[3] = w.K, w.N, 1, 1
        row = int(w.blocks.stride(0))
        t.nb[0], t.nb[1], t.nb[2], t.nb[3] = bb, row, row * w.N, row * w.N
        t.data = w.blocks.data_ptr() if w.blocks.numel() else 0
        return t
    if w.dim() != 2:
        raise ValueError("a float weight is (N, K)")
    return kd_fa.view(w)


def make_desc(w, x, bias, dst) -> KdMmDesc:
    d = KdMmDesc()
    d._keep = (w, x, bias, dst)
    d.w = w_view(w)
    d.x = kd_fa.view(x)
    d.bias = kd_fa.view(bias)
    d.dst = kd_fa.view(dst)
    return d


def supports(w, x, bias=None, dst=None):
    """(ok, reason) of kd_mm_supports for this node."""
    torch = kd_fa._torch()
    if dst is None:
        dst = torch.empty(tuple(x.shape[:-1]) + (w.N if isinstance(w, QuantWeight) else w.shape[0],),
                          dtype=torch.float32, device=x.device)
    reason = ctypes.c_int(0)
    ok = _lib().kd_mm_supports(ctypes.byref(make_desc(w, x, bias, dst)), ctypes.byref(reason))
    return bool(ok), reason.value


def workspace_size(desc: KdMmDesc) -> int:
    return int(_lib().kd_mm_workspace_size(ctypes.byref(desc)))


def run_desc(desc: KdMmDesc, workspace=None, stream=None) -> int:
    torch = kd_fa._torch()
    handle = stream.cuda_stream if stream is not None else torch.cuda.current_stream().cuda_stream
    wp = workspace.data_ptr() if workspace is not None else None
    nbytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    return _lib().kd_mm_run(ctypes.byref(desc), ctypes.c_void_p(wp), nbytes, ctypes.c_void_p(handle))


def dequant(w, stream=None):
    """kd_mm_dequant: the weight as BF16 (N, K) on the weight's device."""
    torch = kd_fa._torch()
    src = w.blocks if isinstance(w, QuantWeight) else w
    N, K = (w.N, w.K) if isinstance(w, QuantWeight) else (w.shape[0], w.shape[1])
    out = torch.empty((N, K), dtype=torch.bfloat16, device=src.device)
    handle = stream.cuda_stream if stream is not None else torch.cuda.current_stream().cuda_stream
    t = w_view(w)
    st = _lib().kd_mm_dequant(ctypes.byref(t), ctypes.c_void_p(out.data_ptr()), out.numel() * 2,
                              ctypes.c_void_p(handle))
    if st != kd_fa.OK:
        raise kd_fa.KdFaError(st, "kd_mm_dequant")
    return out


def linear(x, w, bias=None, dst=None, workspace=None, stream=None):
    """ops::linear on the GPU: x (..., K) -> (..., N) float32."""
    torch = kd_fa._torch()
    N = w.N if isinstance(w, QuantWeight) else w.shape[0]
    if dst is None:
        dst = torch.empty(tuple(x.shape[:-1]) + (N,), dtype=torch.float32, device=x.device)
    d = make_desc(w, x, bias, dst)
    need = workspace_size(d)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    st = run_desc(d, workspace if need else None, stream)
    if st != kd_fa.OK:
        raise kd_fa.KdFaError(st, "kd_mm_run")
    return dst
