"""ctypes binding of libkd_fa.so, the gfx950 GGML_OP_FLASH_ATTN_EXT hook.

Mirrors the reference's operator interface for the CrossDiT attention node:
``flash_attn_ext`` takes the same operands, scale and mask semantics as
``ggml_flash_attn_ext(ctx, q, k, v, mask, scale, max_bias, logit_softcap)``
followed by ``ggml_flash_attn_ext_set_prec(kqv, GGML_PREC_F32)``
(src/core/ops.hpp:176-177), and ``supports`` answers what
``ggml_backend_supports_op`` answers for it (src/core/ops.hpp:179).

Tensors are torch tensors whose shape is ggml's ``ne`` reversed, so the
ggml view ``[ne0, ne1, ne2, ne3]`` is the torch shape ``(ne3, ne2, ne1, ne0)``:

    q    (B,  H,   Lq,  Dk)   float32 / float16 / bfloat16
    k    (Bk, Hkv, Lk,  Dk)   float16 / bfloat16 (float32 in the workspace forms)
    v    (Bk, Hkv, Lk,  Dv)   same dtype as k (float32 in the workspace forms)
    mask (Bm, Hm,  Lq', Lk')  float16, optional
    dst  (B,  Lq,  H,   Dv)   float32   (ggml's permuted [Dv, H, Lq, B])

Strided views are passed through unchanged (byte strides = torch strides x
element size).  All compute runs in libkd_fa.so; a missing library raises.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
# KD_FA_LIB selects another build of the same library (e.g. a tuning variant)
LIB_PATH = os.environ.get("KD_FA_LIB") or os.path.join(_HERE, "libkd_fa.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "kd_fa.h")

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_BF16 = 30
PREC_DEFAULT = 0
PREC_F32 = 10

ROPE_NONE = 0
ROPE_TABLE = 1
ROPE_AXES = 2

OK = 0
ERR_NULL = -1
ERR_TYPE = -2
ERR_SHAPE = -3
ERR_LAYOUT = -4
ERR_PARAM = -5
ERR_ROPE = -6
ERR_LAUNCH = -7
ERR_DEVICE = -8
ERR_SCRATCH = -9
STATIC_SCRATCH_BYTES = 64 << 20
# layout version of the structs below (KD_FA_ABI_VERSION in include/kd_fa.h)
ABI_VERSION = 3

# kd_fa_set_routing flags (comparison hooks for tests and tuning)
ROUTE_DEFAULT = 0
ROUTE_NO_W64 = 1
ROUTE_NO_XRES = 2
ROUTE_D512_R1 = 4
ROUTE_NO_SPLIT = 8
ROUTE_W64_SHORT = 16
ROUTE_STAGED = 32
ROUTE_SUMMARY = 64
ROUTE_NO_XLONG = 128
ROUTE_NO_XLONG64 = 256


class KdFaTensor(ctypes.Structure):
    """struct kd_fa_tensor: a ggml tensor view (type, ne, nb, data)."""

    _fields_ = [
        ("type", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
        ("data", ctypes.c_void_p),
    ]


class KdFaDesc(ctypes.Structure):
    """struct kd_fa_desc: the GGML_OP_FLASH_ATTN_EXT node."""

    _fields_ = [
        ("q", KdFaTensor),
        ("k", KdFaTensor),
        ("v", KdFaTensor),
        ("mask", KdFaTensor),
        ("sinks", KdFaTensor),
        ("dst", KdFaTensor),
        ("scale", ctypes.c_float),
        ("max_bias", ctypes.c_float),
        ("logit_softcap", ctypes.c_float),
        ("prec", ctypes.c_int32),
        ("cast_type", ctypes.c_int32),
    ]


class KdFaRope(ctypes.Structure):
    """struct kd_fa_rope: RoPE rotation fused into the Q/K loads."""

    _fields_ = [
        ("mode", ctypes.c_int32),
        ("table", KdFaTensor),
        ("axes_data", ctypes.c_void_p),
        ("grid", ctypes.c_int32 * 3),
        ("axes", ctypes.c_int32 * 3),
    ]


class KdFaQkNorm(ctypes.Structure):
    """struct kd_fa_qk_norm: RMSNorm weights of the Q and K head rows."""

    _fields_ = [
        ("q_weight", ctypes.c_void_p),
        ("k_weight", ctypes.c_void_p),
        ("eps", ctypes.c_float),
    ]


class KdFaError(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        self.status = status
        msg = _lib().kd_fa_strerror(status).decode() if _LIB is not None else str(status)
        super().__init__(f"{what}: {msg} (status {status})" if what else f"{msg} (status {status})")


_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built: run `make -C kandinsky.cpp_amd` "
                "(or __graft_entry__.build()); there is no fallback path")
        lib = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER
        lib.kd_fa_supports.argtypes = [P(KdFaDesc), P(ctypes.c_int)]
        lib.kd_fa_supports.restype = ctypes.c_int
        lib.kd_fa_rope_supports.argtypes = [P(KdFaDesc), P(KdFaRope), P(ctypes.c_int)]
        lib.kd_fa_rope_supports.restype = ctypes.c_int
        lib.kd_fa_run.argtypes = [P(KdFaDesc), ctypes.c_void_p]
        lib.kd_fa_run.restype = ctypes.c_int
        lib.kd_fa_run_ws.argtypes = [P(KdFaDesc), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.kd_fa_run_ws.restype = ctypes.c_int
        lib.kd_fa_workspace_size.argtypes = [P(KdFaDesc), P(KdFaRope), P(KdFaQkNorm)]
        lib.kd_fa_workspace_size.restype = ctypes.c_size_t
        lib.kd_fa_rope_run.argtypes = [P(KdFaDesc), P(KdFaRope), ctypes.c_void_p]
        lib.kd_fa_rope_run.restype = ctypes.c_int
        lib.kd_fa_rope_run_ws.argtypes = [P(KdFaDesc), P(KdFaRope), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.kd_fa_rope_run_ws.restype = ctypes.c_int
        lib.kd_fa_dit_run.argtypes = [P(KdFaDesc), P(KdFaRope), P(KdFaQkNorm), ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_void_p]
        lib.kd_fa_dit_run.restype = ctypes.c_int
        lib.kd_fa_dit_supports.argtypes = [P(KdFaDesc), P(KdFaRope), P(KdFaQkNorm), P(ctypes.c_int)]
        lib.kd_fa_dit_supports.restype = ctypes.c_int
        lib.kd_fa_rope_workspace_size.argtypes = [P(KdFaDesc)]
        lib.kd_fa_rope_workspace_size.restype = ctypes.c_size_t
        fp = P(ctypes.c_float)
        ip = P(ctypes.c_int)
        lib.kd_fa_rope_visual_table.argtypes = [ctypes.c_int] * 3 + [ip, fp, ctypes.c_float, fp]
        lib.kd_fa_rope_visual_table.restype = ctypes.c_int
        lib.kd_fa_rope_axes_size.argtypes = [ctypes.c_int] * 3 + [ip]
        lib.kd_fa_rope_axes_size.restype = ctypes.c_size_t
        lib.kd_fa_rope_axes_fill.argtypes = [ctypes.c_int] * 3 + [ip, fp, ctypes.c_float, fp]
        lib.kd_fa_rope_axes_fill.restype = ctypes.c_int
        lib.kd_fa_rope_text_table.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, fp]
        lib.kd_fa_rope_text_table.restype = ctypes.c_int
        lib.kd_fa_strerror.argtypes = [ctypes.c_int]
        lib.kd_fa_strerror.restype = ctypes.c_char_p
        lib.kd_fa_version.argtypes = []
        lib.kd_fa_version.restype = ctypes.c_int
        lib.kd_fa_dit_run_static.argtypes = [P(KdFaDesc), P(KdFaRope), P(KdFaQkNorm), ctypes.c_void_p]
        lib.kd_fa_dit_run_static.restype = ctypes.c_int
        lib.kd_fa_set_routing.argtypes = [ctypes.c_int]
        lib.kd_fa_set_routing.restype = ctypes.c_int
        lib.kd_fa_abi_version.argtypes = []
        lib.kd_fa_abi_version.restype = ctypes.c_int
        if lib.kd_fa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} lays out its structs as ABI version {lib.kd_fa_abi_version()}, "
                               f"this binding as {ABI_VERSION}: rebuild the library")
        _LIB = lib
    return _LIB


def lib():
    """The loaded libkd_fa.so (raises if it is not built)."""
    return _lib()


class routing:
    """Context manager over kd_fa_set_routing: ``with routing(ROUTE_NO_W64):``
    runs the enclosed calls with the flagged kernels taken out of the choice
    (a comparison hook for tests; production calls never set it)."""

    def __init__(self, flags: int):
        self.flags = int(flags)
        self.prev = None

    def __enter__(self):
        self.prev = _lib().kd_fa_set_routing(self.flags)
        return self

    def __exit__(self, *exc):
        _lib().kd_fa_set_routing(self.prev)
        return False


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Function names declared in include/kd_fa.h."""
    with open(path) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kd_fa_\w+)\s*\(", text)))


# ---------------------------------------------------------------------------
# tensor views
# ---------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def type_id(dtype) -> int:
    torch = _torch()
    if dtype == torch.float32:
        return TYPE_F32
    if dtype == torch.float16:
        return TYPE_F16
    if dtype == torch.bfloat16:
        return TYPE_BF16
    raise ValueError(f"no ggml type for {dtype}")


def view(t) -> KdFaTensor:
    """ggml view of a torch tensor of rank <= 4 (shape = ne reversed)."""
    if t is None:
        return KdFaTensor()
    if t.dim() > 4:
        raise ValueError("rank > 4")
    es = t.element_size()
    shape = list(t.shape)[::-1]
    strides = [s * es for s in list(t.stride())[::-1]]
    while len(shape) < 4:
        shape.append(1)
        strides.append(strides[-1] * shape[-2] if strides else es)
    d = KdFaTensor()
    d.type = type_id(t.dtype)
    for i in range(4):
        d.ne[i] = int(shape[i])
        d.nb[i] = int(strides[i])
    d.data = t.data_ptr() if t.numel() > 0 else 0
    return d


def make_desc(q, k, v, mask, dst, scale, max_bias=0.0, logit_softcap=0.0, prec=PREC_F32, cast_type=0) -> KdFaDesc:
    """The node over torch tensors.  ``cast_type``: the type an F32 K / V is
    cast to by the workspace forms (0 or TYPE_F16: ggml_cast to F16, as
    ops::attention does; TYPE_BF16)."""
    d = KdFaDesc()
    d._keep = (q, k, v, mask, dst)  # the struct holds raw pointers: keep the tensors alive
    d.q, d.k, d.v = view(q), view(k), view(v)
    d.mask = view(mask)
    d.dst = view(dst)
    d.scale = float(scale)
    d.max_bias = float(max_bias)
    d.logit_softcap = float(logit_softcap)
    d.prec = int(prec)
    d.cast_type = int(cast_type)
    return d


def rope_table(table) -> KdFaRope:
    """RoPE descriptor over a (L, D) float32 table (ggml [D, L])."""
    r = KdFaRope()
    r.mode = ROPE_TABLE
    r.table = view(table)
    r._keep = table  # the struct holds a raw pointer: keep the tensor alive
    return r


def rope_axes(axes_buf, grid, axes) -> KdFaRope:
    """RoPE descriptor over a factorised per-axis table (see kd_fa_rope_axes_fill)."""
    r = KdFaRope()
    r.mode = ROPE_AXES
    r.axes_data = axes_buf.data_ptr()
    r._keep = axes_buf
    for i in range(3):
        r.grid[i] = int(grid[i])
        r.axes[i] = int(axes[i])
    return r


def qk_norm(q_weight=None, k_weight=None, eps=1e-6) -> KdFaQkNorm:
    """RMSNorm descriptor over float32 (D,) device tensors (None: that side
    is not normalised)."""
    n = KdFaQkNorm()
    n.q_weight = q_weight.data_ptr() if q_weight is not None else None
    n.k_weight = k_weight.data_ptr() if k_weight is not None else None
    n.eps = float(eps)
    n._keep = (q_weight, k_weight)  # raw pointers: keep the tensors alive
    return n


def out_shape(q, v):
    """torch shape of dst for q (B, H, Lq, Dk) and v (Bk, Hkv, Lk, Dv)."""
    return (q.shape[0], q.shape[2], q.shape[1], v.shape[3])


# ---------------------------------------------------------------------------
# operator entry points
# ---------------------------------------------------------------------------

def supports(q, k, v, mask=None, dst=None, scale=1.0, max_bias=0.0, logit_softcap=0.0, rope=None, norm=None):
    """(ok, reason): the kd_fa_supports / kd_fa_rope_supports /
    kd_fa_dit_supports (with ``norm``) answer."""
    torch = _torch()
    if dst is None:
        dst = torch.empty(out_shape(q, v), dtype=torch.float32, device=q.device)
    d = make_desc(q, k, v, mask, dst, scale, max_bias, logit_softcap)
    reason = ctypes.c_int(0)
    if norm is not None:
        ok = _lib().kd_fa_dit_supports(ctypes.byref(d), ctypes.byref(rope) if rope is not None else None,
                                       ctypes.byref(norm), ctypes.byref(reason))
    elif rope is None:
        ok = _lib().kd_fa_supports(ctypes.byref(d), ctypes.byref(reason))
    else:
        ok = _lib().kd_fa_rope_supports(ctypes.byref(d), ctypes.byref(rope), ctypes.byref(reason))
    return bool(ok), reason.value


def run_desc(desc: KdFaDesc, rope: KdFaRope | None = None, stream=None, workspace=None,
             norm: KdFaQkNorm | None = None) -> int:
    """Enqueue on `stream` (a torch.cuda.Stream, a raw handle, or None for
    torch's current stream).  With `workspace` (a tensor of at least
    workspace_size(desc) bytes) the RoPE call pre-rotates K into it
    (kd_fa_rope_run_ws); without RoPE the call is kd_fa_run_ws (a masked
    short-key node keeps its mask summary there, given
    workspace_size_full(desc) bytes).  With `norm` the call is
    kd_fa_dit_run.  Returns the status code."""
    torch = _torch()
    if stream is None:
        handle = torch.cuda.current_stream().cuda_stream
    elif isinstance(stream, int):
        handle = stream
    else:
        handle = stream.cuda_stream
    if norm is not None:
        wp, nbytes = None, 0
        if workspace is not None:
            wp, nbytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        return _lib().kd_fa_dit_run(ctypes.byref(desc), ctypes.byref(rope) if rope is not None else None,
                                    ctypes.byref(norm), ctypes.c_void_p(wp), nbytes, ctypes.c_void_p(handle))
    if rope is None:
        if workspace is not None:
            nbytes = workspace.numel() * workspace.element_size()
            return _lib().kd_fa_run_ws(ctypes.byref(desc), ctypes.c_void_p(workspace.data_ptr()), nbytes,
                                       ctypes.c_void_p(handle))
        return _lib().kd_fa_run(ctypes.byref(desc), ctypes.c_void_p(handle))
    if workspace is not None:
        nbytes = workspace.numel() * workspace.element_size()
        return _lib().kd_fa_rope_run_ws(ctypes.byref(desc), ctypes.byref(rope),
                                        ctypes.c_void_p(workspace.data_ptr()), nbytes,
                                        ctypes.c_void_p(handle))
    return _lib().kd_fa_rope_run(ctypes.byref(desc), ctypes.byref(rope), ctypes.c_void_p(handle))


def run_static(desc: KdFaDesc, rope: KdFaRope | None = None, norm: KdFaQkNorm | None = None, stream=None) -> int:
    """kd_fa_dit_run_static: kd_fa_dit_run with the K workspace in the
    library's static device array (no allocation by anyone).  Returns the
    status code."""
    torch = _torch()
    if stream is None:
        handle = torch.cuda.current_stream().cuda_stream
    elif isinstance(stream, int):
        handle = stream
    else:
        handle = stream.cuda_stream
    return _lib().kd_fa_dit_run_static(ctypes.byref(desc), ctypes.byref(rope) if rope is not None else None,
                                       ctypes.byref(norm) if norm is not None else None, ctypes.c_void_p(handle))


def workspace_size(desc: KdFaDesc) -> int:
    """kd_fa_rope_workspace_size: bytes of workspace kd_fa_rope_run_ws needs
    (the rotated K, and the cast V when V is float32)."""
    return int(_lib().kd_fa_rope_workspace_size(ctypes.byref(desc)))


def workspace_size_full(desc: KdFaDesc, rope: KdFaRope | None = None, norm: KdFaQkNorm | None = None) -> int:
    """kd_fa_workspace_size: bytes of workspace the node can use (the
    transformed K, the cast V, then the mask summary of a masked short-key
    node)."""
    return int(_lib().kd_fa_workspace_size(ctypes.byref(desc), ctypes.byref(rope) if rope is not None else None,
                                           ctypes.byref(norm) if norm is not None else None))


def flash_attn_ext(q, k, v, mask=None, scale=None, max_bias=0.0, logit_softcap=0.0,
                   dst=None, rope=None, stream=None, workspace=None, norm=None, out_dtype=None, cast_type=0):
    """GGML_OP_FLASH_ATTN_EXT on the GPU; returns dst (B, Lq, H, Dv).

    ``rope`` is a KdFaRope (rope_table / rope_axes) to rotate Q and K on load;
    ``norm`` a KdFaQkNorm (qk_norm) to RMS-normalise them first
    (kd_fa_dit_run).  dst defaults to float32 (the node's type); ``out_dtype``
    torch.bfloat16 / torch.float16 stores O rounded instead.  float32 K / V
    (with a workspace, through ``norm`` or ``rope``) are cast to ``cast_type``
    by the pre-pass.  Raises KdFaError on any non-zero status (nothing is
    enqueued then)."""
    torch = _torch()
    if scale is None:
        scale = 1.0 / float(q.shape[-1]) ** 0.5
    if dst is None:
        dst = torch.empty(out_shape(q, v), dtype=out_dtype or torch.float32, device=q.device)
    d = make_desc(q, k, v, mask, dst, scale, max_bias, logit_softcap, cast_type=cast_type)
    st = run_desc(d, rope, stream, workspace, norm)
    if st != OK:
        name = "kd_fa_dit_run" if norm is not None else "kd_fa_rope_run" if rope is not None else "kd_fa_run"
        raise KdFaError(st, name)
    return dst


# ---------------------------------------------------------------------------
# RoPE tables (host side, src/rope.hpp:23-102)
# ---------------------------------------------------------------------------

def _fptr(a):
    return ctypes.cast(a.ctypes.data, ctypes.POINTER(ctypes.c_float))


def visual_rope_table(T, Hp, Wp, axes=(32, 48, 48), scale_factor=(1.0, 2.0, 2.0), theta=10000.0):
    """numpy float32 (T*Hp*Wp, sum(axes)): rope::compute_visual_rope."""
    import numpy as np
    out = np.empty((T * Hp * Wp, sum(axes)), dtype=np.float32)
    ax = (ctypes.c_int * 3)(*axes)
    sf = (ctypes.c_float * 3)(*scale_factor)
    st = _lib().kd_fa_rope_visual_table(T, Hp, Wp, ax, sf, theta, _fptr(out))
    if st != OK:
        raise KdFaError(st, "kd_fa_rope_visual_table")
    return out


def axes_rope_table(T, Hp, Wp, axes=(32, 48, 48), scale_factor=(1.0, 2.0, 2.0), theta=10000.0):
    """numpy float32 factorised table for KD_FA_ROPE_AXES."""
    import numpy as np
    ax = (ctypes.c_int * 3)(*axes)
    n = _lib().kd_fa_rope_axes_size(T, Hp, Wp, ax)
    if n == 0:
        raise KdFaError(ERR_ROPE, "kd_fa_rope_axes_size")
    out = np.empty(n, dtype=np.float32)
    sf = (ctypes.c_float * 3)(*scale_factor)
    st = _lib().kd_fa_rope_axes_fill(T, Hp, Wp, ax, sf, theta, _fptr(out))
    if st != OK:
        raise KdFaError(st, "kd_fa_rope_axes_fill")
    return out


def text_rope_table(L, D=128, theta=10000.0):
    """numpy float32 (L, D): rope::compute_text_rope."""
    import numpy as np
    out = np.empty((L, D), dtype=np.float32)
    st = _lib().kd_fa_rope_text_table(L, D, theta, _fptr(out))
    if st != OK:
        raise KdFaError(st, "kd_fa_rope_text_table")
    return out
