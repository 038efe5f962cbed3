"""The C ABI of libkd_fa.so, host side only (no GPU needed): the library
loads, exports every function include/kd_fa.h declares, its structs have
the layout ctypes assumes, and kd_fa_supports gives the answers that
ggml_backend_supports_op would need (src/core/ops.hpp:179) -- accepting the
node as the reference builds it and rejecting what the kernel cannot run,
with the reason code, without touching a GPU."""
import ctypes
import os
import subprocess
import tempfile

import pytest
import torch

import kd_fa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_header_symbol():
    lib = kd_fa.lib()
    syms = kd_fa.header_symbols()
    assert len(syms) >= 10
    for s in syms:
        assert hasattr(lib, s), s
    out = subprocess.run(["nm", "-D", "--defined-only", kd_fa.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert set(syms) <= exported


def test_struct_layout_matches_c():
    src = r"""
    #include <stdio.h>
    #include <stddef.h>
    #include "kd_fa.h"
    int main(void) {
      printf("%zu %zu %zu %zu %zu\n", sizeof(kd_fa_tensor), offsetof(kd_fa_tensor, ne),
             offsetof(kd_fa_tensor, nb), offsetof(kd_fa_tensor, data), sizeof(kd_fa_desc));
      printf("%zu %zu %zu %zu %zu\n", offsetof(kd_fa_desc, sinks), offsetof(kd_fa_desc, dst),
             offsetof(kd_fa_desc, scale), offsetof(kd_fa_desc, prec), sizeof(kd_fa_rope));
      printf("%zu %zu %zu %zu\n", offsetof(kd_fa_rope, table), offsetof(kd_fa_rope, axes_data),
             offsetof(kd_fa_rope, grid), offsetof(kd_fa_rope, axes));
      printf("%zu %zu %zu\n", sizeof(kd_fa_qk_norm), offsetof(kd_fa_qk_norm, k_weight),
             offsetof(kd_fa_qk_norm, eps));
      return 0;
    }
    """
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        with open(c, "w") as f:
            f.write(src)
        subprocess.run(["gcc", "-std=c99", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        got = [int(x) for x in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    T, Dd, R = kd_fa.KdFaTensor, kd_fa.KdFaDesc, kd_fa.KdFaRope
    want = [ctypes.sizeof(T), T.ne.offset, T.nb.offset, T.data.offset, ctypes.sizeof(Dd),
            Dd.sinks.offset, Dd.dst.offset, Dd.scale.offset, Dd.prec.offset, ctypes.sizeof(R),
            R.table.offset, R.axes_data.offset, R.grid.offset, R.axes.offset,
            ctypes.sizeof(kd_fa.KdFaQkNorm), kd_fa.KdFaQkNorm.k_weight.offset, kd_fa.KdFaQkNorm.eps.offset]
    assert got == want


def test_header_compiles_as_c_and_cxx():
    for cc, std in (("gcc", "-std=c99"), ("g++", "-std=c++11")):
        with tempfile.TemporaryDirectory() as d:
            c = os.path.join(d, "t.c")
            with open(c, "w") as f:
                f.write('#include "kd_fa.h"\nint main(void){return kd_fa_version() < 0;}\n')
            subprocess.run([cc, std, "-Wall", "-Werror", "-fsyntax-only", "-I", os.path.join(ROOT, "include"),
                            "-x", "c" if cc == "gcc" else "c++", c], check=True)


def test_version_and_strerror():
    lib = kd_fa.lib()
    assert lib.kd_fa_version() >= 100
    for code in range(0, -10, -1):
        assert lib.kd_fa_strerror(code)
    assert b"unknown" in lib.kd_fa_strerror(-99)


# ----------------------------------------------------------------------------
# kd_fa_supports: the node as the reference builds it, and rejections
# ----------------------------------------------------------------------------

def _node(B=1, H=4, Lq=64, Lk=48, kt=torch.float16, qt=torch.float32, mask=False, Hkv=None):
    """ops.hpp:122-177 as the reference calls it: q F32 [D, Lq, H], K/V F16."""
    Hkv = H if Hkv is None else Hkv
    q = torch.zeros((B, H, Lq, 128), dtype=qt)
    k = torch.zeros((B, Hkv, Lk, 128), dtype=kt)
    v = torch.zeros((B, Hkv, Lk, 128), dtype=kt)
    m = torch.zeros((B, 1, Lq, Lk), dtype=torch.float16) if mask else None
    dst = torch.zeros((B, Lq, H, 128), dtype=torch.float32)
    return q, k, v, m, dst


def _sup(q, k, v, m, dst, **kw):
    return kd_fa.supports(q, k, v, m, dst, scale=kw.pop("scale", 0.08838834764831845), **kw)


@pytest.mark.parametrize("qt,kt", [(torch.float32, torch.float16), (torch.bfloat16, torch.bfloat16),
                                   (torch.float16, torch.float16), (torch.float32, torch.bfloat16)])
def test_accepts_reference_node(qt, kt):
    assert _sup(*_node(qt=qt, kt=kt)) == (True, 0)
    assert _sup(*_node(qt=qt, kt=kt, mask=True, B=2)) == (True, 0)
    assert _sup(*_node(qt=qt, kt=kt, H=8, Hkv=2)) == (True, 0)


def test_vae_node_d512():
    """The 2-D VAE attention block's node (vae.hpp:60-101: one head, D = 512,
    Q F32, K/V F16) is accepted plain; a mask, RoPE or RMSNorm weights with
    D = 512 are not, nor any D other than 128 and 512."""
    def node(D, Lq=64, Lk=48, B=1, H=1):
        q = torch.zeros((B, H, Lq, D), dtype=torch.float32)
        k = torch.zeros((B, H, Lk, D), dtype=torch.float16)
        v = torch.zeros((B, H, Lk, D), dtype=torch.float16)
        dst = torch.zeros((B, Lq, H, D), dtype=torch.float32)
        return q, k, v, dst
    q, k, v, dst = node(512)
    assert _sup(q, k, v, None, dst, scale=512 ** -0.5) == (True, 0)
    assert _sup(*[t.to(torch.bfloat16) if t is not q and t is not dst else t for t in (q, k, v)], None, dst) == (True, 0)
    assert _sup(q, k, v, None, dst.half()) == (True, 0)
    assert _sup(q, k, v, torch.zeros((1, 1, 64, 48), dtype=torch.float16), dst) == (False, kd_fa.ERR_SHAPE)
    buf = torch.zeros(4096, dtype=torch.float32)
    assert _sup(q, k, v, None, dst, rope=kd_fa.rope_axes(buf, (3, 4, 5), (32, 48, 48))) == (False, kd_fa.ERR_ROPE)
    w = torch.ones(512, dtype=torch.float32)
    assert _sup(q, k, v, None, dst, norm=kd_fa.qk_norm(w, None)) == (False, kd_fa.ERR_ROPE)
    for D in (64, 256, 384, 1024):
        assert _sup(*node(D)[:3], None, node(D)[3]) == (False, kd_fa.ERR_SHAPE)


def test_rejections_carry_reason():
    q, k, v, m, dst = _node()
    assert _sup(q[..., :64], k[..., :64], v[..., :64], None, dst[..., :64]) == (False, kd_fa.ERR_SHAPE)
    assert _sup(q, k, v, m, dst, max_bias=8.0) == (False, kd_fa.ERR_PARAM)
    assert _sup(q, k, v, m, dst, logit_softcap=30.0) == (False, kd_fa.ERR_PARAM)
    assert _sup(q, k, v, m, dst, scale=float("nan")) == (False, kd_fa.ERR_PARAM)
    # attention sinks (newer ggml's src[4], never set by ops.hpp:176): refused
    d = kd_fa.make_desc(q, k, v, m, dst, 0.1)
    sinks = torch.zeros(4, dtype=torch.float32)
    d.sinks = kd_fa.view(sinks)
    reason = ctypes.c_int(0)
    assert kd_fa.lib().kd_fa_supports(ctypes.byref(d), ctypes.byref(reason)) == 0
    assert reason.value == kd_fa.ERR_PARAM
    assert kd_fa.lib().kd_fa_run(ctypes.byref(d), None) == kd_fa.ERR_PARAM
    assert _sup(q, k.float(), v.float(), m, dst) == (False, kd_fa.ERR_TYPE)          # F32 K
    assert _sup(q, k, v.to(torch.bfloat16), m, dst) == (False, kd_fa.ERR_TYPE)       # V type != K type
    assert _sup(q, k, v, m, dst.half()) == (True, 0)                                 # F16 dst: a fused cast
    assert _sup(q, k, v, m, dst.bfloat16()) == (True, 0)                             # BF16 dst
    d = kd_fa.make_desc(q, k, v, m, dst, 0.1)
    d.dst.type = 8                                                                   # a quantised type
    reason = ctypes.c_int(0)
    assert kd_fa.lib().kd_fa_supports(ctypes.byref(d), ctypes.byref(reason)) == 0 and reason.value == kd_fa.ERR_TYPE
    assert _sup(q, k, v, torch.zeros((1, 1, 64, 48)), dst) == (False, kd_fa.ERR_TYPE)  # F32 mask
    assert _sup(q, k, v, torch.zeros((1, 1, 63, 48), dtype=torch.float16), dst) == (False, kd_fa.ERR_SHAPE)
    assert _sup(q, k, v, torch.zeros((1, 1, 64, 47), dtype=torch.float16), dst) == (False, kd_fa.ERR_SHAPE)
    assert _sup(*_node(H=6, Hkv=4)) == (False, kd_fa.ERR_SHAPE)                       # H % Hkv
    assert _sup(q, k[:, :, :40], v, m, dst) == (False, kd_fa.ERR_SHAPE)               # Lk(K) != Lk(V)
    assert _sup(q, k, v, m, dst[:, :, :2]) == (False, kd_fa.ERR_SHAPE)                # dst heads
    # layouts: non-unit innermost stride, rows not 16-byte aligned
    kk = torch.zeros((1, 4, 48, 136), dtype=torch.float16)[..., :128]                  # 272-byte rows
    assert _sup(q, kk, v, m, dst) == (True, 0)
    kk = torch.zeros((1, 4, 48, 132), dtype=torch.float16)[..., :128]                  # 264-byte rows
    assert _sup(q, kk, v, m, dst) == (False, kd_fa.ERR_LAYOUT)
    kt = torch.zeros((1, 4, 128, 48), dtype=torch.float16).transpose(-1, -2)           # ne0 stride != 2
    assert _sup(q, kt, v, m, dst) == (False, kd_fa.ERR_LAYOUT)


def test_null_and_empty():
    lib = kd_fa.lib()
    r = ctypes.c_int(0)
    assert lib.kd_fa_supports(None, ctypes.byref(r)) == 0 and r.value == kd_fa.ERR_NULL
    assert lib.kd_fa_run(None, None) == kd_fa.ERR_NULL
    d = kd_fa.make_desc(*_node()[:3], None, _node()[4], 0.1)
    d.k.data = None
    assert lib.kd_fa_supports(ctypes.byref(d), ctypes.byref(r)) == 0 and r.value == kd_fa.ERR_NULL


def test_rope_descriptor_checks():
    q, k, v, m, dst = _node(Lq=60, Lk=60, qt=torch.bfloat16, kt=torch.bfloat16)
    good = kd_fa.rope_table(torch.zeros((60, 128)))
    assert _sup(q, k, v, None, dst, rope=good) == (True, 0)
    assert _sup(q, k, v, None, dst, rope=kd_fa.rope_table(torch.zeros((59, 128)))) == (False, kd_fa.ERR_ROPE)
    assert _sup(q, k, v, None, dst, rope=kd_fa.rope_table(torch.zeros((60, 64)))) == (False, kd_fa.ERR_ROPE)
    assert _sup(q, k, v, None, dst, rope=kd_fa.rope_table(torch.zeros((60, 128), dtype=torch.float16))) \
        == (False, kd_fa.ERR_ROPE)
    buf = torch.zeros(1024)
    assert _sup(q, k, v, None, dst, rope=kd_fa.rope_axes(buf, (3, 4, 5), (32, 48, 48))) == (True, 0)
    assert _sup(q, k, v, None, dst, rope=kd_fa.rope_axes(buf, (3, 4, 4), (32, 48, 48))) == (False, kd_fa.ERR_ROPE)
    assert _sup(q, k, v, None, dst, rope=kd_fa.rope_axes(buf, (3, 4, 5), (32, 48, 40))) == (False, kd_fa.ERR_ROPE)
    assert _sup(q, k, v, None, dst, rope=kd_fa.rope_axes(buf, (3, 4, 5), (36, 44, 48))) == (False, kd_fa.ERR_ROPE)
    bad = kd_fa.KdFaRope()
    bad.mode = 7
    assert _sup(q, k, v, None, dst, rope=bad) == (False, kd_fa.ERR_ROPE)
    none = kd_fa.KdFaRope()
    assert _sup(q, k, v, None, dst, rope=none) == (True, 0)


def test_run_validates_before_touching_the_device():
    """Invalid nodes return their error code from kd_fa_run with nothing
    enqueued, on any host (the device is only queried for valid nodes)."""
    q, k, v, m, dst = _node()
    d = kd_fa.make_desc(q, k, v, m, dst, 0.1, max_bias=1.0)
    assert kd_fa.lib().kd_fa_run(ctypes.byref(d), None) == kd_fa.ERR_PARAM
    d = kd_fa.make_desc(q[..., :64], k[..., :64], v[..., :64], m, dst[..., :64], 0.1)
    assert kd_fa.lib().kd_fa_run(ctypes.byref(d), None) == kd_fa.ERR_SHAPE


def test_no_keys_is_refused():
    """Lk = 0 is not supported (reason: shape), so that the caller keeps its
    fallback: the kernels clamp key rows to Lk - 1."""
    q, k, v, m, dst = _node(Lk=0, mask=True)
    for mask in (None, m):
        d = kd_fa.make_desc(q, k, v, mask, dst, 0.1)
        d.k.data = d.v.data = 16     # zero rows: any aligned non-null pointer, never read
        if mask is not None:
            d.mask.data = 16
        r = ctypes.c_int(0)
        assert kd_fa.lib().kd_fa_supports(ctypes.byref(d), ctypes.byref(r)) == 0 and r.value == kd_fa.ERR_SHAPE
        assert kd_fa.lib().kd_fa_run(ctypes.byref(d), None) == kd_fa.ERR_SHAPE


def test_empty_query_is_a_no_op():
    q, k, v, m, dst = _node(Lq=0)
    d = kd_fa.make_desc(q, k, v, None, dst, 0.1)
    d.q.data = 16        # zero rows: any aligned non-null pointer, never read
    d.dst.data = 16
    assert kd_fa.lib().kd_fa_run(ctypes.byref(d), None) == kd_fa.OK


def test_workspace_size_and_null_workspace():
    q, k, v, m, dst = _node(B=2, H=8, Lq=60, Lk=60, qt=torch.bfloat16, kt=torch.bfloat16, Hkv=2)
    d = kd_fa.make_desc(q, k, v, None, dst, 0.1)
    assert kd_fa.workspace_size(d) == 128 * 60 * 2 * 2 * 2
    bad = kd_fa.make_desc(q[..., :64], k[..., :64], v[..., :64], None, dst[..., :64], 0.1)
    assert kd_fa.workspace_size(bad) == 0
    rope = kd_fa.rope_table(torch.zeros((60, 128)))
    assert kd_fa.lib().kd_fa_rope_run_ws(ctypes.byref(d), ctypes.byref(rope), None, 0, None) == kd_fa.ERR_NULL


def test_full_workspace_size_holds_k_then_mask_summary():
    """kd_fa_workspace_size: the transformed K when K is transformed, then
    (256-byte aligned) 4 bytes per mask batch, mask head and 32 query rows
    for a masked node with at most 256 keys; nothing else."""
    q, k, v, m, dst = _node(B=2, H=8, Lq=100, Lk=77, qt=torch.bfloat16, kt=torch.bfloat16, mask=True)
    m = torch.zeros((2, 1, 100, 80), dtype=torch.float16)       # rows padded to whole 8-key chunks
    d = kd_fa.make_desc(q, k, v, m, dst, 0.1)
    words = 2 * 1 * ((100 + 31) // 32)
    assert kd_fa.workspace_size_full(d) == 4 * words
    m8 = torch.zeros((1, 8, 100, 80), dtype=torch.float16)      # per-head mask, batch broadcast
    assert kd_fa.workspace_size_full(kd_fa.make_desc(q, k, v, m8, dst, 0.1)) == 4 * 8 * ((100 + 31) // 32)
    wk = torch.ones(128)
    norm = kd_fa.qk_norm(wk, wk)
    kbytes = 128 * 77 * 8 * 2 * 2
    assert kd_fa.workspace_size_full(d, norm=norm) == (kbytes + 255) // 256 * 256 + 4 * words
    # no mask: K only (or nothing); a mask with more than 256 keys: K only
    nm = kd_fa.make_desc(q, k, v, None, dst, 0.1)
    assert kd_fa.workspace_size_full(nm) == 0
    assert kd_fa.workspace_size_full(nm, norm=norm) == kbytes
    rope = kd_fa.rope_table(torch.zeros((100, 128)))
    assert kd_fa.workspace_size_full(nm, rope=rope) == kbytes
    ql, kl, vl, _, dl = _node(B=1, H=2, Lq=64, Lk=300, qt=torch.bfloat16, kt=torch.bfloat16)
    ml = torch.zeros((1, 1, 64, 304), dtype=torch.float16)
    assert kd_fa.workspace_size_full(kd_fa.make_desc(ql, kl, vl, ml, dl, 0.1)) == 0
    # an invalid node uses none
    bad = kd_fa.make_desc(q[..., :64], k[..., :64], v[..., :64], None, dst[..., :64], 0.1)
    assert kd_fa.workspace_size_full(bad) == 0


def test_vae_node_workspace_is_the_key_split():
    """The D = 512 node takes a workspace for its key split when fewer than
    512 blocks of 32 query rows run (two workgroups per CU) and there are at
    least four key tiles: 4 ranges at 4,096 tokens, 8 at 1,024, 2 at 8,192,
    none at 16,384; 2,056 bytes per query row and range."""
    def size(Lq, Lk, H=1, B=1):
        q = torch.zeros((B, H, Lq, 512))
        k = torch.zeros((B, H, Lk, 512), dtype=torch.float16)
        dst = torch.zeros((B, Lq, H, 512))
        return kd_fa.workspace_size_full(kd_fa.make_desc(q, k, k, None, dst, 0.04))
    assert size(4096, 4096) == 4 * 4096 * 2056
    assert size(8192, 8192) == 2 * 8192 * 2056
    assert size(1024, 1024) == 8 * 1024 * 2056
    assert size(300, 1000) == 8 * 300 * 2056          # 32 tiles / 8 ranges of 4
    assert size(64, 130) == 5 * 64 * 2056             # five tiles, five ranges
    assert size(64, 96) == 0                          # three tiles: the merge would cost more
    assert size(16384, 16384) == 0                    # 512 blocks fill the chip


def test_run_ws_checks_workspace_alignment_before_device_work():
    """kd_fa_run_ws refuses a workspace that is not 16-byte aligned
    (KD_FA_ERR_LAYOUT) before touching the device; an invalid node keeps its
    own reason."""
    q, k, v, m, dst = _node(B=1, H=2, Lq=64, Lk=64, qt=torch.bfloat16, kt=torch.bfloat16, mask=True)
    d = kd_fa.make_desc(q, k, v, m, dst, 0.1)
    assert kd_fa.lib().kd_fa_run_ws(ctypes.byref(d), ctypes.c_void_p(4104), 4096, None) == kd_fa.ERR_LAYOUT
    d = kd_fa.make_desc(q, k, v, m, dst, 0.1, max_bias=1.0)
    assert kd_fa.lib().kd_fa_run_ws(ctypes.byref(d), ctypes.c_void_p(4096), 4096, None) == kd_fa.ERR_PARAM


def test_norm_descriptor_checks():
    q, k, v, m, dst = _node(Lq=60, Lk=60, qt=torch.float32, kt=torch.bfloat16)
    w = torch.ones(132)
    sup = kd_fa.lib().kd_fa_dit_supports

    def ask(norm, rope=None):
        d = kd_fa.make_desc(q, k, v, None, dst, 0.1)
        reason = ctypes.c_int(0)
        ok = sup(ctypes.byref(d), ctypes.byref(rope) if rope is not None else None,
                 ctypes.byref(norm) if norm is not None else None, ctypes.byref(reason))
        return bool(ok), reason.value

    assert ask(None) == (True, 0)
    assert ask(kd_fa.qk_norm(w[:128], w[:128])) == (True, 0)
    assert ask(kd_fa.qk_norm(None, w[:128], 1e-5)) == (True, 0)
    assert ask(kd_fa.qk_norm(w[:128], None), kd_fa.rope_table(torch.zeros((60, 128)))) == (True, 0)
    assert ask(kd_fa.qk_norm(w[1:129], w[:128])) == (False, kd_fa.ERR_LAYOUT)     # 4-byte aligned weight
    assert ask(kd_fa.qk_norm(w[:128], w[:128], float("nan"))) == (False, kd_fa.ERR_ROPE)
    assert ask(kd_fa.qk_norm(w[:128], w[:128], -1.0)) == (False, kd_fa.ERR_ROPE)


def test_f32_k_v_supports_agrees_with_run():
    """kd_fa_dit_supports answers for the workspace form, whose pre-pass
    casts an F32 K and V (the projection outputs ops::attention receives,
    src/core/ops.hpp:167-169): it accepts them with or without a K transform,
    and kd_fa_dit_run without a workspace names the missing buffer.  The node
    itself (kd_fa_supports, kd_fa_run, kd_fa_rope_run) keeps 16-bit K and V.
    All answers come before any device work, so they are checked here on the
    host."""
    q, k, v, m, dst = _node(Lq=60, Lk=60, qt=torch.float32, kt=torch.bfloat16)
    w = torch.ones(128)
    lib = kd_fa.lib()
    table = kd_fa.rope_table(torch.zeros((60, 128)))

    def ask(kk, vv, rope, norm, cast_type=0):
        d = kd_fa.make_desc(q, kk, vv, None, dst, 0.1, cast_type=cast_type)
        reason = ctypes.c_int(0)
        ok = lib.kd_fa_dit_supports(ctypes.byref(d), ctypes.byref(rope) if rope is not None else None,
                                    ctypes.byref(norm) if norm is not None else None, ctypes.byref(reason))
        run = lib.kd_fa_dit_run(ctypes.byref(d), ctypes.byref(rope) if rope is not None else None,
                                ctypes.byref(norm) if norm is not None else None, None, 0, None)
        return bool(ok), reason.value, run

    k32, v32 = k.float(), v.float()
    for kk, vv in ((k32, v), (k, v32), (k32, v32)):
        assert ask(kk, vv, None, None) == (True, 0, kd_fa.ERR_NULL)
        assert ask(kk, vv, table, None) == (True, 0, kd_fa.ERR_NULL)
        assert ask(kk, vv, None, kd_fa.qk_norm(None, w)) == (True, 0, kd_fa.ERR_NULL)
        assert ask(kk, vv, None, None, cast_type=kd_fa.TYPE_BF16) == (True, 0, kd_fa.ERR_NULL)
        # the cast goes to a 16-bit type only
        assert ask(kk, vv, None, None, cast_type=kd_fa.TYPE_F32 + 7)[:2] == (False, kd_fa.ERR_TYPE)
        # the node and its no-workspace forms: 16-bit K and V
        d = kd_fa.make_desc(q, kk, vv, None, dst, 0.1)
        assert _sup(q, kk, vv, None, dst) == (False, kd_fa.ERR_TYPE)
        assert lib.kd_fa_run(ctypes.byref(d), None) == kd_fa.ERR_TYPE
        assert lib.kd_fa_rope_run(ctypes.byref(d), ctypes.byref(table), None) == kd_fa.ERR_TYPE
    # K and V of different 16-bit types stay refused; cast_type is ignored then
    assert ask(k, v.half(), None, None)[:2] == (False, kd_fa.ERR_TYPE)
    assert ask(k, v, None, None, cast_type=99)[:2] == (True, 0)
    # the D = 512 node has no cast pass
    q5 = torch.zeros((1, 1, 64, 512), dtype=torch.float32)
    k5 = torch.zeros((1, 1, 64, 512), dtype=torch.float32)
    d5 = kd_fa.make_desc(q5, k5, k5, None, torch.zeros((1, 64, 1, 512)), 0.1)
    reason = ctypes.c_int(0)
    assert lib.kd_fa_dit_supports(ctypes.byref(d5), None, None, ctypes.byref(reason)) == 0
    assert reason.value == kd_fa.ERR_TYPE


def test_cast_workspace_sizes():
    """Workspace layout of the cast operands: the transformed K, then (at a
    256-byte boundary) the cast V, then the mask summary; an F32 K with no
    transform still takes its K part (the cast)."""
    lib = kd_fa.lib()
    B, H, Lq, Lk = 2, 4, 64, 77
    q = torch.zeros((B, H, Lq, 128), dtype=torch.float32)
    k16 = torch.zeros((B, H, Lk, 128), dtype=torch.bfloat16)
    k32, v32 = k16.float(), k16.float()
    dst = torch.zeros((B, Lq, H, 128), dtype=torch.float32)
    kb = B * H * Lk * 256
    part = (kb + 255) // 256 * 256
    m = torch.zeros((B, 1, Lq, 80), dtype=torch.float16)
    summary = 4 * B * 1 * ((Lq + 31) // 32)

    def full(kk, vv, mask=None, norm=None):
        d = kd_fa.make_desc(q, kk, vv, mask, dst, 0.1)
        return kd_fa.workspace_size_full(d, None, norm)

    def rope_ws(kk, vv):
        return kd_fa.workspace_size(kd_fa.make_desc(q, kk, vv, None, dst, 0.1))

    assert full(k16, k16) == 0
    assert full(k32, k16) == kb
    assert full(k16, v32) == kb
    assert full(k32, v32) == part + kb
    assert full(k16, k16, norm=kd_fa.qk_norm(None, torch.ones(128))) == kb
    assert full(k32, v32, mask=m) == part + part + summary
    assert full(k16, k16, mask=m) == summary
    assert rope_ws(k16, k16) == kb
    assert rope_ws(k16, v32) == part + kb
    assert rope_ws(k32, v32) == part + kb
    assert lib.kd_fa_abi_version() == kd_fa.ABI_VERSION


def test_routing_hook_round_trips():
    """kd_fa_set_routing is process-wide and returns the previous flags; the
    context manager restores them."""
    lib = kd_fa.lib()
    assert lib.kd_fa_set_routing(kd_fa.ROUTE_DEFAULT) == kd_fa.ROUTE_DEFAULT
    with kd_fa.routing(kd_fa.ROUTE_NO_W64 | kd_fa.ROUTE_NO_XRES):
        assert lib.kd_fa_set_routing(kd_fa.ROUTE_NO_W64 | kd_fa.ROUTE_NO_XRES) == \
            kd_fa.ROUTE_NO_W64 | kd_fa.ROUTE_NO_XRES
    assert lib.kd_fa_set_routing(kd_fa.ROUTE_DEFAULT) == kd_fa.ROUTE_DEFAULT


def test_product_reads_no_environment():
    """Kernel choice is a function of the node (and the routing hook) only:
    the shipped library and the loop generator read no environment."""
    import re
    csrc = os.path.join(ROOT, "kandinsky.cpp_amd", "csrc")
    for name in os.listdir(csrc):
        if name.endswith((".cpp", ".hip", ".h", ".py")):
            with open(os.path.join(csrc, name)) as f:
                text = f.read()
            assert not re.search(r"\bgetenv\b|os\.environ", text), name


def test_static_entry_point_refuses_oversize_f32_before_device_work():
    """kd_fa_dit_run_static checks the transformed K and cast V against its
    static scratch (KD_FA_STATIC_SCRATCH_BYTES) on the host, before any
    device call: an F32 K or V one row over the limit is refused with
    KD_FA_ERR_SCRATCH (their cast needs the workspace), an invalid node with
    its own reason.  (A 16-bit K over the limit runs without the workspace:
    a GPU test covers it.)"""
    lib = kd_fa.lib()
    L = kd_fa.STATIC_SCRATCH_BYTES // (128 * 2) + 1          # one K row over
    q = torch.zeros((1, 1, 4, 128), dtype=torch.bfloat16)
    k = torch.zeros((1, 1, L, 128), dtype=torch.bfloat16)
    dst = torch.zeros((1, 4, 1, 128), dtype=torch.float32)
    d = kd_fa.make_desc(q, k, k, None, dst, 0.1)
    tab = torch.zeros((L, 128))
    rope = kd_fa.rope_table(tab)
    assert kd_fa.workspace_size(d) == kd_fa.STATIC_SCRATCH_BYTES + 256
    for kk, vv in ((k.float(), k), (k, k.float())):
        d32 = kd_fa.make_desc(q, kk, vv, None, dst, 0.1)
        assert lib.kd_fa_dit_run_static(ctypes.byref(d32), ctypes.byref(rope), None, None) == kd_fa.ERR_SCRATCH
    bad = kd_fa.make_desc(q, k, k, None, dst, 0.1, max_bias=1.0)
    assert lib.kd_fa_dit_run_static(ctypes.byref(bad), ctypes.byref(rope), None, None) == kd_fa.ERR_PARAM
    assert b"static scratch" in lib.kd_fa_strerror(kd_fa.ERR_SCRATCH)


def test_python_constants_equal_the_header():
    """Every KD_FA_<NAME> = <value> enumerator and KD_FA_ABI_VERSION of
    include/kd_fa.h has the same value as kd_fa.<NAME> (the ctypes mirror),
    and the mirror defines no routing flag the header lacks."""
    import re
    text = open(kd_fa.HEADER_PATH).read()
    enums = {m.group(1): int(m.group(2)) for m in re.finditer(r"\bKD_FA_([A-Z0-9_]+)\s*=\s*(-?\d+)", text)}
    assert len(enums) >= 25
    for name, value in enums.items():
        assert getattr(kd_fa, name) == value, name
    abi = re.search(r"#define\s+KD_FA_ABI_VERSION\s+(\d+)", text)
    assert abi and int(abi.group(1)) == kd_fa.ABI_VERSION
    mirrored = {n for n in dir(kd_fa) if n.startswith("ROUTE_")}
    assert mirrored == {n for n in enums if n.startswith("ROUTE_")}
