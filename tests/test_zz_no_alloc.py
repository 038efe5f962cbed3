"""kd_fa_dit_run_static, the allocation-free variant of kd_fa_dit_run: the
K workspace is the library's static device array, so the caller passes only
inputs and outputs.  Through the C ABI, its output must be bitwise equal to
kd_fa_dit_run's with a caller workspace -- the same kernels on the same
operands -- on consecutive calls whose second input is smaller than the
first (the array keeps the last call's contents), and on a node that
transforms no K (no workspace at all)."""
import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import AXES, D, SCALE_FACTOR, THETA, assert_parity, gather_rows, qkv, randn

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _pair(q, k, v, rope, norm, out_dtype=torch.float32):
    """(static entry point output, caller-workspace entry point output)."""
    B, H, Lq = q.shape[0], q.shape[1], q.shape[2]
    out_s = torch.full((B, Lq, H, v.shape[3]), float("nan"), dtype=out_dtype, device=DEV)
    out_w = torch.full_like(out_s, float("nan"))
    ds = kd_fa.make_desc(q, k, v, None, out_s, 1.0 / D ** 0.5)
    dw = kd_fa.make_desc(q, k, v, None, out_w, 1.0 / D ** 0.5)
    st = kd_fa.run_static(ds, rope, norm)
    assert st == kd_fa.OK, kd_fa.lib().kd_fa_strerror(st)
    ws = torch.empty(max(kd_fa.workspace_size(dw), 16), dtype=torch.uint8, device=DEV)
    st = kd_fa.run_desc(dw, rope, None, ws, norm if norm is not None else kd_fa.qk_norm(None, None))
    assert st == kd_fa.OK
    torch.cuda.synchronize()
    return out_s, out_w


def _rope(T, Hp, Wp):
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    return table, kd_fa.rope_table(torch.from_numpy(table).to(DEV))


def test_static_scratch_equals_caller_workspace_two_calls():
    _need_gpu()
    # call 1: the DiT self-attention from the projections on -- Q and K F32,
    # V bf16, query/key RMSNorm, RoPE over a 4x16x16 grid, 8 heads
    _announce("static scratch call 1: [128,1024,8,1] q/k F32 norm+rope, v bf16")
    T, Hp, Wp, H = 4, 16, 16, 8
    L = T * Hp * Wp
    q = randn((1, H, L, D), torch.float32, 301).to(DEV)
    k = (randn((1, H, L, D), torch.float32, 302) * 2.0).to(DEV)
    v = randn((1, H, L, D), torch.bfloat16, 303).to(DEV)
    wq = (randn((D,), torch.float32, 304) * 0.3 + 1.0).to(DEV)
    wk = (randn((D,), torch.float32, 305) * 0.3 + 1.0).to(DEV)
    table, rope = _rope(T, Hp, Wp)
    norm = kd_fa.qk_norm(wq, wk, 1e-6)
    a, b = _pair(q, k, v, rope, norm)
    assert torch.equal(a, b)
    assert torch.isfinite(a).all()
    # call 2, smaller: the 1,280-token shape's neighbour at 2x8x8 tokens,
    # f16, RoPE only, 16-bit output
    _announce("static scratch call 2: [128,128,2,1] f16 rope, f16 out")
    T, Hp, Wp, H = 2, 8, 8, 2
    L = T * Hp * Wp
    qs, ks, vs = (t.to(DEV) for t in qkv(1, H, L, L, torch.float16, seed=306))
    table2, rope2 = _rope(T, Hp, Wp)
    a2, b2 = _pair(qs, ks, vs, rope2, None, torch.float16)
    assert torch.equal(a2, b2)
    ref = orc.fa_f64(qs.cpu(), ks.cpu(), vs.cpu(), rope=orc.rope_table(torch.from_numpy(table2)))
    assert_parity(gather_rows(a2.float(), np.arange(H * L), H, L), ref, "static call 2")


def test_static_scratch_c1_shape_and_plain_node():
    """The 1,280-token self-attention (K 10.5 MB, inside the array) and a
    node that transforms no K (it needs no workspace)."""
    _need_gpu()
    _announce("static scratch: C1 [128,1280,32,1] f16 rope; plain node")
    T, Hp, Wp = 5, 16, 16
    L = T * Hp * Wp
    q, k, v = (t.to(DEV) for t in qkv(1, 32, L, L, torch.float16, seed=1))
    _, rope = _rope(T, Hp, Wp)
    a, b = _pair(q, k, v, rope, None)
    assert torch.equal(a, b)
    a, b = _pair(q, k, v, None, None)
    assert torch.equal(a, b)


def test_static_scratch_k_over_the_limit_runs_without_it():
    """A 16-bit K whose transformed copy exceeds the static array (32 heads
    x 8,193 keys x 256 B = 64 MiB + 8 KiB) runs without a workspace (K
    transformed in staged groups or on load) and gives the caller-workspace
    call's bits."""
    _need_gpu()
    _announce("static scratch: [128,8193,32,1] bf16 rope, K over the array")
    L, H = 8193, 32
    q, k, v = (t.to(DEV) for t in qkv(1, H, L, L, torch.bfloat16, seed=311))
    table = kd_fa.text_rope_table(L, D)
    rope = kd_fa.rope_table(torch.from_numpy(table).to(DEV))
    d = kd_fa.make_desc(q, k, v, None, torch.empty((1, L, H, D), device=DEV), 1.0 / D ** 0.5)
    assert kd_fa.workspace_size(d) > kd_fa.STATIC_SCRATCH_BYTES
    a, b = _pair(q, k, v, rope, None)
    assert torch.equal(a, b)
    assert torch.isfinite(a).all()


def test_static_scratch_f32_k_and_v():
    """Q, K, V F32 (the projections ops::attention receives), K and V cast to
    F16 into the static array: the caller-workspace call's bits."""
    _need_gpu()
    _announce("static scratch: [128,1280,32,1] all F32, cast F16, rope")
    T, Hp, Wp = 5, 16, 16
    L = T * Hp * Wp
    q, k, v = (t.to(DEV) for t in qkv(1, 32, L, L, torch.float32, seed=312))
    _, rope = _rope(T, Hp, Wp)
    a, b = _pair(q, k, v, rope, kd_fa.qk_norm(None, None, 1e-6))
    assert torch.equal(a, b)
    assert torch.isfinite(a).all()
