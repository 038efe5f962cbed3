"""GPU parity of the gfx950 flash-attention hook against the CPU oracle.

Every case calls libkd_fa.so through its C ABI (kd_fa_run / kd_fa_rope_run)
and compares with the float64 textbook oracle on the same rounded operands
(gate: max-abs <= 2e-2 and cosine >= 0.9995); the deviation from the
restated ggml CPU algorithm is checked as well.  At the production shapes
the comparison uses sampled query rows: each output row depends only on its
own query row, so sampled rows are exact references.
"""
import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import (AXES, D, HEADS, SCALE_FACTOR, THETA, assert_parity, gather_rows,
                       metrics, padding_mask, qkv, sample_rows)

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _gpu(*ts):
    return [None if t is None else t.to(DEV) for t in ts]


def _run(q, k, v, mask=None, scale=None, rope=None):
    out = kd_fa.flash_attn_ext(q, k, v, mask=mask, scale=scale, rope=rope)
    torch.cuda.synchronize()
    return out


def _check_all_rows(q, k, v, mask=None, scale=None, rope_gpu=None, rope_cpu=None, what=""):
    qg, kg, vg, mg = _gpu(q, k, v, mask)
    out = _run(qg, kg, vg, mg, scale, rope_gpu)
    B, H, Lq = q.shape[0], q.shape[1], q.shape[2]
    ref = orc.fa_f64(q, k, v, mask=mask, scale=scale, rope=rope_cpu)
    got = gather_rows(out, np.arange(B * H * Lq), H, Lq)
    return assert_parity(got, ref, what), out


# ---------------------------------------------------------------------------
# small and ragged shapes, every row
# ---------------------------------------------------------------------------

SMALL = [
    # B, H, Hkv, Bk, Lq, Lk, kv dtype, q dtype, mask
    (1, 2, 2, 1, 128, 64, torch.bfloat16, torch.bfloat16, None),
    (1, 2, 2, 1, 100, 77, torch.float16, torch.float16, None),
    (2, 4, 2, 1, 130, 200, torch.bfloat16, torch.float32, "pad"),
    (1, 3, 1, 1, 33, 1, torch.float16, torch.float32, None),
    (2, 2, 2, 2, 257, 300, torch.float16, torch.bfloat16, "rand"),
    (1, 1, 1, 1, 5, 513, torch.bfloat16, torch.float16, "pad"),
]


@pytest.mark.parametrize("case", SMALL, ids=lambda c: f"B{c[0]}H{c[1]}kv{c[2]}Lq{c[4]}Lk{c[5]}{c[6]}{c[8]}")
def test_small_shapes(case):
    _need_gpu()
    B, H, Hkv, Bk, Lq, Lk, dt, qdt, mk = case
    _announce(f"small {case}")
    q, k, v = qkv(B, H, Lq, Lk, dt, seed=11, Hkv=Hkv, Bk=Bk, q_dtype=qdt)
    mask = None
    if mk == "pad":
        mask = padding_mask(B, Lq, Lk, [max(1, Lk // (b + 2)) for b in range(B)], pad_rows=3)
    elif mk == "rand":
        g = torch.Generator().manual_seed(5)
        mask = (torch.randn((B, 1, Lq, Lk), generator=g) * 2).to(torch.float16)
        mask[torch.rand((B, 1, Lq, Lk), generator=g) < 0.3] = float("-inf")
    m, out = _check_all_rows(q, k, v, mask, what=f"small {case}")
    ggml, _ = orc.fa_ggml(q, k, v, mask=mask)
    mg = metrics(out.cpu().double().numpy(), ggml.double().numpy())
    assert mg["max_abs"] <= 2e-2 and mg["cos"] >= 0.9995, mg


def test_fully_masked_rows_are_zero():
    _need_gpu()
    _announce("fully masked rows")
    B, H, Lq, Lk = 1, 2, 64, 96
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=3)
    mask = torch.zeros((1, 1, Lq, Lk), dtype=torch.float16)
    mask[:, :, ::3, :] = float("-inf")  # every third query sees no key
    qg, kg, vg, mg = _gpu(q, k, v, mask)
    out = _run(qg, kg, vg, mg).cpu()
    assert torch.all(out[:, ::3] == 0)
    ref = orc.fa_f64(q, k, v, mask=mask)
    assert_parity(gather_rows(out, np.arange(B * H * Lq), H, Lq), ref, "masked rows")


def test_single_valid_key_returns_its_value():
    _need_gpu()
    _announce("single valid key")
    B, H, Lq, Lk = 1, 1, 32, 64
    q, k, v = qkv(B, H, Lq, Lk, torch.float16, seed=4)
    mask = torch.full((1, 1, Lq, Lk), float("-inf"), dtype=torch.float16)
    j = torch.arange(Lq) % Lk
    mask[0, 0, torch.arange(Lq), j] = 0.0
    qg, kg, vg, mg = _gpu(q, k, v, mask)
    out = _run(qg, kg, vg, mg).cpu()
    expect = v[0, 0, j, :].float()
    assert torch.equal(out[0, :, 0, :], expect)


def test_strided_activation_views():
    """Q/K/V read straight from [D*H, L] activations viewed as [D, L, H]
    (no cont/permute pass, unlike ops.hpp:122-131)."""
    _need_gpu()
    _announce("strided views")
    L, H = 96, 4
    g = torch.Generator().manual_seed(9)
    act = [torch.randn((1, L, H, D), generator=g).to(torch.bfloat16) for _ in range(3)]
    q, k, v = [a.permute(0, 2, 1, 3) for a in act]  # (B, H, L, D) views, nb1 = H*D*2
    assert not q.is_contiguous()
    qg, kg, vg = [a.to(DEV).permute(0, 2, 1, 3) for a in act]
    out = _run(qg, kg, vg)
    ref = orc.fa_f64(q.contiguous(), k.contiguous(), v.contiguous())
    assert_parity(gather_rows(out, np.arange(H * L), H, L), ref, "strided")


@pytest.mark.parametrize("scale", [-0.0883883, 0.0, 0.5], ids=["neg", "zero", "large"])
def test_scale_values(scale):
    """Any finite scale: a negative one is applied as |scale| on -q."""
    _need_gpu()
    _announce(f"scale {scale}")
    q, k, v = qkv(1, 2, 70, 90, torch.bfloat16, seed=17)
    qg, kg, vg = _gpu(q, k, v)
    out = _run(qg, kg, vg, scale=scale)
    ref = orc.fa_f64(q, k, v, scale=scale)
    assert_parity(gather_rows(out, np.arange(2 * 70), 2, 70), ref, f"scale {scale}")


def test_deterministic():
    _need_gpu()
    _announce("determinism")
    q, k, v = _gpu(*qkv(2, 4, 300, 333, torch.bfloat16, seed=21))
    a = _run(q, k, v).clone()
    b = _run(q, k, v)
    assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# RoPE fusion
# ---------------------------------------------------------------------------

def _rot(x, table, dtype):
    """rope::apply in F32 by the oracle, rounded to dtype: x (B, H, L, D)."""
    xb = x.float().permute(0, 2, 1, 3).contiguous().numpy()  # (B, L, H, D)
    r = orc.rope_apply(xb, table[: x.shape[2]])
    return torch.from_numpy(r).permute(0, 2, 1, 3).contiguous().to(dtype)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_rope_fused_equals_prerotated(dt):
    """kd_fa_rope_run(q, k, v) == kd_fa_run(round(rot(q)), round(rot(k)), v), bitwise."""
    _need_gpu()
    _announce(f"rope fused vs prerotated {dt}")
    T, Hp, Wp = 3, 4, 6
    L = T * Hp * Wp
    q, k, v = qkv(1, 4, L, L, dt, seed=31, q_dtype=torch.float32)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    tab_g = torch.from_numpy(table).to(DEV)
    qg, kg, vg = _gpu(q, k, v)
    fused = _run(qg, kg, vg, rope=kd_fa.rope_table(tab_g)).clone()
    q2, k2 = _rot(q, table, dt), _rot(k, table, dt)
    plain = _run(*_gpu(q2, k2, v))
    assert torch.equal(fused, plain)
    ref = orc.fa_f64(q, k, v, rope=orc.rope_table(torch.from_numpy(table)))
    assert_parity(gather_rows(fused, np.arange(4 * L), 4, L), ref, "rope fused")


@pytest.mark.parametrize("mode", ["table", "axes"])
def test_rope_workspace_equals_fused(mode):
    """kd_fa_rope_run_ws (K rotated once into a workspace) == kd_fa_rope_run,
    bitwise, with GQA, batch broadcast, strided K and a partial last tile."""
    _need_gpu()
    _announce(f"rope workspace vs fused ({mode})")
    T, Hp, Wp = 3, 5, 7
    L = T * Hp * Wp                     # 105 tokens: partial 64-key tile
    B, H, Hkv = 2, 4, 2
    q, k, v = qkv(B, H, L, L, torch.bfloat16, seed=51, Hkv=Hkv, Bk=1, q_dtype=torch.float32)
    qg, vg = _gpu(q, v)
    kbig = torch.zeros((1, Hkv, L, D + 8), dtype=torch.bfloat16)
    kbig[..., :D] = k
    kg = kbig.to(DEV)[..., :D]          # 272-byte rows
    if mode == "table":
        tab = torch.from_numpy(kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)).to(DEV)
        rope = kd_fa.rope_table(tab)
    else:
        ax = torch.from_numpy(kd_fa.axes_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)).to(DEV)
        rope = kd_fa.rope_axes(ax, (T, Hp, Wp), AXES)
    fused = _run(qg, kg, vg, rope=rope).clone()
    d = kd_fa.make_desc(qg, kg, vg, None, torch.empty_like(fused), 1.0 / D ** 0.5)
    nbytes = kd_fa.workspace_size(d)
    assert nbytes == 128 * L * Hkv * 1 * 2
    ws = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=DEV)
    out = kd_fa.flash_attn_ext(qg, kg, vg, rope=rope, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out, fused)
    # the workspace holds the rotated K: equal to the oracle's rotation
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    assert torch.equal(ws.view(1, Hkv, L, D).cpu(), _rot(k, table, torch.bfloat16))
    small = torch.empty(nbytes // 2 - 8, dtype=torch.bfloat16, device=DEV)
    assert kd_fa.run_desc(d, rope, None, small) == kd_fa.ERR_LAYOUT


def test_rope_axes_equals_table():
    _need_gpu()
    _announce("rope axes vs table")
    T, Hp, Wp = 5, 16, 16
    L = T * Hp * Wp
    q, k, v = _gpu(*qkv(1, 2, L, L, torch.float16, seed=41))
    table = torch.from_numpy(kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)).to(DEV)
    axes = torch.from_numpy(kd_fa.axes_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)).to(DEV)
    a = _run(q, k, v, rope=kd_fa.rope_table(table)).clone()
    b = _run(q, k, v, rope=kd_fa.rope_axes(axes, (T, Hp, Wp), AXES))
    assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# the workload shapes
# ---------------------------------------------------------------------------

def test_c1_self_attention_full():
    """1,280-token self-attention, f16, RoPE grid 5x16x16: every row."""
    _need_gpu()
    _announce("C1 full: [128,1280,32,1] f16 rope 5x16x16")
    T, Hp, Wp = 5, 16, 16
    L = T * Hp * Wp
    q, k, v = qkv(1, HEADS, L, L, torch.float16, seed=1)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    tab_c = torch.from_numpy(table)
    m, out = _check_all_rows(q, k, v, rope_gpu=kd_fa.rope_table(tab_c.to(DEV)),
                             rope_cpu=orc.rope_table(tab_c), what="C1")
    print(f"[C1] vs f64: {m}", flush=True)
    ggml, _ = orc.fa_ggml(q, k, v, rope=orc.rope_table(tab_c), f16_vacc=True)
    mg = metrics(out.cpu().double().numpy(), ggml.double().numpy())
    print(f"[C1] vs ggml restatement (f16 V accumulator): {mg}", flush=True)
    assert mg["max_abs"] <= 2e-2 and mg["cos"] >= 0.9995


def test_c2_cross_attention_sampled():
    """Text cross-attention: Q 31,744 tokens, K/V 256, batch 2, mask 120/40."""
    _need_gpu()
    _announce("C2 sampled: Q [128,31744,32,2] KV [128,256,32,2] bf16 mask 120/40")
    B, Lq, Lk = 2, 31744, 256
    q = _rand_dev((B, HEADS, Lq, D), 2)
    k = _rand_dev((B, HEADS, Lk, D), 1002)
    v = _rand_dev((B, HEADS, Lk, D), 2002)
    mask = padding_mask(B, Lq, Lk, [120, 40], device=DEV)
    out = _run(q, k, v, mask)
    rows = sample_rows(B, HEADS, Lq, 64, seed=2)
    ref = orc.fa_f64(q.cpu(), k.cpu(), v.cpu(), mask=mask.cpu(), rows=rows)
    m = assert_parity(gather_rows(out, rows, HEADS, Lq), ref, "C2")
    print(f"[C2] {m}", flush=True)


def _rand_dev(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(shape, generator=g, device=DEV, dtype=torch.float32).to(dtype)


@pytest.mark.parametrize("cfg", [("C3", 2, 31, 3), ("C4", 1, 61, 4)], ids=lambda c: c[0])
def test_self_attention_production_sampled(cfg):
    """31,744-token (B=2) and 62,464-token (B=1) self-attention with fused
    3-D RoPE over a (T, 32, 32) grid, sampled rows."""
    _need_gpu()
    name, B, T, seed = cfg
    Hp = Wp = 32
    L = T * Hp * Wp
    _announce(f"{name} sampled: [128,{L},32,{B}] bf16 rope {T}x32x32")
    q = _rand_dev((B, HEADS, L, D), seed)
    k = _rand_dev((B, HEADS, L, D), seed + 1000)
    v = _rand_dev((B, HEADS, L, D), seed + 2000)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    tab_c = torch.from_numpy(table)
    out = _run(q, k, v, rope=kd_fa.rope_table(tab_c.to(DEV)))
    rows = sample_rows(B, HEADS, L, 64, seed=seed)
    ref = orc.fa_f64(q.cpu(), k.cpu(), v.cpu(), rope=orc.rope_table(tab_c), rows=rows)
    m = assert_parity(gather_rows(out, rows, HEADS, L), ref, name)
    print(f"[{name}] {m}", flush=True)


@pytest.mark.parametrize("with_norm", [False, True])
def test_cpp_ops_attention_mirror_on_gpu(tmp_path, with_norm):
    """kd::attention (C++ mirror of ops::attention) on the reference's
    activation layout q [C, Lq, N] F32, k/v [C, Lk, N] bf16, with the RoPE
    table (and the query/key RMSNorm, K through a workspace), run by the
    compiled driver kandinsky.cpp_amd/kd_attention_run."""
    import os
    import subprocess
    _need_gpu()
    exe = os.path.join(os.path.dirname(kd_fa.LIB_PATH), "kd_attention_run")
    if not os.path.exists(exe):
        pytest.fail("kd_attention_run is not built (make -C kandinsky.cpp_amd)")
    _announce("C++ ops::attention mirror")
    N, H, T, Hp, Wp = 2, 4, 2, 6, 8
    L = T * Hp * Wp
    g = torch.Generator().manual_seed(61)
    qa = torch.randn((N, L, H * D), generator=g)                      # F32 activations
    ka = torch.randn((N, L, H * D), generator=g).to(torch.bfloat16)
    va = torch.randn((N, L, H * D), generator=g).to(torch.bfloat16)
    table = kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)
    files = {n: str(tmp_path / f"{n}.bin") for n in ("q", "k", "v", "o", "r")}
    qa.numpy().tofile(files["q"])
    ka.view(torch.int16).numpy().tofile(files["k"])
    va.view(torch.int16).numpy().tofile(files["v"])
    table.tofile(files["r"])
    args = [exe, str(H), str(L), str(L), str(N), "bf16", files["q"], files["k"], files["v"], files["o"], files["r"]]
    wq = (torch.randn(D, generator=g) * 0.3 + 1.0).float()
    wk = (torch.randn(D, generator=g) * 0.3 + 1.0).float()
    if with_norm:
        wq.numpy().tofile(str(tmp_path / "wq.bin"))
        wk.numpy().tofile(str(tmp_path / "wk.bin"))
        args += [str(tmp_path / "wq.bin"), str(tmp_path / "wk.bin")]
    res = subprocess.run(args, capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stderr
    out = torch.from_numpy(np.fromfile(files["o"], dtype=np.float32).reshape(N, L, H, D))
    q4 = qa.view(N, L, H, D).permute(0, 2, 1, 3).contiguous()
    k4 = ka.view(N, L, H, D).permute(0, 2, 1, 3).contiguous()
    v4 = va.view(N, L, H, D).permute(0, 2, 1, 3).contiguous()
    if with_norm:
        q4 = torch.from_numpy(orc.rms_norm(q4.numpy(), wq.numpy(), 1e-6))
        k4 = torch.from_numpy(orc.rms_norm(k4.float().numpy(), wk.numpy(), 1e-6))
    ref = orc.fa_f64(q4, k4.to(torch.bfloat16) if with_norm else k4, v4,
                     rope=orc.rope_table(torch.from_numpy(table)))
    assert_parity(gather_rows(out, np.arange(N * H * L), H, L), ref, "C++ mirror")
