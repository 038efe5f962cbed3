"""Run-to-run determinism of every kernel route: each route is called three
times on one input, and the three outputs must be equal bit for bit.

A missing wait state between a matrix-unit result and its vector reader
(the compiler does not check inline-asm operands against those hazards)
shows up as outputs that change from run to run, not as a fault; this is
the regression test for that class.  The routes are those the kernel
choice of kd_fa_run / kd_fa_run_ws / kd_fa_rope_run / kd_fa_dit_run takes:
the 64-row kernel, the 32-row kernel (pipelined unmasked loop with 4- and
8-wave workgroups, masked loop, K rotated on load), the short-key kernel
(masked, unmasked, F32 Q, with the mask summary), the persistent
long-prompt kernels (the 64-row one for F32 Q; the 32-row one for F32 and
16-bit Q), the staged schedule, the
F32 cast pre-pass, and the D = 512 kernel with and without its key split.
"""
import pytest
import torch

import kd_fa
from fa_common import AXES, D, SCALE_FACTOR, THETA, padding_mask

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _rand(shape, seed, dtype, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV, dtype=torch.float32) * scale).to(dtype)


def _three(fn):
    outs = []
    for _ in range(3):
        o = fn()
        torch.cuda.synchronize()
        outs.append(o.clone())
    assert torch.isfinite(outs[0].float()).all()
    for o in outs[1:]:
        assert torch.equal(outs[0], o), float((outs[0].float() - o.float()).abs().max())


def _rope(T, Hp, Wp):
    return kd_fa.rope_table(torch.from_numpy(kd_fa.visual_rope_table(T, Hp, Wp, AXES, SCALE_FACTOR, THETA)).to(DEV))


# (name, Lk, mask, routing flags, dtype, Q dtype): plain node routes
PLAIN = [
    ("w64", 1030, False, kd_fa.ROUTE_DEFAULT, torch.bfloat16, torch.bfloat16),
    ("w64_f16_q32", 1030, False, kd_fa.ROUTE_DEFAULT, torch.float16, torch.float32),
    ("d128_pipelined_8w", 1030, False, kd_fa.ROUTE_NO_W64, torch.bfloat16, torch.bfloat16),
    ("d128_pipelined_4w", 512, False, kd_fa.ROUTE_DEFAULT, torch.float16, torch.float32),
    ("d128_masked", 300, True, kd_fa.ROUTE_DEFAULT, torch.bfloat16, torch.bfloat16),
    ("xres_masked", 256, True, kd_fa.ROUTE_DEFAULT, torch.bfloat16, torch.bfloat16),
    ("xres_unmasked_q32", 77, False, kd_fa.ROUTE_DEFAULT, torch.float16, torch.float32),
    ("d128_short_masked", 200, True, kd_fa.ROUTE_NO_XRES, torch.float16, torch.float16),
    ("xlong64_f16_q32", 512, False, kd_fa.ROUTE_DEFAULT, torch.float16, torch.float32),
    ("xlong_f16_q32", 512, False, kd_fa.ROUTE_NO_XLONG64, torch.float16, torch.float32),
    ("xlong_bf16_tail", 300, False, kd_fa.ROUTE_DEFAULT, torch.bfloat16, torch.bfloat16),
]


@pytest.mark.parametrize("case", PLAIN, ids=lambda c: c[0])
def test_plain_routes_repeat_bitwise(case):
    _need_gpu()
    name, Lk, masked, route, dt, qdt = case
    B, H, Lq = 2, 8, 2048
    _announce(f"determinism {name}: B={B} H={H} Lq={Lq} Lk={Lk} {dt} q {qdt} mask={masked}")
    # logits with std 3 so that the lazy row max leaves its fast path now and then
    q = _rand((B, H, Lq, D), 1, qdt, 1.7)
    k = _rand((B, H, Lk, D), 2, dt, 1.7)
    v = _rand((B, H, Lk, D), 3, dt)
    m = padding_mask(B, Lq, Lk, (Lk, Lk // 3 + 1), device=DEV) if masked else None
    with kd_fa.routing(route):
        _three(lambda: kd_fa.flash_attn_ext(q, k, v, mask=m))


def test_mask_summary_repeat_bitwise():
    _need_gpu()
    _announce("determinism mask summary + short-key kernel (kd_fa_run_ws)")
    B, H, Lq, Lk = 2, 8, 2048, 256
    q, k, v = _rand((B, H, Lq, D), 4, torch.bfloat16), _rand((B, H, Lk, D), 5, torch.bfloat16), \
        _rand((B, H, Lk, D), 6, torch.bfloat16)
    m = padding_mask(B, Lq, Lk, (120, 40), device=DEV)
    dst = torch.empty((B, Lq, H, D), device=DEV)
    d = kd_fa.make_desc(q, k, v, m, dst, D ** -0.5)
    ws = torch.empty(kd_fa.workspace_size_full(d), dtype=torch.uint8, device=DEV)
    with kd_fa.routing(kd_fa.ROUTE_SUMMARY):
        def call():
            assert kd_fa.run_desc(d, None, None, ws) == kd_fa.OK
            return dst
        _three(call)


@pytest.mark.parametrize("form", ["on_load", "staged", "workspace", "f32_cast_norm"])
def test_rope_routes_repeat_bitwise(form):
    """Self-attention with 3-D RoPE: K rotated on load (one launch), the
    staged groups, the workspace pre-pass, and F32 Q/K/V cast by the
    pre-pass with the query/key RMSNorm."""
    _need_gpu()
    T, Hp, Wp = 4, 16, 16
    L = T * Hp * Wp
    B, H = 1, 8
    _announce(f"determinism RoPE {form}: [128,{L},{H},{B}]")
    dt = torch.float32 if form == "f32_cast_norm" else torch.bfloat16
    q, k, v = _rand((B, H, L, D), 7, dt), _rand((B, H, L, D), 8, dt), _rand((B, H, L, D), 9, dt)
    rope = _rope(T, Hp, Wp)
    dst = torch.empty((B, L, H, D), device=DEV)
    d = kd_fa.make_desc(q, k, v, None, dst, D ** -0.5)
    norm = None
    if form == "f32_cast_norm":
        norm = kd_fa.qk_norm(_rand((D,), 10, torch.float32, 0.3) + 1.0, _rand((D,), 11, torch.float32, 0.3) + 1.0)
    ws = None
    if form in ("workspace", "f32_cast_norm"):
        ws = torch.empty(kd_fa.workspace_size_full(d, rope, norm), dtype=torch.uint8, device=DEV)
    route = kd_fa.ROUTE_STAGED if form == "staged" else kd_fa.ROUTE_DEFAULT
    with kd_fa.routing(route):
        def call():
            assert kd_fa.run_desc(d, rope, None, ws, norm) == kd_fa.OK
            return dst
        _three(call)


@pytest.mark.parametrize("split", [False, True])
def test_d512_repeat_bitwise(split):
    """The VAE's one-head D = 512 attention at 1,024 tokens: one pass, and
    the key split merged through the workspace."""
    _need_gpu()
    L = 1024
    _announce(f"determinism D=512 L={L} split={split}")
    q = _rand((1, 1, L, 512), 12, torch.float32)
    k = _rand((1, 1, L, 512), 13, torch.float16)
    v = _rand((1, 1, L, 512), 14, torch.float16)
    dst = torch.empty((1, L, 1, 512), device=DEV)
    d = kd_fa.make_desc(q, k, v, None, dst, 512 ** -0.5)
    ws = torch.empty(max(kd_fa.workspace_size_full(d), 16), dtype=torch.uint8, device=DEV) if split else None
    if split:
        assert kd_fa.workspace_size_full(d) > 0

    def call():
        assert kd_fa.run_desc(d, None, None, ws) == kd_fa.OK
        return dst
    _three(call)
