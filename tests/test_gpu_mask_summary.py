"""GPU checks of kd_fa_run_ws's mask summary: for a masked node with at most
256 keys (the text cross-attention, src/models/crossdit.hpp:174-200), a pass
over the mask writes one word per (mask batch, mask head, 32-row query
block) into the caller's workspace, bit t set when 64-key tile t holds a
value other than -inf for one of the block's rows, and the short-key kernel
then skips the other tiles without loading their mask rows.

Skipping a tile whose mask is -inf for every row of a block is what the
kernel does anyway after loading that tile's mask chunks, so the output must
be bitwise kd_fa_run's.  Each case checks that, on a workspace filled with
garbage first, and checks the summary words themselves against numpy.  The
masks walk the cases that decide a word: per-batch padding (different dead
tiles per batch), a staircase whose live tiles change from block to block,
rows with no key at all, a single finite key in an otherwise dead tile, NaN
entries (not -inf, so live), masks shared by all heads or per head and
broadcast over batches, ragged key counts (a partial last tile) and ragged
query counts (the last block's rows past Lq read row Lq - 1).  The query /
key RMSNorm path (K transformed into the workspace, the summary after it)
and the allocation-free entry point take the summary too; the production
shape closes the file.  Below 65,536 query rows in all the library skips the
pass (its launch would not pay back); the small cases here build it with
KD_FA_ROUTE_SUMMARY, and one case checks that the default leaves the
workspace untouched there.
"""

import ctypes

import numpy as np
import pytest
import torch

import kd_fa
import kd_oracle as orc
from fa_common import D, assert_parity, gather_rows, padding_mask, qkv, randn, sample_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _announce(msg):
    print(f"[case] {msg}", flush=True)


def _mask(kind, B, H, Lq, Lk, seed):
    """F16 mask (Bm, Hm, Lq + 3, ne0) with rows padded to whole 8-key chunks."""
    ne0 = (Lk + 7) // 8 * 8
    g = torch.Generator().manual_seed(seed)
    rows = Lq + 3
    if kind == "pad":
        m = padding_mask(B, rows - 3, ne0, [max(1, (Lk * (b + 1)) // (B + 2)) for b in range(B)], pad_rows=3)
    elif kind == "stair":
        # row r sees keys below 1 + (r * 7) % Lk: live tiles change per block
        m = torch.full((B, 1, rows, ne0), float("-inf"), dtype=torch.float16)
        for r in range(rows):
            m[:, :, r, : 1 + (r * 7) % Lk] = 0.0
    elif kind == "dead_rows":
        m = (torch.randn((B, 1, rows, ne0), generator=g)).to(torch.float16)
        m[:, :, ::3, :] = float("-inf")
        m[:, :, : min(rows, 64), 64:] = float("-inf")       # the first two blocks: only tile 0 live
    elif kind == "single":
        # every tile dead except one finite key of one row in tile (block % n_tiles)
        m = torch.full((B, 1, rows, ne0), float("-inf"), dtype=torch.float16)
        n_t = (Lk + 63) // 64
        for qb in range((Lq + 31) // 32):
            t = qb % n_t
            key = min(t * 64 + 63, Lk - 1)
            m[:, :, qb * 32 + (qb % 32) if qb * 32 + (qb % 32) < Lq else Lq - 1, key] = -3.0
    elif kind == "nan":
        m = torch.full((B, 1, rows, ne0), float("-inf"), dtype=torch.float16)
        m[:, :, :, 0] = 0.0                                  # every row sees key 0
        m[:, :, 5, min(Lk - 1, 70)] = float("nan")           # NaN is not -inf: that tile is live
    elif kind == "rand_per_head":
        m = (torch.randn((B, H, rows, ne0), generator=g) * 2).to(torch.float16)
        m[torch.rand((B, H, rows, ne0), generator=g) < 0.97] = float("-inf")
    elif kind == "bcast_batch":
        m = torch.full((1, H, rows, ne0), float("-inf"), dtype=torch.float16)
        for h in range(H):
            m[0, h, :, : max(1, (Lk * (h + 1)) // (H + 1))] = 0.0
    else:
        raise ValueError(kind)
    # keys past Lk in the padded chunk hold values that must not count
    if ne0 > Lk:
        m[..., Lk:] = 1.0
    return m


def _summary_ref(m, Lq, Lk):
    """The summary words, from the mask on the host (numpy)."""
    mm = m.float().numpy()
    Bm, Hm = mm.shape[0], mm.shape[1]
    nqb = (Lq + 31) // 32
    n_t = (Lk + 63) // 64
    out = np.zeros((Bm, Hm, nqb), dtype=np.uint32)
    for qb in range(nqb):
        rows = np.minimum(qb * 32 + np.arange(32), Lq - 1)
        for t in range(n_t):
            sub = mm[:, :, rows, t * 64: min(t * 64 + 64, Lk)]
            live = np.any(sub != -np.inf, axis=(2, 3))
            out[:, :, qb] |= live.astype(np.uint32) << t
    return out.reshape(-1)


def _garbage_ws(nbytes):
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
    ws.fill_(0xA5)
    return ws


CASES = [
    # B, H, Lq, Lk, mask kind, Q dtype, dst dtype
    (2, 4, 300, 256, "pad", torch.bfloat16, torch.float32),
    (2, 3, 200, 256, "stair", torch.bfloat16, torch.float32),
    (1, 2, 257, 200, "stair", torch.float32, torch.float32),
    (2, 2, 150, 130, "dead_rows", torch.bfloat16, torch.bfloat16),
    (1, 3, 190, 256, "single", torch.float32, torch.float32),
    (1, 2, 100, 77, "nan", torch.float32, torch.float32),
    (2, 4, 96, 256, "rand_per_head", torch.bfloat16, torch.float16),
    (3, 4, 130, 100, "bcast_batch", torch.float32, torch.float32),
    (2, 2, 33, 64, "pad", torch.bfloat16, torch.float32),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}q{c[2]}k{c[3]}{c[4]}")
def test_summary_skips_dead_tiles_bitwise(case):
    _need_gpu()
    B, H, Lq, Lk, kind, qt, ot = case
    _announce(f"mask summary {case}")
    kt = torch.float16 if kind in ("nan", "single") else torch.bfloat16
    q, k, v = qkv(B, H, Lq, Lk, kt, seed=B * 31 + H * 7 + Lk, q_dtype=qt)
    m = _mask(kind, B, H, Lq, Lk, seed=Lq)
    mv = m[:, :, :Lq, :]                       # ggml view: rows = Lq, row stride of the padded tensor
    q, k, v, md = q.to(DEV), k.to(DEV), v.to(DEV), mv.to(DEV)
    dst = torch.empty((B, Lq, H, D), dtype=ot, device=DEV)
    dst_ws = torch.empty_like(dst)
    d = kd_fa.make_desc(q, k, v, md, dst, D ** -0.5)
    d_ws = kd_fa.make_desc(q, k, v, md, dst_ws, D ** -0.5)
    need = kd_fa.workspace_size_full(d_ws)
    Bm, Hm = m.shape[0], m.shape[1]
    assert need == 4 * Bm * Hm * ((Lq + 31) // 32)
    ws = _garbage_ws(need)
    assert kd_fa.run_desc(d) == kd_fa.OK
    with kd_fa.routing(kd_fa.ROUTE_SUMMARY):
        assert kd_fa.run_desc(d_ws, workspace=ws) == kd_fa.OK
    torch.cuda.synchronize()
    words = ws[:need].cpu().numpy().view(np.uint32)
    ref_words = _summary_ref(mv, Lq, Lk)
    assert np.array_equal(words, ref_words), (words[:16], ref_words[:16])
    assert torch.equal(dst, dst_ws) or torch.equal(torch.nan_to_num(dst, nan=7.0), torch.nan_to_num(dst_ws, nan=7.0))


def test_summary_parity_against_oracle():
    """The summary path against the float64 oracle (every row)."""
    _need_gpu()
    B, H, Lq, Lk = 2, 3, 160, 256
    _announce("mask summary parity")
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=5)
    m = _mask("stair", B, H, Lq, Lk, seed=1)[:, :, :Lq, :]
    dst = torch.empty((B, Lq, H, D), dtype=torch.float32, device=DEV)
    d = kd_fa.make_desc(q.to(DEV), k.to(DEV), v.to(DEV), m.to(DEV), dst, D ** -0.5)
    ws = _garbage_ws(kd_fa.workspace_size_full(d))
    with kd_fa.routing(kd_fa.ROUTE_SUMMARY):
        assert kd_fa.run_desc(d, workspace=ws) == kd_fa.OK
    torch.cuda.synchronize()
    ref = orc.fa_f64(q, k, v, mask=m, scale=D ** -0.5)
    assert_parity(gather_rows(dst, np.arange(B * H * Lq), H, Lq), ref, "mask summary")


def test_summary_after_transformed_k_and_static_entry():
    """kd_fa_dit_run with query/key RMSNorm and a mask: K normalised into the
    workspace, the summary after it (256-byte aligned); bitwise equal to the
    call with a K-sized workspace (no summary), to the call without one (K
    normalised on load) and to the allocation-free entry point."""
    _need_gpu()
    B, H, Lq, Lk = 2, 4, 230, 200
    _announce("mask summary after normalised K")
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=12, q_dtype=torch.float32)
    m = _mask("stair", B, H, Lq, Lk, seed=2)[:, :, :Lq, :].to(DEV)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    wq = (randn((D,), torch.float32, 3) * 0.3 + 1.0).to(DEV)
    wk = (randn((D,), torch.float32, 4) * 0.3 + 1.0).to(DEV)
    norm = kd_fa.qk_norm(wq, wk, 1e-6)
    outs = [torch.empty((B, Lq, H, D), dtype=torch.float32, device=DEV) for _ in range(4)]
    descs = [kd_fa.make_desc(q, k, v, m, o, D ** -0.5) for o in outs]
    full = kd_fa.workspace_size_full(descs[0], norm=norm)
    kbytes = kd_fa.workspace_size(descs[0])
    assert full == (kbytes + 255) // 256 * 256 + 4 * 2 * ((Lq + 31) // 32)
    ws_full, ws_k = _garbage_ws(full), _garbage_ws(kbytes)
    with kd_fa.routing(kd_fa.ROUTE_SUMMARY):
        assert kd_fa.run_desc(descs[0], None, None, ws_full, norm) == kd_fa.OK
        assert kd_fa.run_desc(descs[1], None, None, ws_k, norm) == kd_fa.OK
        assert kd_fa.run_desc(descs[2], None, None, None, norm) == kd_fa.OK
        assert kd_fa.run_static(descs[3], None, norm) == kd_fa.OK
    torch.cuda.synchronize()
    words = ws_full[(kbytes + 255) // 256 * 256: full].cpu().numpy().view(np.uint32)
    assert np.array_equal(words, _summary_ref(m.cpu(), Lq, Lk))
    for o in outs[1:]:
        assert torch.equal(outs[0], o)


def test_summary_production_cross_attention():
    """The 31,744-token text cross-attention (Q bf16 [128, 31744, 32, 2], K/V
    256 keys, padding mask 120 / 40 valid keys): bitwise kd_fa_run's output,
    summary words as numpy computes them, sampled rows against the oracle."""
    _need_gpu()
    B, H, L, Lk = 2, 32, 31744, 256
    _announce(f"mask summary production [128,{L},{H},{B}] x {Lk}")
    g = torch.Generator(device=DEV).manual_seed(11)
    q, k, v = (torch.randn((B, H, n, D), generator=g, device=DEV).to(torch.bfloat16) for n in (L, Lk, Lk))
    m = padding_mask(B, L, Lk, [120, 40], device=DEV)
    dst = torch.empty((B, L, H, D), dtype=torch.float32, device=DEV)
    dst_ws = torch.empty_like(dst)
    d = kd_fa.make_desc(q, k, v, m, dst, D ** -0.5)
    d_ws = kd_fa.make_desc(q, k, v, m, dst_ws, D ** -0.5)
    need = kd_fa.workspace_size_full(d_ws)
    ws = _garbage_ws(need)
    assert kd_fa.run_desc(d) == kd_fa.OK
    assert kd_fa.run_desc(d_ws, workspace=ws) == kd_fa.OK
    torch.cuda.synchronize()
    assert torch.equal(dst, dst_ws)
    words = ws[:need].cpu().numpy().view(np.uint32).reshape(B, -1)
    assert np.all(words[0] == 0b11) and np.all(words[1] == 0b1)
    rows = sample_rows(B, H, L, 16, seed=3)
    ref = orc.fa_f64(q.cpu(), k.cpu(), v.cpu(), mask=m.cpu(), scale=D ** -0.5, rows=rows)
    assert_parity(gather_rows(dst_ws, rows, H, L), ref, "mask summary production")


def test_small_or_missing_workspace_is_kd_fa_run():
    """kd_fa_run_ws with a workspace below kd_fa_workspace_size, or none,
    runs as kd_fa_run (bitwise); an unmasked node uses no workspace."""
    _need_gpu()
    B, H, Lq, Lk = 2, 2, 130, 200
    _announce("mask summary: small / missing workspace")
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=21)
    m = _mask("stair", B, H, Lq, Lk, seed=3)[:, :, :Lq, :].to(DEV)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = [torch.empty((B, Lq, H, D), dtype=torch.float32, device=DEV) for _ in range(3)]
    descs = [kd_fa.make_desc(q, k, v, m, o, D ** -0.5) for o in outs]
    need = kd_fa.workspace_size_full(descs[0])
    small = _garbage_ws(need - 16)
    assert kd_fa.run_desc(descs[0]) == kd_fa.OK
    assert kd_fa.run_desc(descs[1], workspace=small) == kd_fa.OK
    lib = kd_fa.lib()
    h = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.kd_fa_run_ws(ctypes.byref(descs[2]), None, 0, h) == kd_fa.OK
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    nm = kd_fa.make_desc(q, k, v, None, outs[0], D ** -0.5)
    assert kd_fa.workspace_size_full(nm) == 0


def test_summary_skipped_below_the_row_threshold():
    """Below 65,536 query rows the default route runs without the summary
    (the workspace is left as it was); KD_FA_ROUTE_SUMMARY builds it; both
    give kd_fa_run's bits."""
    _need_gpu()
    B, H, Lq, Lk = 1, 2, 200, 256
    _announce("mask summary threshold")
    q, k, v = qkv(B, H, Lq, Lk, torch.bfloat16, seed=31)
    m = _mask("stair", B, H, Lq, Lk, seed=4)[:, :, :Lq, :].to(DEV)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = [torch.empty((B, Lq, H, D), dtype=torch.float32, device=DEV) for _ in range(3)]
    descs = [kd_fa.make_desc(q, k, v, m, o, D ** -0.5) for o in outs]
    need = kd_fa.workspace_size_full(descs[0])
    ws_a, ws_b = _garbage_ws(need), _garbage_ws(need)
    assert kd_fa.run_desc(descs[0]) == kd_fa.OK
    assert kd_fa.run_desc(descs[1], workspace=ws_a) == kd_fa.OK
    with kd_fa.routing(kd_fa.ROUTE_SUMMARY):
        assert kd_fa.run_desc(descs[2], workspace=ws_b) == kd_fa.OK
    torch.cuda.synchronize()
    assert torch.all(ws_a[:need] == 0xA5)
    assert np.array_equal(ws_b[:need].cpu().numpy().view(np.uint32), _summary_ref(m.cpu(), Lq, Lk))
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
