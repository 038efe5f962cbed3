"""Pins the oracle's attention (kdo_fa_f64, and the restated ggml per-row
algorithm kdo_fa_ggml) against the golden fixtures (float64 torch SDPA) and
against closed-form special cases of GGML_OP_FLASH_ATTN_EXT."""
import glob
import os

import numpy as np
import pytest
import torch

import kd_oracle as orc
from fa_common import D, gather_rows, metrics, qkv

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _all_rows(q):
    return np.arange(q.shape[0] * q.shape[1] * q.shape[2])


def _load(path):
    z = np.load(path, allow_pickle=False)
    dt = DT[str(z["dtype"])]
    q = torch.from_numpy(z["q"]).to(dt)
    k = torch.from_numpy(z["k"]).to(dt)
    v = torch.from_numpy(z["v"]).to(dt)
    assert torch.equal(q.float(), torch.from_numpy(z["q"]))   # values are exact in dt
    mask = torch.from_numpy(z["mask"]).to(torch.float16) if z["mask"].size else None
    rope = None
    if "rope_grid" in z.files:
        T, Hp, Wp = (int(x) for x in z["rope_grid"])
        rope = orc.rope_table(torch.from_numpy(orc.visual_rope_table(T, Hp, Wp)))
    return q, k, v, mask, float(z["scale"]), rope, z["out"]


FIXTURES = sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


def test_fixtures_present():
    assert len(FIXTURES) >= 4


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_f64_matches_golden(path):
    q, k, v, mask, scale, rope, out = _load(path)
    H, Lq = q.shape[1], q.shape[2]
    got = orc.fa_f64(q, k, v, mask=mask, scale=scale, rope=rope)
    ref = gather_rows(torch.from_numpy(out), _all_rows(q), H, Lq)
    # RoPE fixtures rotate in float64 before rounding to the storage type,
    # the oracle in float32 (as rope::apply does): an operand may land one
    # storage ulp apart, so those cases get a looser (still tight) bound.
    tol = 5e-3 if rope is not None else 1e-9
    assert np.max(np.abs(got - ref)) <= tol


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
@pytest.mark.parametrize("f16_vacc", [False, True])
def test_ggml_restatement_matches_golden(path, f16_vacc):
    q, k, v, mask, scale, rope, out = _load(path)
    H, Lq = q.shape[1], q.shape[2]
    dst, _ = orc.fa_ggml(q, k, v, mask=mask, scale=scale, rope=rope, f16_vacc=f16_vacc)
    got = gather_rows(dst, _all_rows(q), H, Lq)
    ref = gather_rows(torch.from_numpy(out), _all_rows(q), H, Lq)
    fp16_acc = f16_vacc and v.dtype == torch.float16
    tol = 5e-3 if (rope is not None or fp16_acc) else 2e-6
    assert np.max(np.abs(got - ref)) <= tol


# ----------------------------------------------------------------------------
# closed forms
# ----------------------------------------------------------------------------

def _both(q, k, v, mask=None, scale=None):
    f = orc.fa_f64(q, k, v, mask=mask, scale=scale)
    g, _ = orc.fa_ggml(q, k, v, mask=mask, scale=scale, f16_vacc=False)
    return f, gather_rows(g, _all_rows(q), q.shape[1], q.shape[2])


def test_single_key_returns_its_value():
    q, k, v = qkv(1, 2, 5, 1, torch.bfloat16, seed=1)
    f, g = _both(q, k, v)
    ref = v[0, :, 0, :].float().numpy().repeat(5, axis=0)
    assert np.array_equal(f, ref) and np.array_equal(g, ref)


def test_identical_keys_give_mean_of_values():
    q, k, v = qkv(1, 1, 4, 9, torch.float16, seed=2)
    k = k[:, :, :1].expand(-1, -1, 9, -1).contiguous()
    f, g = _both(q, k, v)
    ref = v[0, 0].double().mean(0).numpy()
    assert np.allclose(f, ref[None], atol=1e-12)
    assert np.allclose(g, ref[None], atol=1e-6)


def test_zero_scale_gives_mean_of_unmasked_values():
    q, k, v = qkv(1, 1, 3, 10, torch.bfloat16, seed=3)
    mask = torch.zeros((1, 1, 3, 10), dtype=torch.float16)
    mask[..., 6:] = float("-inf")
    f, g = _both(q, k, v, mask=mask, scale=0.0)
    ref = v[0, 0, :6].double().mean(0).numpy()
    assert np.allclose(f, ref[None], atol=1e-12) and np.allclose(g, ref[None], atol=1e-6)


def test_one_open_key_and_fully_masked_rows():
    q, k, v = qkv(1, 1, 6, 8, torch.bfloat16, seed=4)
    mask = torch.full((1, 1, 6, 8), float("-inf"), dtype=torch.float16)
    for i in range(5):
        mask[0, 0, i, (3 * i) % 8] = 0.0          # row 5 stays fully masked
    f, g = _both(q, k, v, mask=mask)
    for i in range(5):
        assert np.array_equal(f[i], v[0, 0, (3 * i) % 8].float().numpy())
        assert np.array_equal(g[i], v[0, 0, (3 * i) % 8].float().numpy())
    assert np.all(f[5] == 0) and np.all(g[5] == 0)


def test_permuting_keys_with_values_changes_nothing():
    q, k, v = qkv(2, 2, 5, 17, torch.bfloat16, seed=5)
    perm = torch.randperm(17, generator=torch.Generator().manual_seed(0))
    a = orc.fa_f64(q, k, v)
    b = orc.fa_f64(q, k[:, :, perm].contiguous(), v[:, :, perm].contiguous())
    assert np.allclose(a, b, atol=1e-12)


def test_linear_in_values():
    q, k, _ = qkv(1, 2, 4, 12, torch.float32, seed=6)
    v1 = torch.randn((1, 2, 12, D), generator=torch.Generator().manual_seed(1))
    v2 = torch.randn((1, 2, 12, D), generator=torch.Generator().manual_seed(2))
    a = orc.fa_f64(q, k, 2.0 * v1 - 3.0 * v2)
    b = 2.0 * orc.fa_f64(q, k, v1) - 3.0 * orc.fa_f64(q, k, v2)
    # the combined V is itself rounded to float32 on input
    assert np.allclose(a, b, atol=4e-6)


def test_constant_mask_shift_is_invariant():
    q, k, v = qkv(1, 1, 4, 12, torch.bfloat16, seed=7)
    zero = torch.zeros((1, 1, 4, 12), dtype=torch.float16)
    a = orc.fa_f64(q, k, v, mask=zero)
    b = orc.fa_f64(q, k, v, mask=zero + 3.5)
    assert np.allclose(a, b, atol=1e-12)


def test_mask_enters_additively():
    """softmax(scale*qk + m): an additive log(2) on one key doubles its weight."""
    q, k, v = qkv(1, 1, 1, 2, torch.float32, seed=8)
    m = torch.zeros((1, 1, 1, 2), dtype=torch.float16)
    m[..., 0] = float(np.log(2.0))
    got = orc.fa_f64(q, k, v, mask=m)[0]
    s = (q[0, 0, 0].double() @ k[0, 0].double().T) / np.sqrt(D)
    mf = float(m[0, 0, 0, 0])                  # log(2) as stored in F16
    w = torch.exp(s - s.max()) * torch.tensor([np.exp(mf), 1.0], dtype=torch.float64)
    ref = (w / w.sum()) @ v[0, 0].double()
    assert np.allclose(got, ref.numpy(), atol=1e-12)


def test_gqa_and_batch_broadcast_equal_explicit_repeat():
    q, k, v = qkv(2, 4, 6, 9, torch.bfloat16, seed=9, Hkv=2, Bk=1)
    a = orc.fa_f64(q, k, v)
    kr = k.repeat_interleave(2, dim=1).expand(2, -1, -1, -1).contiguous()
    vr = v.repeat_interleave(2, dim=1).expand(2, -1, -1, -1).contiguous()
    b = orc.fa_f64(q, kr, vr)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("f64", [True, False])
def test_k_and_v_broadcast_separately(f64):
    """ggml maps a query head to its K head and its V head separately
    (h / (H / Hk), h / (H / Hv)); with 2 K heads and 4 V heads for H = 4, and
    K over batch but V not, the result equals explicitly repeated operands."""
    q, _, _ = qkv(2, 4, 6, 9, torch.float16, seed=19)
    k = qkv(1, 2, 1, 9, torch.float16, seed=20)[1]
    v = qkv(2, 4, 1, 9, torch.float16, seed=21)[2]
    kr = k.repeat_interleave(2, dim=1).expand(2, -1, -1, -1).contiguous()
    if f64:
        assert np.array_equal(orc.fa_f64(q, k, v), orc.fa_f64(q, kr, v))
    else:
        a, _ = orc.fa_ggml(q, k, v)
        b, _ = orc.fa_ggml(q, kr, v)
        assert torch.equal(a, b)
    # V indexed with the K head (V heads 0, 0, 1, 1 for query heads 0..3)
    # gives another result
    vw = v[:, :2].repeat_interleave(2, dim=1).contiguous()
    assert not np.allclose(orc.fa_f64(q, k, v), orc.fa_f64(q, k, vw))


def test_mask_broadcast_over_heads_and_rows_beyond_lq():
    q, k, v = qkv(2, 2, 5, 7, torch.bfloat16, seed=10)
    g = torch.Generator().manual_seed(3)
    m = torch.randn((2, 1, 8, 7), generator=g).to(torch.float16)  # 8 >= Lq rows, per batch
    a = orc.fa_f64(q, k, v, mask=m)
    full = m[:, :, :5].expand(2, 2, 5, 7).contiguous()
    b = orc.fa_f64(q, k, v, mask=full)
    assert np.array_equal(a, b)


def test_softcap_formula():
    q, k, v = qkv(1, 1, 3, 6, torch.float32, seed=11)
    got = orc.fa_f64(q, k, v, logit_softcap=2.0)
    s = (q[0, 0].double() @ k[0, 0].double().T) * float(np.float32(1 / np.sqrt(D)))
    s = 2.0 * torch.tanh(s)
    ref = torch.softmax(s, -1) @ v[0, 0].double()
    assert np.allclose(got, ref.numpy(), atol=1e-9)


def test_alibi_rejected():
    q, k, v = qkv(1, 1, 2, 2, torch.float32, seed=12)
    with pytest.raises(RuntimeError):
        orc.fa_f64(q, k, v, max_bias=8.0)


def test_ggml_restatement_f16_accumulator_deviation_is_small():
    q, k, v = qkv(1, 2, 32, 300, torch.float16, seed=13)
    f = orc.fa_f64(q, k, v)
    g16, _ = orc.fa_ggml(q, k, v, f16_vacc=True)
    g32, _ = orc.fa_ggml(q, k, v, f16_vacc=False)
    r16 = gather_rows(g16, _all_rows(q), 2, 32)
    r32 = gather_rows(g32, _all_rows(q), 2, 32)
    assert metrics(r32, f)["max_abs"] < 2e-6
    m16 = metrics(r16, f)
    assert 0 < m16["max_abs"] < 5e-3 and m16["cos"] > 0.9999


def test_row_subset_equals_full():
    q, k, v = qkv(2, 3, 20, 33, torch.bfloat16, seed=14)
    rows = np.array([5, 0, 119, 64, 77])
    sub = orc.fa_f64(q, k, v, rows=rows)
    full = orc.fa_f64(q, k, v)
    assert np.array_equal(sub, full[rows])
    dst, _ = orc.fa_ggml(q, k, v, rows=rows)
    got = gather_rows(dst, rows, 3, 20)
    assert np.allclose(got, full[rows], atol=2e-6)
