"""The hot window lifecycle oracle (CPU): value-norm ranking, kept-token selection, the
cooling step and the host-side checks of phasekv_amd.cache, pinned against torch's own
norm / top-k (the calls the reference makes), brute force and closed forms."""
import numpy as np
import pytest
import torch

from oracle import cache_oracle as co
from oracle import packing_oracle as po


def _rng(seed):
    return np.random.default_rng(seed)


def test_value_norms_close_to_float64_and_exact_on_closed_forms():
    v = (_rng(1).standard_normal((2, 3, 50, 128)) * 3).astype(np.float16)
    got = co.value_norms(v)
    want = np.sqrt((v.astype(np.float64) ** 2).sum(-1))
    np.testing.assert_allclose(got, want, rtol=2e-6)
    assert got.dtype == np.float32
    # a single non-zero channel: the norm is |x| exactly, wherever the channel sits
    for hd in (64, 96, 128, 256):
        for c in (0, 17, hd - 1):
            x = np.zeros((1, hd), np.float16)
            x[0, c] = -3.5
            assert co.value_norms(x)[0] == np.float32(3.5)
    # 3-4-5 over two channels in different lanes and different rounds
    x = np.zeros((1, 128), np.float16)
    x[0, 5], x[0, 64 + 9] = 3, 4
    assert co.value_norms(x)[0] == np.float32(5)


@pytest.mark.parametrize("seed", range(6))
def test_selection_equals_torch_topk_sort_on_tie_free_inputs(seed):
    rng = _rng(seed)
    aged = int(rng.integers(2, 90))
    keep = int(rng.integers(1, aged + 1))
    v = rng.standard_normal((2, 4, aged, 128)).astype(np.float16)
    norms = co.value_norms(v)
    ref = torch.linalg.vector_norm(torch.from_numpy(v).float(), dim=-1)
    # torch's norm and the oracle's differ at most in the last bits; no near ties here
    np.testing.assert_allclose(norms, ref.numpy(), rtol=1e-6)
    want = ref.topk(keep, dim=-1).indices.sort(dim=-1).values.numpy()
    assert np.array_equal(co.select_kept(norms, keep), want)


def test_selection_ties_and_nan_by_brute_force():
    rng = _rng(7)
    for _ in range(200):
        n = int(rng.integers(1, 12))
        keep = int(rng.integers(1, n + 1))
        vals = rng.choice(np.array([0.5, 1.0, 2.0, np.nan], np.float32), size=n)
        # explicit ranking: u above t if (NaN over numbers) or larger, equal -> earlier
        def above(u, t):
            nu, nt = vals[u], vals[t]
            if np.isnan(nu) != np.isnan(nt):
                return bool(np.isnan(nu))
            if np.isnan(nu) or nu == nt:
                return u < t
            return nu > nt
        kept = [t for t in range(n) if sum(above(u, t) for u in range(n)) < keep]
        assert co.select_kept(vals[None], keep)[0].tolist() == kept


def test_equal_norms_keep_the_earliest_tokens():
    v = np.ones((1, 1, 10, 64), np.float16)
    assert co.select_kept(co.value_norms(v), 4).tolist() == [[[0, 1, 2, 3]]]


def test_keep_count_uses_python_round():
    assert co.keep_count(5, 0.5) == 2      # round(2.5) == 2
    assert co.keep_count(7, 0.5) == 4      # round(3.5) == 4
    assert co.keep_count(16, 1.0) == 16
    assert co.keep_count(16, 0.01) == 1    # at least one token
    from phasekv_amd.cache import keep_count
    for aged in range(1, 40):
        for r in (0.01, 0.25, 0.5, 0.7, 1.0):
            assert keep_count(aged, r) == co.keep_count(aged, r)


def _hot(seed, B=2, H=3, cap=48, hd=64):
    rng = _rng(seed)
    k = (rng.standard_normal((B, H, cap, hd)) * 2).astype(np.float16)
    v = rng.standard_normal((B, H, cap, hd)).astype(np.float16)
    return k, v


def test_cooling_is_a_no_op_until_lazy_g_tokens_aged():
    k, v = _hot(1)
    k0, v0 = k.copy(), v.copy()
    seg, hot_len, idx = co.cool_aged_tokens(k, v, 47, 32, 16, 0.5, 4, 32)
    assert seg is None and hot_len == 47 and idx.shape[-1] == 0
    assert np.array_equal(k, k0) and np.array_equal(v, v0)


def test_cooling_keep_all_packs_the_aged_rows_and_shifts_the_tail():
    k, v = _hot(2)
    k0, v0 = k.copy(), v.copy()
    seg, hot_len, idx = co.cool_aged_tokens(k, v, 48, 32, 16, 1.0, 4, 32)
    assert hot_len == 32
    assert np.array_equal(idx[0, 0], np.arange(16))
    want_k = po.quantize_pack(k0[:, :, :16], 4, -2, 32)
    want_v = po.quantize_pack(v0[:, :, :16], 4, -1, 32)
    # K groups along the 16 cooled tokens (group min(32, 16)), V along head_dim
    assert seg[0].group_size == 16 and seg[1].group_size == 32
    for got, want in ((seg[0], want_k), (seg[1], want_v)):
        assert got.group_size == want.group_size
        assert np.array_equal(got.packed, want.packed)
        assert np.array_equal(got.scale, want.scale) and np.array_equal(got.mins, want.mins)
    assert np.array_equal(k[:, :, :32], k0[:, :, 16:48])
    assert np.array_equal(v[:, :, :32], v0[:, :, 16:48])


def test_cooling_keeps_the_largest_value_rows():
    k, v = _hot(3)
    v[:, :, :16] = np.float16(0.01)
    big = [3, 7, 8, 15]
    for t in big:
        v[:, :, t] = np.float16(1 + t)           # distinct, clearly largest norms
    k0 = k.copy()
    seg, hot_len, idx = co.cool_aged_tokens(k, v, 48, 32, 16, 0.25, 2, 32)
    assert hot_len == 32 and (idx == np.array(big)).all()
    want_k = po.quantize_pack(k0[:, :, big], 2, -2, 32)
    assert np.array_equal(seg[0].packed, want_k.packed)


def test_a_reversed_tie_break_is_caught():
    """Planted mistake on the CPU: ranking later tokens first on equal norms changes the
    kept set, so the tie test above would fail for it."""
    norms = np.ones((1, 6), np.float32)
    key = np.where(np.isnan(norms), -np.inf, -norms.astype(np.float64))[0]
    wrong = np.sort(np.lexsort((-np.arange(6), key))[:2])
    assert wrong.tolist() != co.select_kept(norms, 2)[0].tolist()


def test_host_checks_before_any_launch():
    from phasekv_amd import cache
    with pytest.raises(ValueError, match="cold_bits"):
        cache._validate_config(2, 3, 32, 32, 16, 1.0)
    with pytest.raises(ValueError, match="decode_keep_ratio"):
        cache._validate_config(2, 4, 32, 32, 16, 0.0)
    with pytest.raises(ValueError, match="lazy_g"):
        cache._validate_config(2, 4, 32, 32, 0, 1.0)

    class Dense:
        key_cache = [torch.zeros(1, 2, 8, 64, dtype=torch.float16)]
        value_cache = [torch.zeros(1, 2, 8, 64, dtype=torch.float16)]

    # host tensors are refused: there is no CPU path
    with pytest.raises(ValueError, match="ROCm GPU"):
        cache.PhaseKVCache.from_dense_prefill(Dense(), prompt_len=8)
    with pytest.raises(TypeError):
        cache.PhaseKVCache.from_dense_prefill(object(), prompt_len=8)
    hk = torch.zeros(1, 2, 48, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="ROCm GPU"):
        cache.cool_hot(hk, hk.clone(), 48, 16, 8)
