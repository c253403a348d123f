"""The prefill prompt-selection oracle (CPU), pinned against the torch calls the reference
makes (float sums, max_pool1d / avg_pool1d, topk), brute force and hand-worked plans."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import select_oracle as so


def test_selection_plan_hand_worked():
    # prompt 100, keep 0.3 -> budget 30; sink 4; recent min(16, 26, 96) = 16; select 10
    assert so.selection_plan(100, 0.3, 4, 16) == (30, 4, 84, 10)
    # short prompt: the budget is spent on sinks, then recents
    assert so.selection_plan(10, 0.5, 4, 16) == (5, 4, 9, 0)
    # keep everything: nothing to select
    assert so.selection_plan(40, 1.0, 4, 16) == (40, 4, 24, 20)
    from phasekv_amd.prompt_tier import selection_plan
    for args in ((100, 0.3, 4, 16), (10, 0.5, 4, 16), (40, 1.0, 4, 16), (7, 0.1, 0, 3),
                 (4096, 0.25, 4, 32), (33, 0.5, 40, 8)):
        assert selection_plan(*args) == so.selection_plan(*args)


def _attn(seed, B=2, hq=8, q=40, kv=40):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, hq, q, kv)).astype(np.float32) * 3
    e = np.exp(x - x.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(np.float32)


def test_votes_equal_torch_sums():
    a = _attn(1)
    got = so.observation_votes(a, 2, 8)
    t = torch.from_numpy(a)[:, :, -8:, :].float().sum(dim=2).view(2, 2, 4, 40).sum(dim=2)
    np.testing.assert_allclose(got, t.numpy(), rtol=1e-6, atol=1e-7)
    # one query head per kv head and a one-row window: the votes are that row exactly
    assert np.array_equal(so.observation_votes(a, 8, 1), a[:, :, -1, :])


@pytest.mark.parametrize("mode", ["maxpool", "avgpool"])
@pytest.mark.parametrize("k", [1, 2, 3, 5, 7, 8])
def test_pooling_equals_torch(mode, k):
    rng = np.random.default_rng(k)
    s = rng.standard_normal((3, 4, 50)).astype(np.float32)
    got = so.pool_scores(s, k, mode)
    if k <= 1:
        assert np.array_equal(got, s)
        return
    x = torch.from_numpy(s).reshape(12, 1, 50)
    f = F.max_pool1d if mode == "maxpool" else F.avg_pool1d
    want = f(x, kernel_size=k, stride=1, padding=k // 2)[..., :50].reshape(3, 4, 50).numpy()
    if mode == "maxpool":
        assert np.array_equal(got, want)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
    if mode == "maxpool":   # brute-force window max
        for j in (0, 1, 25, 48, 49):
            lo, hi = max(0, j - k // 2), min(50, j - k // 2 + k)
            assert got[1, 2, j] == s[1, 2, lo:hi].max()


def test_maxpool_propagates_nan():
    s = np.arange(10, dtype=np.float32)[None, None]
    s[0, 0, 4] = np.nan
    got = so.pool_scores(s, 3, "maxpool")
    assert np.isnan(got[0, 0, 3:6]).all() and not np.isnan(got[0, 0, [2, 6]]).any()


def test_topk_ties_and_nan_by_brute_force():
    rng = np.random.default_rng(3)
    for _ in range(200):
        n = int(rng.integers(1, 12))
        k = int(rng.integers(1, n + 1))
        vals = rng.choice(np.array([0.5, 1.0, 2.0, np.nan], np.float32), size=n)

        def above(u, t):
            nu, nt = vals[u], vals[t]
            if np.isnan(nu) != np.isnan(nt):
                return bool(np.isnan(nu))
            if np.isnan(nu) or nu == nt:
                return u < t
            return nu > nt
        kept = [t for t in range(n) if sum(above(u, t) for u in range(n)) < k]
        assert so.topk_sorted(vals[None], k)[0].tolist() == kept


@pytest.mark.parametrize("pooling,kernel", [("maxpool", 5), ("avgpool", 5), ("avgpool", 4),
                                            ("maxpool", 1)])
@pytest.mark.parametrize("seed", range(3))
def test_kept_positions_equal_the_torch_pipeline(seed, pooling, kernel):
    """Against the torch calls of select_prompt_indices.  Max pooling repeats a window's
    maximum over neighbouring candidates, so exact ties are common; torch.topk does not fix
    which tied candidate it returns, so there the selected score multiset must be torch's
    and ties must resolve to the earlier position.  Elsewhere the positions are equal."""
    rng = np.random.default_rng(seed)
    B, hkv, g, L = 2, 2, 3, int(rng.integers(30, 90))
    a = _attn(seed, B, hkv * g, L, L)
    kw = dict(prompt_len=L, prefill_keep_ratio=0.4, sink_tokens=3, obs_window=8,
              pool_kernel=kernel, pooling=pooling)
    got = so.select_prompt_indices([a], num_kv_heads=hkv, **kw)[0]
    budget, sink, rs, k = so.selection_plan(L, 0.4, 3, 8)
    t = torch.from_numpy(a)
    votes = t[:, :, -8:, :].float().sum(dim=2).view(B, hkv, g, L).sum(dim=2)
    cand = votes[..., sink:rs]
    if kernel > 1:
        f = F.max_pool1d if pooling == "maxpool" else F.avg_pool1d
        cand = f(cand.reshape(B * hkv, 1, rs - sink), kernel_size=kernel, stride=1,
                 padding=kernel // 2)[..., :rs - sink].reshape(B, hkv, rs - sink)
    top = cand.topk(k, dim=-1).indices + sink
    want = torch.cat([torch.arange(sink).expand(B, hkv, -1), top,
                      torch.arange(rs, L).expand(B, hkv, -1)], dim=-1).sort(dim=-1).values
    assert (np.diff(got, axis=-1) > 0).all() and got.shape[-1] == budget
    if pooling == "maxpool" and kernel > 1:
        c = cand.numpy()
        for b in range(B):
            for h in range(hkv):
                mine = got[b, h, sink:sink + k] - sink
                theirs = want[b, h, sink:sink + k].numpy() - sink
                assert np.array_equal(np.sort(c[b, h, mine]), np.sort(c[b, h, theirs]))
                thr = np.sort(c[b, h])[::-1][k - 1]
                tied = np.nonzero(c[b, h] == thr)[0]
                n_tied = int((c[b, h, mine] == thr).sum())
                assert np.array_equal(np.sort(mine[c[b, h, mine] == thr]), tied[:n_tied])
    else:
        assert np.array_equal(got, want.numpy())
