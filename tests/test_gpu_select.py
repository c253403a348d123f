"""Prefill prompt selection on the GPU against the oracle: votes bit-exact, kept positions
identical (ties included), across dtypes, pooling modes and plans."""
import numpy as np
import pytest
import torch

from oracle import select_oracle as so

pytestmark = pytest.mark.gpu


class _Cfg:
    def __init__(self, hkv):
        self.num_key_value_heads = hkv
        self.num_attention_heads = 4 * hkv


def _attn(seed, B, hq, q, kv):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, hq, q, kv, generator=g) * 3
    return torch.softmax(x, dim=-1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_votes_bit_exact(gpu, dtype):
    from phasekv_amd.prompt_tier import prompt_votes
    a = _attn(1, 2, 12, 50, 300).to(dtype)
    got = prompt_votes(a.to(gpu), 4, 16).cpu().numpy()
    want = so.observation_votes(a.float().numpy(), 4, 16)
    assert np.array_equal(got, want)
    # a strided view (the last 20 query rows of a longer attention) is read in place
    got = prompt_votes(a.to(gpu)[:, :, 30:, :], 4, 8).cpu().numpy()
    assert np.array_equal(got, so.observation_votes(a[:, :, 30:].float().numpy(), 4, 8))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,hq,hkv,kv", [(2, 16, 8, 4096), (1, 28, 4, 8192), (1, 6, 2, 998),
                                          (1, 4, 4, 2048), (2, 40, 2, 1024)])
def test_votes_bit_exact_per_load_width(gpu, dtype, B, hq, hkv, kv):
    """16-bit attention takes 4 keys per lane when that gives every CU a workgroup
    (2 x 8 kv heads x 4096 keys), else 2 (C4's 4 kv heads x 8192) or 1 (rows of 998 keys);
    query heads per kv head 1 (one wave) to 20 (16 waves, some with two heads).  Windows
    of 24, 64 and 70 rows: below, at and past the 32 (2 keys per lane) or 16 (4 keys)
    rows of raw loads a wave keeps in flight, with a tail of converted loads."""
    from phasekv_amd.prompt_tier import prompt_votes
    a = _attn(B + kv, B, hq, 70, kv).to(dtype)
    for w in (24, 64, 70):
        print(f"case B={B} hq={hq} hkv={hkv} kv={kv} {dtype} w={w}", flush=True)
        got = prompt_votes(a.to(gpu), hkv, w).cpu().numpy()
        assert np.array_equal(got, so.observation_votes(a.float().numpy(), hkv, w)), w


@pytest.mark.parametrize("pooling,kernel", [("maxpool", 7), ("avgpool", 7), ("maxpool", 4),
                                            ("avgpool", 2), ("maxpool", 1)])
@pytest.mark.parametrize("L,ratio,sink,obs", [(300, 0.3, 4, 32), (2048, 0.1, 4, 64),
                                              (37, 0.5, 40, 8), (100, 1.0, 4, 16),
                                              (513, 0.02, 0, 8)])
def test_kept_positions_match_the_oracle(gpu, pooling, kernel, L, ratio, sink, obs):
    from phasekv_amd.prompt_tier import select_prompt_indices
    print(f"case L={L} ratio={ratio} sink={sink} obs={obs} {pooling} {kernel}", flush=True)
    B, hkv, g = 2, 4, 7
    attns = [_attn(L + i, B, hkv * g, min(L, 96), L) for i in range(2)]
    kw = dict(prompt_len=L, prefill_keep_ratio=ratio, sink_tokens=sink, obs_window=obs,
              pool_kernel=kernel, pooling=pooling)
    got = select_prompt_indices([a.to(gpu) for a in attns], model_config=_Cfg(hkv), **kw)
    want = so.select_prompt_indices([a.numpy() for a in attns], num_kv_heads=hkv, **kw)
    for gl, wl in zip(got, want):
        assert gl.dtype == torch.int64 and tuple(gl.shape) == wl.shape
        assert np.array_equal(gl.cpu().numpy(), wl)


def test_ties_keep_the_earliest_positions(gpu):
    """Uniform attention: every candidate's vote is equal, so the earliest are kept."""
    from phasekv_amd.prompt_tier import select_prompt_indices
    a = torch.full((1, 2, 10, 64), 1.0 / 64)
    got = select_prompt_indices([a.to(gpu)], prompt_len=64, model_config=_Cfg(1),
                                prefill_keep_ratio=0.25, sink_tokens=2, obs_window=4,
                                pool_kernel=3, pooling="maxpool")[0]
    assert got.cpu().tolist() == [[list(range(0, 12)) + list(range(60, 64))]]


def test_errors(gpu):
    from phasekv_amd.prompt_tier import select_prompt_indices
    a = torch.zeros(1, 2, 4, 16, device=gpu)
    with pytest.raises(ValueError, match="pooling"):
        select_prompt_indices([a], prompt_len=16, model_config=_Cfg(2), prefill_keep_ratio=0.5,
                              sink_tokens=1, obs_window=2, pool_kernel=3, pooling="median")
    with pytest.raises(ValueError, match="key length"):
        select_prompt_indices([a], prompt_len=15, model_config=_Cfg(2), prefill_keep_ratio=0.5,
                              sink_tokens=1, obs_window=2, pool_kernel=3, pooling="maxpool")


@pytest.mark.parametrize("pooling,kernel", [("maxpool", 7), ("avgpool", 5)])
@pytest.mark.parametrize("L", [20000, 32768])
def test_long_prompts_beyond_the_lds_staging(gpu, pooling, kernel, L):
    """Rows of more than 18432 candidates: the kernel recomputes the pooled keys from the
    global votes on every radix and scan pass instead of staging them in LDS."""
    from phasekv_amd.prompt_tier import select_prompt_indices
    print(f"case L={L} {pooling} {kernel}", flush=True)
    B, hkv, g, obs = 1, 2, 4, 32
    attns = [_attn(L + 7, B, hkv * g, obs, L)]
    kw = dict(prompt_len=L, prefill_keep_ratio=0.1, sink_tokens=4, obs_window=obs,
              pool_kernel=kernel, pooling=pooling)
    got = select_prompt_indices([a.to(gpu) for a in attns], model_config=_Cfg(hkv), **kw)
    want = so.select_prompt_indices([a.numpy() for a in attns], num_kv_heads=hkv, **kw)
    for gl, wl in zip(got, want):
        assert gl.dtype == torch.int64 and tuple(gl.shape) == wl.shape
        assert np.array_equal(gl.cpu().numpy(), wl)
