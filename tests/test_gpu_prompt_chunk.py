"""Causal attention of a whole input chunk over the packed cache in one pass, against the
per-token loop the reference's adapter runs (one decode per chunk token over the tiers as
they stand after that token's append), in the oracle and in this library."""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import attention_oracle as ao
from oracle import packing_oracle as po

pytestmark = pytest.mark.gpu


class _Dense:
    def __init__(self, keys, values):
        self.key_cache, self.value_cache = keys, values


def _segments(tiers, hot_rows):
    segs = []
    for seg in [tiers.prompt, *tiers.prompt_extensions, *tiers.cold]:
        k = po.dequantize_float(po.PackedArrays(
            seg.key.packed.cpu().numpy(), seg.key.scale.cpu().numpy(), seg.key.mins.cpu().numpy(),
            seg.key.bits, seg.key.axis, seg.key.group_size, tuple(seg.key.orig_shape),
            seg.key.axis_len))[0]
        v = po.dequantize_float(po.PackedArrays(
            seg.value.packed.cpu().numpy(), seg.value.scale.cpu().numpy(),
            seg.value.mins.cpu().numpy(), seg.value.bits, seg.value.axis, seg.value.group_size,
            tuple(seg.value.orig_shape), seg.value.axis_len))[0]
        segs.append((k, v))
    hk, hv = tiers.hot_k[0, :, :hot_rows].cpu().numpy(), tiers.hot_v[0, :, :hot_rows].cpu().numpy()
    segs.append((hk, hv))
    return segs


@pytest.mark.parametrize("hq,hkv,hd,T,decode_steps", [
    (28, 4, 128, 5, 20), (28, 4, 128, 37, 60), (8, 2, 64, 1, 3), (8, 2, 64, 24, 0),
    (32, 8, 128, 16, 50),
])
def test_chunk_attention_matches_the_per_token_loop(gpu, hq, hkv, hd, T, decode_steps):
    from phasekv_amd.cache import PhaseKVCache
    from phasekv_amd.kernels.attention_triton import (fused_phasekv_decode,
                                                      fused_phasekv_prompt_chunk_attention)
    print(f"case hq={hq} hkv={hkv} hd={hd} T={T} steps={decode_steps}", flush=True)
    g = torch.Generator().manual_seed(T + hd + decode_steps)
    S = 300
    k = (torch.randn(1, hkv, S, hd, generator=g) * 2).to(torch.float16).to(gpu)
    v = torch.randn(1, hkv, S, hd, generator=g).to(torch.float16).to(gpu)
    cache = PhaseKVCache.from_dense_prefill(_Dense([k], [v]), prompt_len=S, prompt_bits=2,
                                            cold_bits=4, decode_keep_ratio=0.5)
    for _ in range(decode_steps):
        t = torch.randn(1, hkv, 1, hd, generator=g).to(torch.float16).to(gpu)
        cache.append_hot(0, t, t * 0.5)
        cache.finish_decode_step()
    cache.begin_prompt_chunk(T)
    ck = (torch.randn(1, hkv, T, hd, generator=g) * 2).to(torch.float16).to(gpu)
    cv = torch.randn(1, hkv, T, hd, generator=g).to(torch.float16).to(gpu)
    for t in range(T):
        cache.append_prompt_token(0, ck[:, :, t:t + 1], cv[:, :, t:t + 1])
    tiers = cache.layer_tiers(0)
    start = tiers.hot_len - T
    q = torch.randn(T, hq, hd, generator=g).to(torch.float16)
    out = fused_phasekv_prompt_chunk_attention(q.to(gpu), tiers, hq).float().cpu().numpy()
    for method in ("heads", "batch"):
        other = fused_phasekv_prompt_chunk_attention(q.to(gpu), tiers, hq, method=method)
        np.testing.assert_allclose(other.float().cpu().numpy(), out, atol=1e-3, rtol=1e-2)
    loop = np.stack([fused_phasekv_decode(q[t].to(gpu), dataclasses.replace(tiers, hot_len=start + t + 1),
                                          hq).float().cpu().numpy() for t in range(T)])
    want = np.stack([ao.segments_attention(q[t].numpy(), _segments(tiers, start + t + 1), hq)
                     for t in range(T)])
    np.testing.assert_allclose(out, want, atol=2e-3, rtol=1e-2)
    np.testing.assert_allclose(out, loop, atol=1e-3, rtol=1e-2)
    cache.finish_prompt_chunk()


def test_chunk_attention_rejects_a_chunk_longer_than_the_window(gpu):
    from phasekv_amd.cache import PhaseKVCache
    from phasekv_amd.kernels.attention_triton import fused_phasekv_prompt_chunk_attention
    k = torch.randn(1, 2, 64, 64).to(torch.float16).to(gpu)
    cache = PhaseKVCache.from_dense_prefill(_Dense([k], [k]), prompt_len=64)
    q = torch.zeros(3, 8, 64, dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError, match="last rows"):
        fused_phasekv_prompt_chunk_attention(q, cache.layer_tiers(0), 8)


def test_chunk_attention_graph_replays_take_the_heads_form(gpu):
    """Under graph capture ``auto`` takes the heads form from a smaller chunk than in an
    eager call (no host cost per replay): a 128-token chunk over a 4K-token cache is
    eager batch and captured heads.  The captured call finds the per-stream workspace
    sized for the batch form and takes its own buffer from the graph's pool; every
    replay, with eager work in between, matches an eager heads call bit for bit."""
    from phasekv_amd.cache import PhaseKVCache
    from phasekv_amd.kernels import attention_triton as at
    g = torch.Generator().manual_seed(41)
    hq, hkv, hd, S, T = 28, 4, 128, 4096, 128
    k = torch.randn(1, hkv, S, hd, generator=g).to(torch.float16).to(gpu)
    v = torch.randn(1, hkv, S, hd, generator=g).to(torch.float16).to(gpu)
    cache = PhaseKVCache.from_dense_prefill(_Dense([k], [v]), prompt_len=S, prompt_bits=2)
    cache.begin_prompt_chunk(T)
    ck = torch.randn(1, hkv, T, hd, generator=g).to(torch.float16).to(gpu)
    cv = torch.randn(1, hkv, T, hd, generator=g).to(torch.float16).to(gpu)
    cache.append_prompt_chunk(0, ck, cv)
    tiers = cache.layer_tiers(0)
    context = tiers.hot_len + sum(s.key.orig_shape[-2] for s in [tiers.prompt, *tiers.cold])
    work = T * context * hkv * hd
    assert at.CHUNK_HEADS_MIN_WORK <= work < at.CHUNK_HEADS_MIN_WORK_EAGER
    q = torch.randn(T, hq, hd, generator=g).to(torch.float16).to(gpu)
    heads = at.fused_phasekv_prompt_chunk_attention(q, tiers, hq, method="heads")
    batch = at.fused_phasekv_prompt_chunk_attention(q, tiers, hq, method="batch")
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        eager = at.fused_phasekv_prompt_chunk_attention(q, tiers, hq)     # batch, eager
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = at.fused_phasekv_prompt_chunk_attention(q, tiers, hq)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(eager, batch)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        junk = torch.randn(1 << 20, device=gpu).sum()    # eager work between replays
        assert torch.equal(out, heads)
        del junk
    np.testing.assert_allclose(out.float().cpu().numpy(), batch.float().cpu().numpy(),
                               atol=1e-3, rtol=1e-2)
    cache.finish_prompt_chunk()
