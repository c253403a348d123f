"""Device-resident segment table: a decode over many cold segments is one partials launch.

The reference appends one cold segment per cooling event (phasekv_cache.py:322-340) and
launches once per segment (attention_triton.py:662-665).  Here the cold segments' descriptors
live in device memory and the decode reads them from there; these tests check the result
against the oracle over the same packed tiers, the launch structure, the incremental
extension across cooling events and the C ABI's checks.
"""
import ctypes
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import attention_oracle as ao
from oracle import cache_oracle as co
from oracle import packing_oracle as po

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _np_pt(pt):
    return po.PackedArrays(pt.packed.cpu().numpy(), pt.scale.cpu().numpy(), pt.mins.cpu().numpy(),
                           pt.bits, pt.axis, pt.group_size, tuple(pt.orig_shape), pt.axis_len)


def _oracle_tiers(t):
    seg = lambda s: ao.SegmentArrays(_np_pt(s.key), _np_pt(s.value))
    hk, hv = t.hot_views()
    return ao.LayerTiersArrays(seg(t.prompt), [seg(s) for s in t.prompt_extensions],
                               [seg(s) for s in t.cold], hk.cpu().numpy(), hv.cpu().numpy())


def _rand(g, *shape):
    return torch.randn(*shape, generator=g).to(torch.float16)


def _long_generation_tiers(gpu, g, batch, hkv, hd, prompt, cold_lens, cold_bits, hot):
    """A cache after a long generation: a 2-bit prompt, many short cold segments (the
    output of lazy cooling, packed like pack_kv packs them) and an FP16 window."""
    from phasekv_amd.tiers import LayerTiers, pack_kv
    p = pack_kv(_rand(g, batch, hkv, prompt, hd).to(gpu), _rand(g, batch, hkv, prompt, hd).to(gpu),
                2, 32)
    cold = []
    for i, n in enumerate(cold_lens):
        bits = cold_bits[i % len(cold_bits)]
        kb, vb = bits if isinstance(bits, tuple) else (bits, bits)
        seg = pack_kv(_rand(g, batch, hkv, n, hd).to(gpu), _rand(g, batch, hkv, n, hd).to(gpu),
                      kb, 32)
        if vb != kb:
            other = pack_kv(_rand(g, batch, hkv, n, hd).to(gpu),
                            _rand(g, batch, hkv, n, hd).to(gpu), vb, 32)
            seg = replace(seg, value=other.value)
        cold.append(seg)
    hot_k = torch.zeros(batch, hkv, hot + 8, hd, dtype=torch.float16, device=gpu)
    hot_v = torch.zeros_like(hot_k)
    hot_k[:, :, :hot] = _rand(g, batch, hkv, hot, hd).to(gpu)
    hot_v[:, :, :hot] = _rand(g, batch, hkv, hot, hd).to(gpu)
    return LayerTiers(p, [], cold, hot_k, hot_v, hot)


def test_64_cold_segments_in_one_partials_launch(gpu):
    """C2's shape after about 1024 generated tokens (64 cold segments of 16 tokens at
    4 bits, lazy_g 16): the packed segments beyond one launch's list go to the device
    table, the step is one partials launch, and the output matches the oracle and the
    per-8-segment launches of the segment list alone."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.attention_triton import _reused_problem, fused_phasekv_decode
    g = torch.Generator().manual_seed(11)
    hq, hkv, hd = 28, 4, 128
    tiers = _long_generation_tiers(gpu, g, 1, hkv, hd, 4096, [16] * 64, [4], 40)
    q = _rand(g, hq, hd).to(gpu)
    out = fused_phasekv_decode(q, tiers, hq)
    problem = _reused_problem(q, tiers, hq)
    assert problem.table is not None and problem.table.count == 64
    assert problem.c.num_segments == 2 <= dec._lib.PK_MAX_SEGMENTS_PER_LAUNCH   # prompt + hot
    want = ao.layer_tiers_attention(q.cpu().numpy(), _oracle_tiers(tiers), hq)
    np.testing.assert_allclose(out.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
    # the same segments as one list (nine partials launches)
    segs = [problem.segments[0], *problem.table.segments, problem.segments[1]]
    inline = dec.fused_decode(dec.Problem(q, segs, hq))[0]
    np.testing.assert_allclose(out.float().cpu().numpy(), inline.float().cpu().numpy(),
                               atol=1e-3, rtol=1e-2)


@pytest.mark.parametrize("hd", [64, 128])
def test_table_of_mixed_widths_and_lengths(gpu, hd):
    """Cold segments of every 2/4-bit K/V pair and of 1 to 100 tokens (one and several
    32-token groups, ragged last groups) in one table, plus prompt extensions kept in
    the launch's own list."""
    from phasekv_amd.kernels.attention_triton import fused_phasekv_decode, phasekv_problem
    from phasekv_amd.tiers import pack_kv
    g = torch.Generator().manual_seed(hd)
    hq, hkv = 16, 2
    lens = [1, 7, 16, 31, 32, 33, 48, 64, 65, 100, 5, 16, 24]
    widths = [(2, 2), (2, 4), (4, 2), (4, 4)]
    tiers = _long_generation_tiers(gpu, g, 1, hkv, hd, 700, lens, widths, 21)
    tiers.prompt_extensions = [pack_kv(_rand(g, 1, hkv, n, hd).to(gpu),
                                       _rand(g, 1, hkv, n, hd).to(gpu), 2, 32) for n in (40, 9)]
    q = _rand(g, hq, hd).to(gpu)
    problem = phasekv_problem(q, tiers, hq)
    assert problem.table is not None and problem.table.count == len(lens)
    out = fused_phasekv_decode(q, tiers, hq).float().cpu().numpy()
    want = ao.layer_tiers_attention(q.cpu().numpy(), _oracle_tiers(tiers), hq)
    np.testing.assert_allclose(out, want, atol=ATOL, rtol=RTOL)


def test_batched_ragged_rows_over_a_table(gpu):
    """Batch 3 with ragged prompt rows and 20 cold segments in the table."""
    from phasekv_amd.kernels.attention_triton import fused_phasekv_decode_batched, phasekv_problem
    g = torch.Generator().manual_seed(3)
    hq, hkv, hd, B = 28, 4, 128, 3
    tiers = _long_generation_tiers(gpu, g, B, hkv, hd, 512, [16] * 20, [2, 4], 33)
    lens = torch.tensor([512, 300, 97], dtype=torch.int32, device=gpu)
    q = _rand(g, B, hq, hd).to(gpu)
    assert phasekv_problem(q, tiers, hq, batched=True, prompt_lens=lens).table.count == 20
    out = fused_phasekv_decode_batched(q, tiers, hq, lens).float().cpu().numpy()
    t = _oracle_tiers(tiers)
    for b, L in enumerate(lens.tolist()):
        cut = lambda pt, n, ax: po.PackedArrays(
            pt.packed[b:b + 1, :, :, :-(-n // (8 // pt.bits))] if ax == 2 else pt.packed[b:b + 1, :, :n],
            pt.scale[b:b + 1, :, :, :-(-n // pt.group_size)] if ax == 2 else pt.scale[b:b + 1, :, :n],
            pt.mins[b:b + 1, :, :, :-(-n // pt.group_size)] if ax == 2 else pt.mins[b:b + 1, :, :n],
            pt.bits, ax, pt.group_size, (1,) + pt.orig_shape[1:2] + (n,) + pt.orig_shape[3:],
            n if ax == 2 else pt.axis_len)
        sl = lambda pt: po.PackedArrays(pt.packed[b:b + 1], pt.scale[b:b + 1], pt.mins[b:b + 1],
                                        pt.bits, pt.axis, pt.group_size,
                                        (1,) + tuple(pt.orig_shape[1:]), pt.axis_len)
        row = ao.LayerTiersArrays(
            ao.SegmentArrays(cut(t.prompt.key, L, 2), cut(t.prompt.value, L, 3)), [],
            [ao.SegmentArrays(sl(s.key), sl(s.value)) for s in t.cold],
            t.hot_k[b:b + 1], t.hot_v[b:b + 1])
        want = ao.layer_tiers_attention(q[b].cpu().numpy(), row, hq)
        np.testing.assert_allclose(out[b], want, atol=ATOL, rtol=RTOL)


class _Dense:
    def __init__(self, keys, values):
        self.key_cache, self.value_cache = keys, values


def test_cooling_events_extend_the_table_in_place(gpu):
    """A decode loop with lazy cooling every 4 steps: once the segments exceed one launch's
    list the cold segments move to a table, which later cooling events extend (the same
    table object, one write per new segment); every step matches the oracle."""
    from phasekv_amd.cache import PhaseKVCache
    from phasekv_amd.kernels.attention_triton import _reused_problem, fused_phasekv_decode
    g = torch.Generator().manual_seed(21)
    B, H, hq, hd, S = 1, 2, 8, 128, 96
    keys = torch.randn(B, H, S, hd, generator=g).to(torch.float16)
    values = torch.randn(B, H, S, hd, generator=g).to(torch.float16)
    keep = torch.stack([torch.randperm(S, generator=g)[:80] for _ in range(H)])[None]
    cache = PhaseKVCache.from_dense_prefill(
        _Dense([keys.to(gpu)], [values.to(gpu)]), prompt_len=S, keep_indices=[keep.to(gpu)],
        prompt_bits=2, cold_bits=4, group_size=32, recent_window=8, lazy_g=4,
        decode_keep_ratio=1.0)
    idx = np.sort(keep.numpy(), -1)
    ref_prompt = (po.quantize_pack(np.take_along_axis(keys.numpy(), idx[..., None], 2), 2, -2, 32),
                  po.quantize_pack(np.take_along_axis(values.numpy(), idx[..., None], 2), 2, -1, 32))
    ref = {"cold": [], "hot_k": np.zeros((B, H, 12, hd), np.float16),
           "hot_v": np.zeros((B, H, 12, hd), np.float16), "hot_len": 0}
    tables = []
    for step in range(60):
        nk = torch.randn(B, H, 1, hd, generator=g).to(torch.float16)
        nv = torch.randn(B, H, 1, hd, generator=g).to(torch.float16)
        cache.append_hot(0, nk.to(gpu), nv.to(gpu))
        ref["hot_len"] = co.append_hot(ref["hot_k"], ref["hot_v"], ref["hot_len"], nk.numpy(),
                                       nv.numpy())
        cache.finish_decode_step()
        seg, ref["hot_len"], _ = co.cool_aged_tokens(ref["hot_k"], ref["hot_v"], ref["hot_len"],
                                                     8, 4, 1.0, 4, 32)
        if seg is not None:
            ref["cold"].append(seg)
        tiers = cache.layer_tiers(0)
        q = torch.randn(hq, hd, generator=g).to(torch.float16)
        out = fused_phasekv_decode(q.to(gpu), tiers, hq).float().cpu().numpy()
        segs = [(po.dequantize_float(ref_prompt[0])[0], po.dequantize_float(ref_prompt[1])[0])]
        segs += [(po.dequantize_float(a)[0], po.dequantize_float(b)[0]) for a, b in ref["cold"]]
        if ref["hot_len"]:
            segs.append((ref["hot_k"][0, :, :ref["hot_len"]], ref["hot_v"][0, :, :ref["hot_len"]]))
        want = ao.segments_attention(q.numpy(), segs, hq)
        np.testing.assert_allclose(out, want, atol=ATOL, rtol=RTOL, err_msg=f"step {step}")
        table = _reused_problem(q.to(gpu), tiers, hq).table
        if table is not None:
            tables.append(table)
    assert len(cache.layer_tiers(0).cold) > 12
    assert tables and all(t is tables[0] for t in tables)
    assert tables[-1].count == len(cache.layer_tiers(0).cold)


def test_graph_replays_over_a_table_match_eager(gpu):
    from phasekv_amd.kernels.attention_triton import fused_phasekv_decode
    g = torch.Generator().manual_seed(5)
    hq, hkv, hd = 28, 4, 128
    tiers = _long_generation_tiers(gpu, g, 1, hkv, hd, 2048, [16] * 30, [4], 35)
    q = _rand(g, hq, hd).to(gpu)
    eager = fused_phasekv_decode(q, tiers, hq)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fused_phasekv_decode(q, tiers, hq)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            out = fused_phasekv_decode(q, tiers, hq)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        junk = torch.randn(1000, device=gpu).sum()
        assert torch.equal(out, eager)
        del junk


def test_table_write_refuses_other_storage(gpu):
    """pk_segment_table_write takes only what the wave path reads; the rest fails with
    PK_ERR_INVALID before anything is written."""
    from phasekv_amd import _lib
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(9)
    k, v = _rand(g, 2, 16, 128).to(gpu), _rand(g, 2, 16, 128).to(gpu)
    table = torch.zeros(4 * _lib.load().pk_segment_table_entry_bytes(), dtype=torch.uint8,
                        device=gpu)
    good = dec.packed_segment(quantize_pack(k, 4, -2, 32), quantize_pack(v, 4, -1, 32),
                              batched=False)
    assert dec.table_eligible(good)
    channel_major = dec.packed_segment(quantize_pack(k, 4, -2, 32), quantize_pack(v, 4, -1, 32),
                                       batched=False)
    channel_major.desc.k_data_layout = _lib.PK_CODES_CHANNEL_MAJOR
    bad = [dec.packed_segment(quantize_pack(k, 8, -2, 32), quantize_pack(v, 8, -1, 32),
                              batched=False),                        # 8-bit codes
           channel_major,                                            # channel-major K codes
           dec.fp16_segment(k, v, batched=False)]                    # uncompressed
    lib = _lib.load()
    for sg in bad:
        assert not dec.table_eligible(sg)
        arr = (_lib.PkSegment * 1)(sg.desc)
        rc = lib.pk_segment_table_write(table.data_ptr(), 0, 1, arr, 128, _lib.stream_ptr(gpu))
        assert rc == _lib.PK_ERR_INVALID, lib.pk_last_error()
    torch.cuda.synchronize()
    assert int(table.sum()) == 0                                     # nothing written
    arr = (_lib.PkSegment * 1)(good.desc)
    assert lib.pk_segment_table_write(table.data_ptr(), 0, 1, arr, 100, None) == _lib.PK_ERR_INVALID
