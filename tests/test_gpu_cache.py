"""The HIP hot window lifecycle against the oracle: appends, the cooling launch (kept
indices, gathered rows, shifted tail) bit-exact, and a multi-layer decode loop whose
cold segments, hot windows and attention output match the oracle's."""
import numpy as np
import pytest
import torch

from oracle import attention_oracle as ao
from oracle import cache_oracle as co
from oracle import packing_oracle as po

pytestmark = pytest.mark.gpu


def _np_pt(pt):
    return po.PackedArrays(pt.packed.cpu().numpy(), pt.scale.cpu().numpy(), pt.mins.cpu().numpy(),
                           pt.bits, pt.axis, pt.group_size, tuple(pt.orig_shape), pt.axis_len)


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


@pytest.mark.parametrize("B,H,hd,cap,hot_len,aged,keep", [
    (1, 4, 128, 48, 48, 16, 8), (2, 3, 64, 48, 48, 16, 16), (1, 2, 256, 80, 70, 30, 1),
    (3, 2, 96, 40, 33, 17, 9), (1, 1, 128, 700, 640, 300, 150), (2, 2, 128, 48, 16, 16, 5),
])
def test_cool_hot_matches_the_oracle(gpu, B, H, hd, cap, hot_len, aged, keep):
    from phasekv_amd.cache import cool_hot
    print(f"case B={B} H={H} hd={hd} hot_len={hot_len} aged={aged} keep={keep}", flush=True)
    rng = np.random.default_rng(hd + aged + keep)
    k = (rng.standard_normal((B, H, cap, hd)) * 2).astype(np.float16)
    v = rng.standard_normal((B, H, cap, hd)).astype(np.float16)
    if B * H > 1:
        v[0, 0, 1] = v[0, 0, 0]          # an exact tie of norms (the earlier token wins)
    hk, hv = torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu)
    kept_k, kept_v, idx = cool_hot(hk, hv, hot_len, aged, keep, with_index=True)
    if keep < aged:
        want_idx = co.select_kept(co.value_norms(v[:, :, :aged]), keep)
    else:
        want_idx = np.broadcast_to(np.arange(aged), (B, H, aged))
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    want_k = np.take_along_axis(k[:, :, :aged], want_idx[..., None], axis=2)
    want_v = np.take_along_axis(v[:, :, :aged], want_idx[..., None], axis=2)
    assert np.array_equal(_u16(kept_k), want_k.view(np.int16))
    assert np.array_equal(_u16(kept_v), want_v.view(np.int16))
    rem = hot_len - aged
    assert np.array_equal(_u16(hk[:, :, :rem]), k[:, :, aged:hot_len].view(np.int16))
    assert np.array_equal(_u16(hv[:, :, :rem]), v[:, :, aged:hot_len].view(np.int16))
    # rows past the old hot length are untouched
    assert np.array_equal(_u16(hk[:, :, hot_len:]), k[:, :, hot_len:].view(np.int16))


def test_cool_hot_nan_rows_rank_first(gpu):
    from phasekv_amd.cache import cool_hot
    v = np.ones((1, 1, 20, 64), np.float16)
    v[0, 0, 9, 3] = np.nan
    v[0, 0, 4] = 2
    k = np.zeros_like(v)
    hk, hv = torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu)
    _, _, idx = cool_hot(hk, hv, 20, 16, 3, with_index=True)
    assert idx.cpu().numpy().tolist() == [[[0, 4, 9]]]
    assert co.select_kept(co.value_norms(v[:, :, :16]), 3).tolist() == [[[0, 4, 9]]]


def test_append_hot_writes_one_row(gpu):
    from phasekv_amd import _lib
    rng = np.random.default_rng(3)
    hot = torch.zeros(2, 3, 10, 64, dtype=torch.float16, device=gpu)
    hot_v = torch.zeros_like(hot)
    src = torch.from_numpy(rng.standard_normal((2, 3, 1, 64)).astype(np.float16)).to(gpu)
    src_v = src * 2
    lib = _lib.load()
    _lib.check(lib.pk_append_hot(src.data_ptr(), src_v.data_ptr(), src.stride(0), src.stride(1),
                                 src_v.stride(0), src_v.stride(1), hot.data_ptr(),
                                 hot_v.data_ptr(), hot.stride(0), hot.stride(1), hot.stride(2),
                                 2, 3, 64, 7, 10, _lib.stream_ptr(hot.device)), "append_hot")
    want = torch.zeros(2, 3, 10, 64, dtype=torch.float16)
    want[:, :, 7:8] = src.cpu()
    assert torch.equal(hot.cpu(), want)
    want[:, :, 7:8] = src_v.cpu()
    assert torch.equal(hot_v.cpu(), want)
    with pytest.raises(ValueError, match="full"):
        _lib.check(lib.pk_append_hot(src.data_ptr(), src_v.data_ptr(), 0, 0, 0, 0, hot.data_ptr(),
                                     hot_v.data_ptr(), hot.stride(0), hot.stride(1), hot.stride(2),
                                     2, 3, 64, 10, 10, _lib.stream_ptr(hot.device)), "append_hot")


class _Dense:
    def __init__(self, keys, values):
        self.key_cache, self.value_cache = keys, values


@pytest.mark.parametrize("ratio,cold_bits", [(1.0, 4), (0.5, 2), (0.3, 8)])
def test_decode_loop_matches_the_oracle(gpu, ratio, cold_bits):
    """Two layers, a selected prompt, 70 decode steps (cooling at steps 48 and 64): cold
    segments and hot windows bit-exact, and the packed decode over the cache within the
    attention tolerance of the oracle over the oracle's cache."""
    from phasekv_amd.cache import PhaseKVCache
    from phasekv_amd.kernels.attention_triton import fused_phasekv_decode
    print(f"case ratio={ratio} cold_bits={cold_bits}", flush=True)
    g = torch.Generator().manual_seed(int(ratio * 10) + cold_bits)
    L, B, H, hq, hd, S = 2, 1, 2, 8, 128, 200
    keys = [torch.randn(B, H, S, hd, generator=g).to(torch.float16) for _ in range(L)]
    values = [torch.randn(B, H, S, hd, generator=g).to(torch.float16) for _ in range(L)]
    keep = [torch.stack([torch.randperm(S, generator=g)[:150] for _ in range(H)])[None]
            for _ in range(L)]
    cache = PhaseKVCache.from_dense_prefill(
        _Dense([k.to(gpu) for k in keys], [v.to(gpu) for v in values]), prompt_len=S,
        keep_indices=[i.to(gpu) for i in keep], prompt_bits=2, cold_bits=cold_bits,
        group_size=32, recent_window=32, lazy_g=16, decode_keep_ratio=ratio)
    # the oracle's cache
    ref = []
    for l in range(L):
        idx = np.sort(keep[l].numpy(), -1)
        pk = np.take_along_axis(keys[l].numpy(), idx[..., None], axis=2)
        pv = np.take_along_axis(values[l].numpy(), idx[..., None], axis=2)
        ref.append({"prompt": (po.quantize_pack(pk, 2, -2, 32), po.quantize_pack(pv, 2, -1, 32)),
                    "cold": [], "hot_k": np.zeros((B, H, 48, hd), np.float16),
                    "hot_v": np.zeros((B, H, 48, hd), np.float16), "hot_len": 0})
    for l in range(L):
        got = cache.layer_tiers(l).prompt
        assert np.array_equal(got.key.packed.cpu().numpy(), ref[l]["prompt"][0].packed)
        assert np.array_equal(got.value.packed.cpu().numpy(), ref[l]["prompt"][1].packed)
    q = torch.randn(hq, hd, generator=g).to(torch.float16)
    for step in range(70):
        for l in range(L):
            nk = torch.randn(B, H, 1, hd, generator=g).to(torch.float16)
            nv = (torch.randn(B, H, 1, hd, generator=g) * (1 + step % 5)).to(torch.float16)
            cache.append_hot(l, nk.to(gpu), nv.to(gpu))
            r = ref[l]
            r["hot_len"] = co.append_hot(r["hot_k"], r["hot_v"], r["hot_len"], nk.numpy(),
                                         nv.numpy())
        cache.finish_decode_step()
        for l in range(L):
            r = ref[l]
            seg, r["hot_len"], _ = co.cool_aged_tokens(r["hot_k"], r["hot_v"], r["hot_len"], 32,
                                                      16, ratio, cold_bits, 32)
            if seg is not None:
                r["cold"].append(seg)
    assert cache.true_seq_length == S + 70
    for l in range(L):
        tiers, r = cache.layer_tiers(l), ref[l]
        assert tiers.hot_len == r["hot_len"] == 38 and len(tiers.cold) == len(r["cold"]) == 2
        hot_k, hot_v = tiers.hot_views()
        assert np.array_equal(_u16(hot_k), r["hot_k"][:, :, :r["hot_len"]].view(np.int16))
        assert np.array_equal(_u16(hot_v), r["hot_v"][:, :, :r["hot_len"]].view(np.int16))
        for got, (wk, wv) in zip(tiers.cold, r["cold"]):
            for pt, want in ((got.key, wk), (got.value, wv)):
                assert pt.group_size == want.group_size
                assert np.array_equal(pt.packed.cpu().numpy(), want.packed)
                assert np.array_equal(_u16(pt.scale), want.scale.view(np.int16))
                assert np.array_equal(_u16(pt.mins), want.mins.view(np.int16))
        out = fused_phasekv_decode(q.to(gpu), tiers, hq).float().cpu().numpy()
        segs = [(po.dequantize_float(r["prompt"][0])[0], po.dequantize_float(r["prompt"][1])[0])]
        segs += [(po.dequantize_float(a)[0], po.dequantize_float(b)[0]) for a, b in r["cold"]]
        segs.append((r["hot_k"][0, :, :r["hot_len"]], r["hot_v"][0, :, :r["hot_len"]]))
        want = ao.segments_attention(q.numpy(), segs, hq)
        np.testing.assert_allclose(out, want, atol=2e-3, rtol=1e-2)


def test_decode_step_errors(gpu):
    from phasekv_amd.cache import PhaseKVCache
    k = torch.randn(1, 2, 64, 64).to(torch.float16).to(gpu)
    cache = PhaseKVCache.from_dense_prefill(_Dense([k, k], [k, k]), prompt_len=64,
                                            recent_window=2, lazy_g=1)
    tok = torch.zeros(1, 2, 1, 64, dtype=torch.float16, device=gpu)
    cache.append_hot(0, tok, tok)
    with pytest.raises(RuntimeError, match="already appended"):
        cache.append_hot(0, tok, tok)
    with pytest.raises(RuntimeError, match="missing layers"):
        cache.finish_decode_step()
    with pytest.raises(ValueError, match="one token"):
        cache.append_hot(1, tok[:, :, :0], tok)
    with pytest.raises(RuntimeError, match="Cache.update"):
        cache.update(tok, tok, 0)
    cache.append_hot(1, tok, tok)
    cache.finish_decode_step()
    assert cache.get_seq_length() == 65 and cache.true_seq_length == 65


@pytest.mark.parametrize("B,H,hd,cap,hot_len,aged,keep,bits,gs", [
    (1, 4, 128, 48, 48, 16, 16, 4, 32), (1, 4, 128, 48, 48, 16, 8, 2, 32),
    (2, 3, 64, 48, 40, 16, 5, 2, 32), (1, 2, 96, 64, 60, 24, 24, 8, 32),
    (2, 2, 128, 48, 48, 16, 16, 4, 4), (1, 2, 128, 48, 48, 16, 12, 2, 5),
    (1, 1, 64, 40, 17, 17, 3, 4, 2), (1, 2, 256, 80, 70, 30, 7, 4, 32),
])
def test_cool_pack_hot_matches_cool_then_quantize(gpu, B, H, hd, cap, hot_len, aged, keep, bits, gs):
    """The fused cooling + packing launch against the oracle's selection, gather and
    quantize_pack, bit for bit, with the same shapes and views as quantize_pack's output;
    the last case does not fit one workgroup's LDS and takes the three-launch path."""
    from phasekv_amd.cache import cool_pack_hot, cool_pack_supported
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case B={B} H={H} hd={hd} hot_len={hot_len} aged={aged} keep={keep} bits={bits} "
          f"gs={gs}", flush=True)
    rng = np.random.default_rng(hd * 7 + keep * 3 + bits)
    k = (rng.standard_normal((B, H, cap, hd)) * 2).astype(np.float16)
    v = rng.standard_normal((B, H, cap, hd)).astype(np.float16)
    hk, hv = torch.from_numpy(k).to(gpu), torch.from_numpy(v).to(gpu)
    fused = cool_pack_supported(hk, hv, hot_len, aged, keep, gs)
    assert fused == (hd != 256)
    seg, idx = cool_pack_hot(hk, hv, hot_len, aged, keep, bits, gs, with_index=True)
    if keep < aged:
        want_idx = co.select_kept(co.value_norms(v[:, :, :aged]), keep)
    else:
        want_idx = np.broadcast_to(np.arange(aged), (B, H, aged))
    assert np.array_equal(idx.cpu().numpy(), want_idx)
    kept_k = np.take_along_axis(k[:, :, :aged], want_idx[..., None], axis=2)
    kept_v = np.take_along_axis(v[:, :, :aged], want_idx[..., None], axis=2)
    for pt, x, axis in ((seg.key, kept_k, -2), (seg.value, kept_v, -1)):
        want = po.quantize_pack(x, bits, axis, gs)
        assert pt.group_size == want.group_size and tuple(pt.orig_shape) == want.orig_shape
        assert np.array_equal(pt.packed.cpu().numpy(), want.packed), axis
        assert np.array_equal(_u16(pt.scale), want.scale.view(np.int16)), axis
        assert np.array_equal(_u16(pt.mins), want.mins.view(np.int16)), axis
        # the same shapes and strides as quantize_pack gives
        ref = quantize_pack(torch.from_numpy(np.ascontiguousarray(x)).to(gpu), bits, axis, gs)
        for name in ("packed", "scale", "mins"):
            a, b = getattr(pt, name), getattr(ref, name)
            assert a.shape == b.shape and a.stride() == b.stride(), (axis, name)
    rem = hot_len - aged
    assert np.array_equal(_u16(hk[:, :, :rem]), k[:, :, aged:hot_len].view(np.int16))
    assert np.array_equal(_u16(hv[:, :, :rem]), v[:, :, aged:hot_len].view(np.int16))


def test_prompt_chunk_packs_an_extension_and_restores_the_window(gpu):
    """A 40-token input chunk on a cache whose window holds 20 generated tokens: the window
    grows for the chunk, the chunk is packed with prompt_bits into a prompt extension equal
    to the oracle's quantize_pack, the 20 generated tokens stay as FP16, and the decode
    over the result matches the oracle."""
    from phasekv_amd.cache import PhaseKVCache
    from phasekv_amd.kernels.attention_triton import fused_phasekv_decode
    g = torch.Generator().manual_seed(11)
    B, H, hq, hd, S, L = 1, 2, 8, 64, 96, 2
    keys = [torch.randn(B, H, S, hd, generator=g).to(torch.float16) for _ in range(L)]
    cache = PhaseKVCache.from_dense_prefill(_Dense([k.to(gpu) for k in keys],
                                                   [(k * 0.5).to(gpu) for k in keys]),
                                            prompt_len=S, prompt_bits=4, cold_bits=2)
    gen = []
    for step in range(20):
        toks = [(torch.randn(B, H, 1, hd, generator=g).to(torch.float16)) for _ in range(L)]
        for l in range(L):
            cache.append_hot(l, toks[l].to(gpu), (toks[l] * 2).to(gpu))
        cache.finish_decode_step()
        gen.append(toks)
    chunk = [torch.randn(B, H, 40, hd, generator=g).to(torch.float16) for _ in range(L)]
    cache.begin_prompt_chunk(40)
    assert cache.prompt_chunk_len == 40
    with pytest.raises(RuntimeError, match="prompt chunk is open"):
        cache.append_hot(0, chunk[0][:, :, :1].to(gpu), chunk[0][:, :, :1].to(gpu))
    for t in range(40):
        for l in range(L):
            x = chunk[l][:, :, t:t + 1].to(gpu)
            cache.append_prompt_token(l, x, -x)
    with pytest.raises(RuntimeError, match="already holds"):
        cache.append_prompt_token(0, x, x)
    cache.finish_prompt_chunk()
    assert cache.prompt_chunk_len == 0 and cache.true_seq_length == S + 20 + 40
    q = torch.randn(hq, hd, generator=g).to(torch.float16)
    for l in range(L):
        tiers = cache.layer_tiers(l)
        assert tiers.hot_len == 20 and tiers.hot_k.shape[2] == 48 and len(tiers.prompt_extensions) == 1
        ext = tiers.prompt_extensions[0]
        wk = po.quantize_pack(chunk[l].numpy(), 4, -2, 32)
        wv = po.quantize_pack((-chunk[l]).numpy(), 4, -1, 32)
        for pt, want in ((ext.key, wk), (ext.value, wv)):
            assert np.array_equal(pt.packed.cpu().numpy(), want.packed)
            assert np.array_equal(_u16(pt.scale), want.scale.view(np.int16))
        hot_k, _ = tiers.hot_views()
        want_hot = torch.cat([t[l] for t in gen], dim=2)
        assert torch.equal(hot_k.cpu(), want_hot)
        out = fused_phasekv_decode(q.to(gpu), tiers, hq).float().cpu().numpy()
        pk = po.quantize_pack(keys[l].numpy(), 4, -2, 32)
        pv = po.quantize_pack((keys[l] * 0.5).numpy(), 4, -1, 32)
        segs = [(po.dequantize_float(pk)[0], po.dequantize_float(pv)[0]),
                (po.dequantize_float(wk)[0], po.dequantize_float(wv)[0]),
                (want_hot[0].numpy(), (want_hot * 2)[0].numpy())]
        np.testing.assert_allclose(out, ao.segments_attention(q.numpy(), segs, hq),
                                   atol=2e-3, rtol=1e-2)


def test_reorder_cache_keeps_storage_and_rows(gpu):
    """reorder_cache([2, 0, 0]) on a 3-row batch after cooling: every tier's rows follow
    beam_idx, K keeps its transposed storage, and each reordered row decodes like the
    original row it came from."""
    from phasekv_amd.cache import PhaseKVCache
    from phasekv_amd.kernels.attention_triton import fused_phasekv_decode_batched
    g = torch.Generator().manual_seed(5)
    B, H, hq, hd, S = 3, 2, 4, 64, 70
    k = torch.randn(B, H, S, hd, generator=g).to(torch.float16).to(gpu)
    cache = PhaseKVCache.from_dense_prefill(_Dense([k], [k.flip(-1)]), prompt_len=S,
                                            decode_keep_ratio=0.5)
    for step in range(50):
        t = torch.randn(B, H, 1, hd, generator=g).to(torch.float16).to(gpu)
        cache.append_hot(0, t, t * 3)
        cache.finish_decode_step()
    tiers = cache.layer_tiers(0)
    assert len(tiers.cold) == 1
    q = torch.randn(B, hq, hd, generator=g).to(torch.float16).to(gpu)
    before = fused_phasekv_decode_batched(q, tiers, hq)
    old_cold_k = tiers.cold[0].key.packed.clone()
    idx = torch.tensor([2, 0, 0], dtype=torch.long, device=gpu)
    cache.reorder_cache(idx)
    tiers = cache.layer_tiers(0)
    assert torch.equal(tiers.cold[0].key.packed, old_cold_k[idx])
    assert tiers.cold[0].key.packed.transpose(-1, -2).is_contiguous()
    assert tiers.prompt.key.scale.transpose(-1, -2).is_contiguous()
    after = fused_phasekv_decode_batched(q[idx], tiers, hq)
    assert torch.equal(after, before[idx])
    with pytest.raises(ValueError, match="beam_idx"):
        cache.reorder_cache(torch.tensor([3], dtype=torch.long, device=gpu))


def test_reused_decode_problem_matches_a_fresh_one(gpu):
    """The batch-1 decode keeps each layer's problem across steps and only rewrites q and
    the hot length: every step's output equals, bit for bit, the output of a problem built
    from scratch, through a cooling event (new cold segment), a prompt chunk (new
    extension, new hot buffer), a strided q and a new q tensor every step; the oracle
    checks every tenth step."""
    from phasekv_amd import decode as dec
    from phasekv_amd.cache import PhaseKVCache
    from phasekv_amd.kernels.attention_triton import fused_phasekv_decode, phasekv_problem
    g = torch.Generator().manual_seed(11)
    B, H, hq, hd, S = 1, 2, 8, 128, 96
    keys = [torch.randn(B, H, S, hd, generator=g).to(torch.float16)]
    values = [torch.randn(B, H, S, hd, generator=g).to(torch.float16)]
    cache = PhaseKVCache.from_dense_prefill(
        _Dense([k.to(gpu) for k in keys], [v.to(gpu) for v in values]), prompt_len=S,
        prompt_bits=2, cold_bits=4, group_size=32, recent_window=32, lazy_g=16,
        decode_keep_ratio=0.5)
    rebuilt = []

    def step_and_check(step):
        tiers = cache.layer_tiers(0)
        if step % 7 == 3:
            q = torch.randn(hd, hq, generator=g).to(torch.float16).to(gpu).t()   # stride(-1) != 1
        else:
            q = torch.randn(hq, hd, generator=g).to(torch.float16).to(gpu)
        kept = getattr(tiers, "_pk_problem", None)
        got = fused_phasekv_decode(q, tiers, hq)
        rebuilt.append(kept is None or tiers._pk_problem is not kept)
        fresh = dec.fused_decode(phasekv_problem(q, tiers, hq))[0]
        assert torch.equal(got, fresh), f"step {step}"
        if step % 10 == 0:
            segs = [(s.key, s.value) for s in [tiers.prompt, *tiers.prompt_extensions,
                                                *tiers.cold]]
            deq = [(po.dequantize_float(_np_pt(k))[0], po.dequantize_float(_np_pt(v))[0])
                   for k, v in segs]
            hk, hv = tiers.hot_views()
            deq.append((hk[0].cpu().numpy(), hv[0].cpu().numpy()))
            want = ao.segments_attention(q.cpu().numpy(), deq, hq)
            np.testing.assert_allclose(got.float().cpu().numpy(), want, atol=2e-3, rtol=1e-2)

    for step in range(60):
        nk = torch.randn(B, H, 1, hd, generator=g).to(torch.float16).to(gpu)
        nv = torch.randn(B, H, 1, hd, generator=g).to(torch.float16).to(gpu)
        cache.append_hot(0, nk, nv)
        step_and_check(step)
        cache.finish_decode_step()
    assert len(cache.layer_tiers(0).cold) == 1
    cache.begin_prompt_chunk(5)
    for i in range(5):
        cache.append_prompt_token(0, torch.randn(B, H, 1, hd, generator=g).to(torch.float16).to(gpu),
                                  torch.randn(B, H, 1, hd, generator=g).to(torch.float16).to(gpu))
    cache.finish_prompt_chunk()
    for step in range(60, 64):
        cache.append_hot(0, torch.randn(B, H, 1, hd, generator=g).to(torch.float16).to(gpu),
                         torch.randn(B, H, 1, hd, generator=g).to(torch.float16).to(gpu))
        step_and_check(step)
        cache.finish_decode_step()
    # built at the first step, after the cooling at step 47 and after the prompt chunk only
    assert [i for i, r in enumerate(rebuilt) if r] == [0, 48, 60]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,hq,hkv,hd,cos_rows,positions", [
    (1, 28, 4, 128, 1, (5, 4100, 32767)), (2, 8, 2, 64, 2, (0, 77)), (3, 12, 4, 128, 1, (1234,))])
def test_rope_append_hot_matches_apply_rotary_pos_emb(gpu, B, hq, hkv, hd, cos_rows, positions,
                                                      dtype):
    """One launch equals transformers' ``apply_rotary_pos_emb`` on fp16 or bf16 tensors,
    ``.to(float16)`` and ``append_hot``: the rotated q and the window rows bit for bit, at
    short and long positions, with one cos / sin row for every batch row or one per row."""
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    from phasekv_amd.cache import PhaseKVCache
    print(f"case B={B} hq={hq} hkv={hkv} hd={hd} cos_rows={cos_rows} {dtype}", flush=True)
    g = torch.Generator().manual_seed(B * 100 + hd)
    S = 40
    dense = _Dense([torch.randn(B, hkv, S, hd, generator=g).to(torch.float16).to(gpu)],
                   [torch.randn(B, hkv, S, hd, generator=g).to(torch.float16).to(gpu)])
    fused = PhaseKVCache.from_dense_prefill(dense, prompt_len=S, prompt_bits=4, cold_bits=4,
                                            group_size=32, recent_window=32, lazy_g=16)
    plain = PhaseKVCache.from_dense_prefill(dense, prompt_len=S, prompt_bits=4, cold_bits=4,
                                            group_size=32, recent_window=32, lazy_g=16)
    inv = 1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    for pos in positions:
        p = torch.tensor([pos + r for r in range(cos_rows)], dtype=torch.float32)
        freqs = p[:, None] * inv[None, :]
        emb = torch.cat((freqs, freqs), dim=-1)
        cos = emb.cos().to(dtype)[:, None, :].to(gpu)
        sin = emb.sin().to(dtype)[:, None, :].to(gpu)
        q = (torch.randn(B, 1, hq * hd, generator=g) * 4).to(dtype).to(gpu)
        k = (torch.randn(B, 1, hkv * hd, generator=g) * 4).to(dtype).to(gpu)
        v = torch.randn(B, 1, hkv * hd, generator=g).to(dtype).to(gpu)
        got_q = fused.rope_append_hot(0, q, k, v, cos, sin, hq)
        qh = q.view(B, 1, hq, hd).transpose(1, 2)
        kh = k.view(B, 1, hkv, hd).transpose(1, 2)
        want_q, want_k = apply_rotary_pos_emb(qh, kh, cos, sin)
        want_q, want_k = want_q.to(torch.float16), want_k.to(torch.float16)
        plain.append_hot(0, want_k, v.view(B, 1, hkv, hd).transpose(1, 2).to(torch.float16))
        assert torch.equal(got_q, want_q[:, :, 0, :]), f"q at position {pos}"
        fk, fv = fused.layer_tiers(0).hot_views()
        pk_, pv = plain.layer_tiers(0).hot_views()
        assert torch.equal(fk, pk_) and torch.equal(fv, pv), f"window at position {pos}"
        fused.finish_decode_step()
        plain.finish_decode_step()


def test_rope_append_hot_errors(gpu):
    from phasekv_amd.cache import PhaseKVCache
    g = torch.Generator().manual_seed(5)
    dense = _Dense([torch.randn(1, 2, 32, 64, generator=g).to(torch.float16).to(gpu)],
                   [torch.randn(1, 2, 32, 64, generator=g).to(torch.float16).to(gpu)])
    cache = PhaseKVCache.from_dense_prefill(dense, prompt_len=32, prompt_bits=2, cold_bits=2,
                                            group_size=32, recent_window=4, lazy_g=2)
    f16 = dict(dtype=torch.float16, device=gpu)
    q, k, v = torch.zeros(1, 1, 8 * 64, **f16), torch.zeros(1, 1, 128, **f16), torch.zeros(1, 1, 128, **f16)
    cs = torch.ones(1, 1, 64, **f16)
    with pytest.raises(ValueError):
        cache.rope_append_hot(0, q, k, v, cs, cs, 6)               # q is not [1, 1, 6 * 64]
    with pytest.raises(ValueError):
        cache.rope_append_hot(0, q.float(), k, v, cs, cs, 8)       # dtype
    with pytest.raises(ValueError):
        cache.rope_append_hot(0, q.bfloat16(), k, v, cs, cs, 8)    # mixed dtypes
    with pytest.raises(ValueError):
        cache.rope_append_hot(0, q, k, v, cs[..., :32], cs[..., :32], 8)   # cos width
    with pytest.raises(ValueError):
        cache.rope_append_hot(0, q, k, v, cs.cpu(), cs.cpu(), 8)   # device
    cache.rope_append_hot(0, q, k, v, cs, cs, 8)
    with pytest.raises(RuntimeError):
        cache.rope_append_hot(0, q, k, v, cs, cs, 8)               # twice in one step


def test_append_prompt_chunk_matches_per_token_appends(gpu):
    """One ``pk_append_hot_rows`` launch per layer writes the same window rows as the
    per-token loop, in one call or two (3 + 6 rows, strided sources), and refuses rows
    beyond the chunk."""
    from phasekv_amd.cache import PhaseKVCache
    g = torch.Generator().manual_seed(21)
    B, H, hd, S, T = 2, 2, 128, 64, 9
    dense = _Dense([torch.randn(B, H, S, hd, generator=g).to(torch.float16).to(gpu)],
                   [torch.randn(B, H, S, hd, generator=g).to(torch.float16).to(gpu)])
    caches = [PhaseKVCache.from_dense_prefill(dense, prompt_len=S, prompt_bits=4, cold_bits=4,
                                              group_size=32, recent_window=32, lazy_g=16)
              for _ in range(3)]
    gen = [torch.randn(B, H, 1, hd, generator=g).to(torch.float16).to(gpu) for _ in range(5)]
    for c in caches:          # the same generated tokens in every window first
        for k in gen:
            c.append_hot(0, k, k * 2)
            c.finish_decode_step()
    k = torch.randn(B, T, H, hd, generator=g).to(torch.float16).to(gpu).transpose(1, 2)  # strided
    v = torch.randn(B, H, T, hd, generator=g).to(torch.float16).to(gpu)
    for c in caches:
        c.begin_prompt_chunk(T)
    for t in range(T):
        caches[0].append_prompt_token(0, k[:, :, t:t + 1], v[:, :, t:t + 1])
    caches[1].append_prompt_chunk(0, k, v)
    caches[2].append_prompt_chunk(0, k[:, :, :3], v[:, :, :3])
    caches[2].append_prompt_chunk(0, k[:, :, 3:], v[:, :, 3:])
    with pytest.raises(RuntimeError):
        caches[2].append_prompt_chunk(0, k[:, :, :1], v[:, :, :1])
    want_k, want_v = caches[0].layer_tiers(0).hot_views()
    for c in caches[1:]:
        got_k, got_v = c.layer_tiers(0).hot_views()
        assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v)
    for c in caches:
        c.finish_prompt_chunk()
    ext = [c.layer_tiers(0).prompt_extensions[-1] for c in caches]
    for e in ext[1:]:
        assert torch.equal(e.key.packed, ext[0].key.packed)
        assert torch.equal(e.value.packed, ext[0].value.packed)
