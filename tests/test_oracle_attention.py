"""Pins the attention oracle: float64 brute force, closed forms, invariants, planted mistakes."""
import math

import numpy as np
import pytest

from oracle import attention_oracle as ao
from oracle import packing_oracle as po


def _brute(q, k, v, hq):
    """Loop-by-loop float64 attention of q [Hq, hd] over K, V [Hkv, S, hd]."""
    hkv, s_len, hd = k.shape
    g = hq // hkv
    out = np.zeros((hq, hd))
    for h in range(hq):
        kv = h // g
        sc = [sum(float(q[h, d]) * float(k[kv, t, d]) for d in range(hd)) / math.sqrt(hd)
              for t in range(s_len)]
        mx = max(sc)
        w = [math.exp(x - mx) for x in sc]
        tot = sum(w)
        for d in range(hd):
            out[h, d] = sum(w[t] * float(v[kv, t, d]) for t in range(s_len)) / tot
    return out


def _rand(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float16)


def test_reference_attention_matches_brute_force():
    hq, hkv, hd = 6, 2, 8
    q = _rand((1, hq, 1, hd), 1)
    pk = po.quantize_pack(_rand((1, hkv, 11, hd), 2), 4, -2, 4)
    pv = po.quantize_pack(_rand((1, hkv, 11, hd), 3), 4, -1, 4)
    ck = po.quantize_pack(_rand((1, hkv, 5, hd), 4), 2, -2, 4)
    cv = po.quantize_pack(_rand((1, hkv, 5, hd), 5), 2, -1, 4)
    hk, hv = _rand((1, hkv, 3, hd), 6), _rand((1, hkv, 3, hd), 7)
    kv = ao.ThreeTierArrays(pk, pv, ck, cv, hk, hv)
    got = ao.fused_decode_attention_reference(q, kv, hq)[0, :, 0]
    k_all = np.concatenate([po.unpack_dequantize(pk), po.unpack_dequantize(ck), hk], 2)[0]
    v_all = np.concatenate([po.unpack_dequantize(pv), po.unpack_dequantize(cv), hv], 2)[0]
    want = _brute(q[0, :, 0], k_all, v_all, hq)
    np.testing.assert_allclose(got.astype(np.float64), want, atol=2e-3, rtol=2e-3)


def test_uniform_scores_give_mean_of_values():
    hq, hkv, hd, s_len = 4, 2, 16, 37
    q = _rand((hq, hd), 8)
    k = np.zeros((hkv, s_len, hd), np.float16)          # every score is 0
    v = _rand((hkv, s_len, hd), 9)
    out = ao.segments_attention(q, [(k, v)], hq)
    want = np.repeat(v.astype(np.float64).mean(axis=1), hq // hkv, axis=0)
    np.testing.assert_allclose(out, want, atol=1e-12)


def test_one_dominant_key_selects_its_value():
    hq, hkv, hd, s_len = 2, 1, 8, 20
    q = np.full((hq, hd), 4.0, np.float16)
    k = np.zeros((hkv, s_len, hd), np.float16)
    k[0, 13] = 8.0                                       # score 128/sqrt(8) vs 0
    v = _rand((hkv, s_len, hd), 10)
    out = ao.segments_attention(q, [(k, v)], hq)
    np.testing.assert_allclose(out, np.repeat(v[:, 13].astype(np.float64), 2, 0), atol=1e-12)


def test_gqa_head_mapping_is_block_not_interleaved():
    hq, hkv, hd, s_len = 6, 3, 4, 5
    q = _rand((hq, hd), 11)
    k = _rand((hkv, s_len, hd), 12)
    v = _rand((hkv, s_len, hd), 13)
    out = ao.segments_attention(q, [(k, v)], hq)
    for h in range(hq):
        single = ao.segments_attention(q[h:h + 1], [(k[h // 2:h // 2 + 1], v[h // 2:h // 2 + 1])], 1)
        np.testing.assert_allclose(out[h], single[0], atol=1e-12)
    wrong = ao.segments_attention(q[1:2], [(k[1:2], v[1:2])], 1)   # h % Hkv mapping for h=1
    assert not np.allclose(out[1], wrong[0])


@pytest.mark.parametrize("split_len", [1, 3, 7, 16, 64])
def test_split_partials_merge_to_full_attention(split_len):
    hq, hkv, hd, s_len = 8, 2, 16, 50
    q = _rand((hq, hd), 14)
    k = _rand((hkv, s_len, hd), 15, 2.0)
    v = _rand((hkv, s_len, hd), 16)
    full = ao.segments_attention(q, [(k, v)], hq)
    pm, pl, pacc = ao.split_partials(q, k, v, hq, split_len)
    m, l, acc = ao.reduce_splits(pm, pl, pacc)
    np.testing.assert_allclose(acc / l[:, None], full, atol=1e-12)


def test_segment_order_and_merge_associativity():
    hq, hkv, hd = 4, 2, 8
    q = _rand((hq, hd), 17)
    segs = [(_rand((hkv, n, hd), 20 + n), _rand((hkv, n, hd), 40 + n)) for n in (3, 9, 1, 14)]
    a = ao.segments_attention(q, segs, hq)
    b = ao.segments_attention(q, segs[::-1], hq)
    np.testing.assert_allclose(a, b, atol=1e-12)
    parts = [ao.partial_from_dense(q, k, v, hq) for k, v in segs]
    left = ao.reduce_splits(*[np.stack(x, 1) for x in zip(*parts[:2])])
    right = ao.reduce_splits(*[np.stack(x, 1) for x in zip(*parts[2:])])
    nested = ao.merge_partials([left, right], out_dtype=None)
    np.testing.assert_allclose(nested, a, atol=1e-12)


def test_planted_score_scale_mistake_is_detected():
    hq, hkv, hd, s_len = 2, 1, 64, 30
    q = _rand((hq, hd), 30)
    k = _rand((hkv, s_len, hd), 31)
    v = _rand((hkv, s_len, hd), 32)
    good = ao.segments_attention(q, [(k, v)], hq)
    bad = ao.segments_attention(q * np.float16(1.0 / math.sqrt(hd)), [(k, v)], hq)  # 1/hd total
    assert np.abs(good - bad).max() > 1e-2
    brute = _brute(q, k, v, hq)
    np.testing.assert_allclose(good, brute, atol=1e-9)


def test_layer_tiers_attention_equals_dense_concat():
    """Segment-by-segment merge == one softmax over the dequantized concatenation."""
    hq, hkv, hd = 4, 2, 16
    q = _rand((hq, hd), 50)
    pk = po.quantize_pack(_rand((1, hkv, 40, hd), 51), 2, -2, 32)
    pv = po.quantize_pack(_rand((1, hkv, 40, hd), 52), 2, -1, 32)
    ck = po.quantize_pack(_rand((1, hkv, 7, hd), 53), 4, -2, 32)
    cv = po.quantize_pack(_rand((1, hkv, 7, hd), 54), 4, -1, 32)
    hk, hv = _rand((1, hkv, 5, hd), 55), _rand((1, hkv, 5, hd), 56)
    tiers = ao.LayerTiersArrays(ao.SegmentArrays(pk, pv), [], [ao.SegmentArrays(ck, cv)], hk, hv)
    got = ao.layer_tiers_attention(q, tiers, hq)
    k = np.concatenate([po.dequantize_float(pk), po.dequantize_float(ck), hk.astype(np.float32)], 2)[0]
    v = np.concatenate([po.dequantize_float(pv), po.dequantize_float(cv), hv.astype(np.float32)], 2)[0]
    np.testing.assert_allclose(got, _brute(q, k, v, hq), atol=1e-9)
