"""numpy restatement of the reference's decode-attention semantics.

Test infrastructure only (see ``oracle/__init__.py``).

* ``dequant_concat``                   follows ``src/phasekv/kernels/reference.py:43-58``
* ``expand_gqa``                       follows ``src/phasekv/kernels/reference.py:61-69``
* ``fused_decode_attention_reference`` follows ``src/phasekv/kernels/reference.py:72-96``
* ``dense_fp16_attention``             follows ``src/phasekv/kernels/reference.py:99-109``
* ``reduce_splits``                    follows ``src/phasekv/kernels/attention_triton.py:257-266``
* ``merge_partials``                   follows ``src/phasekv/kernels/attention_triton.py:300-307``
* ``fp16_layer_partial``               follows ``src/phasekv/kernels/attention_triton.py:285-297``
* ``segment_partial``                  is the math of one packed segment as computed by
  ``_kivi_layer_partial`` (``src/phasekv/kernels/attention_triton.py:604-639``):
  float32 dequantization, score scale ``1/sqrt(hd)``, split-K online softmax.
* ``layer_tiers_attention``            follows ``fused_phasekv_decode``
  (``src/phasekv/kernels/attention_triton.py:643-669``): every segment of
  ``[prompt, *prompt_extensions, *cold]`` plus the FP16 hot window.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from .packing_oracle import PackedArrays, dequantize_float, unpack_dequantize


@dataclass
class ThreeTierArrays:
    """Host mirror of ``ThreeTierKV`` (``reference.py:27-40``); arrays are [b, Hkv, len, hd]."""

    prompt_k: Optional[PackedArrays] = None
    prompt_v: Optional[PackedArrays] = None
    cold_k: Optional[PackedArrays] = None
    cold_v: Optional[PackedArrays] = None
    hot_k: Optional[np.ndarray] = None
    hot_v: Optional[np.ndarray] = None


def dequant_concat(kv: ThreeTierArrays):
    """Dequantize every tier to float16 and concatenate prompt -> cold -> hot on the token axis."""
    ks: List[np.ndarray] = []
    vs: List[np.ndarray] = []
    if kv.prompt_k is not None:
        ks.append(unpack_dequantize(kv.prompt_k))
        vs.append(unpack_dequantize(kv.prompt_v))
    if kv.cold_k is not None:
        ks.append(unpack_dequantize(kv.cold_k))
        vs.append(unpack_dequantize(kv.cold_v))
    if kv.hot_k is not None:
        ks.append(kv.hot_k.astype(np.float16))
        vs.append(kv.hot_v.astype(np.float16))
    if not ks:
        raise ValueError("all three tiers are empty")
    return np.concatenate(ks, axis=-2), np.concatenate(vs, axis=-2)


def expand_gqa(x: np.ndarray, num_attention_heads: int) -> np.ndarray:
    """Repeat each kv head ``Hq // Hkv`` times: query head h reads kv head ``h // group``."""
    hkv = x.shape[1]
    if hkv == num_attention_heads:
        return x
    if num_attention_heads % hkv:
        raise ValueError("num_attention_heads must be a multiple of the kv heads")
    return np.repeat(x, num_attention_heads // hkv, axis=1)


def _softmax_attention(q, k, v, dtype):
    hd = q.shape[-1]
    scale = 1.0 / math.sqrt(hd)
    scores = np.matmul(q.astype(dtype), np.swapaxes(k.astype(dtype), -1, -2)) * dtype(scale)
    scores = scores - scores.max(axis=-1, keepdims=True)
    e = np.exp(scores)
    probs = e / e.sum(axis=-1, keepdims=True)
    return np.matmul(probs, v.astype(dtype))


def fused_decode_attention_reference(q: np.ndarray, kv: ThreeTierArrays,
                                     num_attention_heads: int, dtype=np.float32) -> np.ndarray:
    """softmax(q K^T / sqrt(hd)) V over all tiers, no causal mask; q [b, Hq, q_len, hd]."""
    if q.ndim != 4:
        raise ValueError("q must be [b, Hq, q_len, hd]")
    k_all, v_all = dequant_concat(kv)
    k_all = expand_gqa(k_all, num_attention_heads)
    v_all = expand_gqa(v_all, num_attention_heads)
    return _softmax_attention(q, k_all, v_all, dtype).astype(np.float16)


def dense_fp16_attention(q, k, v, num_attention_heads: int, dtype=np.float32) -> np.ndarray:
    """The same attention over uncompressed float16 K/V."""
    k = expand_gqa(k, num_attention_heads)
    v = expand_gqa(v, num_attention_heads)
    return _softmax_attention(q, k, v, dtype).astype(np.float16)


# ----------------------------------------------------------------------------
# split-K partials and their log-sum-exp merge
# ----------------------------------------------------------------------------
def reduce_splits(pm: np.ndarray, pl: np.ndarray, pacc: np.ndarray):
    """m = max_s pm; w = exp(pm - m); l = sum w*pl; acc = sum w*pacc (unnormalized)."""
    m = pm.max(axis=1)
    w = np.exp(pm - m[:, None])
    l = (w * pl).sum(axis=1)
    acc = (w[:, :, None] * pacc).sum(axis=1)
    return m, l, acc


def merge_partials(partials, out_dtype=np.float16):
    """Cross-segment merge of (m, l, acc) partials; returns acc / l."""
    ms = np.stack([p[0] for p in partials], axis=1)
    m = ms.max(axis=1)
    w = np.exp(ms - m[:, None])
    l = sum(w[:, i] * partials[i][1] for i in range(len(partials)))
    acc = sum(w[:, i:i + 1] * partials[i][2] for i in range(len(partials)))
    out = acc / l[:, None]
    return out.astype(out_dtype) if out_dtype is not None else out


def partial_from_dense(q: np.ndarray, k: np.ndarray, v: np.ndarray, num_attention_heads: int,
                       dtype=np.float64):
    """(m, l, acc) of q [Hq, hd] against one segment's dense K/V [Hkv, S, hd]."""
    hkv, s_len, hd = k.shape
    group = num_attention_heads // hkv
    # query head h reads kv head h // group (reference.py:61-69); the heads of one kv
    # head are a batch of one matrix product instead of a repeated K/V copy
    qg = q.astype(dtype).reshape(hkv, group, hd)
    s = np.matmul(qg, np.swapaxes(k.astype(dtype), 1, 2)) * dtype(1.0 / math.sqrt(hd))
    s = s.reshape(num_attention_heads, s_len)
    m = s.max(axis=1)
    p = np.exp(s - m[:, None])
    acc = np.matmul(p.reshape(hkv, group, s_len), v.astype(dtype)).reshape(num_attention_heads, hd)
    return m, p.sum(axis=1), acc


def split_partials(q, k, v, num_attention_heads, split_len, dtype=np.float64):
    """Per-split (pm, pl, pacc) [Hq, splits(, hd)] over contiguous token ranges of ``split_len``."""
    s_len = k.shape[1]
    bounds = list(range(0, s_len, split_len))
    parts = [partial_from_dense(q, k[:, b:b + split_len], v[:, b:b + split_len],
                                num_attention_heads, dtype) for b in bounds]
    pm = np.stack([p[0] for p in parts], axis=1)
    pl = np.stack([p[1] for p in parts], axis=1)
    pacc = np.stack([p[2] for p in parts], axis=1)
    return pm, pl, pacc


def segment_partial(q: np.ndarray, key: PackedArrays, value: PackedArrays,
                    num_attention_heads: int, dtype=np.float64):
    """(m, l, acc) of one batch-stripped packed segment, dequantized in float32 like the kernel."""
    k = dequantize_float(key)
    v = dequantize_float(value)
    return partial_from_dense(q, k, v, num_attention_heads, dtype)


def fp16_layer_partial(q, hot_k, hot_v, num_attention_heads, dtype=np.float64):
    """(m, l, acc) of the FP16 hot window [Hkv, hot, hd]."""
    return partial_from_dense(q, hot_k.astype(np.float32), hot_v.astype(np.float32),
                              num_attention_heads, dtype)


@dataclass
class SegmentArrays:
    """Host mirror of ``PackedKVSegment`` (K axis 2, V axis 3 over [B, Hkv, S, hd])."""

    key: PackedArrays
    value: PackedArrays


@dataclass
class LayerTiersArrays:
    """Host mirror of ``LayerTiers`` (``phasekv_cache.py:47-79``)."""

    prompt: SegmentArrays
    prompt_extensions: List[SegmentArrays] = field(default_factory=list)
    cold: List[SegmentArrays] = field(default_factory=list)
    hot_k: Optional[np.ndarray] = None    # [B, Hkv, hot_len, hd] float16
    hot_v: Optional[np.ndarray] = None


def _strip_batch(pt: PackedArrays, b: int) -> PackedArrays:
    return PackedArrays(pt.packed[b], pt.scale[b], pt.mins[b], pt.bits, pt.axis - 1,
                        pt.group_size, pt.orig_shape[1:], pt.axis_len)


def layer_tiers_attention(q: np.ndarray, tiers: LayerTiersArrays, num_attention_heads: int,
                          batch: int = 0, dtype=np.float64) -> np.ndarray:
    """Attention of q [Hq, hd] over every segment and the hot window of one batch row.

    Returns float ``[Hq, hd]`` (not rounded) so tests can apply their tolerance.
    """
    partials = []
    for seg in [tiers.prompt, *tiers.prompt_extensions, *tiers.cold]:
        partials.append(segment_partial(q, _strip_batch(seg.key, batch),
                                        _strip_batch(seg.value, batch),
                                        num_attention_heads, dtype))
    if tiers.hot_k is not None and tiers.hot_k.shape[2] > 0:
        partials.append(fp16_layer_partial(q, tiers.hot_k[batch], tiers.hot_v[batch],
                                           num_attention_heads, dtype))
    return merge_partials(partials, out_dtype=None)


def segments_attention(q: np.ndarray, dense_segments: Sequence, num_attention_heads: int,
                       dtype=np.float64) -> np.ndarray:
    """Attention of q [Hq, hd] over a list of dense (K, V) [Hkv, S, hd] segments."""
    parts = [partial_from_dense(q, k, v, num_attention_heads, dtype) for k, v in dense_segments]
    return merge_partials(parts, out_dtype=None)
