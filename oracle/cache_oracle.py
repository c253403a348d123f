"""numpy restatement of the FP16 hot window lifecycle of the reference's cache.

Test infrastructure only (see ``oracle/__init__.py``).

* ``append_hot``         follows ``src/phasekv/phasekv_cache.py:405-422`` (``_append_token``)
* ``value_norms``        the importance of ``phasekv_cache.py:330``
  (``torch.linalg.vector_norm(value.float(), dim=-1)``), in one fixed float32
  summation order (below)
* ``select_kept``        ``phasekv_cache.py:329-332`` (``topk`` then ``sort`` of the indices)
* ``cool_aged_tokens``   ``phasekv_cache.py:322-340`` (``_cool_aged_tokens``) with
  ``_gather_kv`` (``:110-114``) and ``_pack_kv`` (``:101-107``)

Float order of the norm: the squares of fp16 values are exact in float32; lane l
(l < 64) adds the squares of channels l, l + 64, l + 128, ... in that order, then
the 64 lane sums are combined by the butterfly ``p = p + p[i ^ o]`` for
o = 32, 16, ..., 1, and the norm is the correctly rounded float32 sqrt of ``p[0]``.
The reference's torch reduction order is not specified; on inputs without near
ties the selection is the same (pinned against torch's ``vector_norm`` / ``topk``
in the tests).

Ties: ``torch.topk`` does not define which of equal values it returns.  Here the
earlier token wins an exact tie of norms, and NaN norms rank above every number
(as ``torch.sort`` orders them), equal NaNs by position.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np

from . import packing_oracle as po


def append_hot(hot_k: np.ndarray, hot_v: np.ndarray, hot_len: int, key: np.ndarray,
               value: np.ndarray) -> int:
    """Write one token ``[B, Hkv, 1, hd]`` at row ``hot_len``; returns the new length."""
    if hot_len >= hot_k.shape[2]:
        raise RuntimeError("hot window is full")
    hot_k[:, :, hot_len:hot_len + 1, :] = key
    hot_v[:, :, hot_len:hot_len + 1, :] = value
    return hot_len + 1


def value_norms(v: np.ndarray) -> np.ndarray:
    """float32 L2 norms of fp16 rows ``v[..., hd]`` in the order stated in the module doc."""
    x = v.astype(np.float32)
    hd = x.shape[-1]
    lanes = np.zeros(x.shape[:-1] + (64,), np.float32)
    for start in range(0, hd, 64):
        chunk = x[..., start:start + 64]
        sq = chunk * chunk                           # exact: fp16 * fp16 fits float32
        lanes[..., :chunk.shape[-1]] = lanes[..., :chunk.shape[-1]] + sq
    idx = np.arange(64)
    for o in (32, 16, 8, 4, 2, 1):
        lanes = lanes + lanes[..., idx ^ o]
    return np.sqrt(lanes[..., 0]).astype(np.float32)


def _rank_key(norms: np.ndarray) -> np.ndarray:
    """Sort keys: descending norm, NaN first, then ascending position (a stable sort)."""
    n = norms.shape[-1]
    key = np.where(np.isnan(norms), -np.inf, -norms.astype(np.float64))
    return key, np.arange(n)


def select_kept(norms: np.ndarray, keep: int) -> np.ndarray:
    """Indices ``[..., keep]`` of the kept tokens, ascending (``phasekv_cache.py:331``)."""
    lead = norms.shape[:-1]
    flat = norms.reshape(-1, norms.shape[-1])
    out = np.empty((flat.shape[0], keep), np.int64)
    for r in range(flat.shape[0]):
        key, pos = _rank_key(flat[r])
        order = np.lexsort((pos, key))               # primary key, then position
        out[r] = np.sort(order[:keep])
    return out.reshape(lead + (keep,))


def keep_count(aged: int, decode_keep_ratio: float) -> int:
    """``max(1, round(ratio * aged))`` with Python's round (``phasekv_cache.py:329``)."""
    return max(1, round(decode_keep_ratio * aged))


def cool_aged_tokens(hot_k: np.ndarray, hot_v: np.ndarray, hot_len: int, recent_window: int,
                     lazy_g: int, decode_keep_ratio: float, cold_bits: int,
                     group_size: int) -> Tuple[object, int, np.ndarray]:
    """One cooling step in place on ``hot_k`` / ``hot_v`` ``[B, Hkv, capacity, hd]``.

    Returns ``(segment, new_hot_len, kept_indices)``; ``segment`` is ``None`` when
    fewer than ``lazy_g`` tokens have aged, else ``(packed_k, packed_v)`` packed as
    the cache packs a segment (K along tokens, V along head_dim).
    """
    aged = hot_len - recent_window
    if aged < lazy_g:
        return None, hot_len, np.zeros(hot_k.shape[:2] + (0,), np.int64)
    key = hot_k[:, :, :aged, :].copy()
    value = hot_v[:, :, :aged, :].copy()
    keep = keep_count(aged, decode_keep_ratio)
    if keep < aged:
        idx = select_kept(value_norms(value), keep)
        key = np.take_along_axis(key, idx[..., None], axis=2)
        value = np.take_along_axis(value, idx[..., None], axis=2)
    else:
        idx = np.broadcast_to(np.arange(aged), hot_k.shape[:2] + (aged,)).copy()
    segment = (po.quantize_pack(key, cold_bits, -2, group_size),
               po.quantize_pack(value, cold_bits, -1, group_size))
    remaining = hot_len - aged
    hot_k[:, :, :remaining, :] = hot_k[:, :, aged:hot_len, :].copy()
    hot_v[:, :, :remaining, :] = hot_v[:, :, aged:hot_len, :].copy()
    return segment, remaining, idx
