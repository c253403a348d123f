"""numpy restatement of the reference's prefill prompt selection.

Test infrastructure only (see ``oracle/__init__.py``).

* ``selection_plan``         ``src/phasekv/prompt_tier.py:48-53``
* ``observation_votes``      ``src/phasekv/hetero_cache.py:67-77`` with
  ``aggregate_to_kv_heads`` (``:55-64``): float32, the last ``w`` query rows summed in
  row order, then the group's query heads summed in head order
* ``pool_scores``            ``src/phasekv/hetero_cache.py:80-94``: ``max_pool1d`` /
  ``avg_pool1d`` with stride 1 and padding ``k // 2``, truncated to the length (max:
  padding never wins, NaN propagates; avg: the window's values added left to right,
  padding as 0, divided by ``k``)
* ``select_prompt_indices``  ``src/phasekv/prompt_tier.py:22-76`` with ``topk_per_head``
  (``hetero_cache.py:147-157``); among exactly equal pooled scores the earlier position
  is kept (``torch.topk`` leaves that open), NaN ranks above every number.
"""
from __future__ import annotations

import numpy as np


def selection_plan(prompt_len, prefill_keep_ratio, sink_tokens, obs_window):
    sink = min(sink_tokens, prompt_len)
    budget = min(prompt_len, max(1, sink, round(prompt_len * prefill_keep_ratio)))
    sink_keep = min(sink, budget)
    recent_keep = min(obs_window, budget - sink_keep, prompt_len - sink_keep)
    recent_start = prompt_len - recent_keep
    select_k = budget - sink_keep - recent_keep
    return budget, sink_keep, recent_start, select_k


def observation_votes(attn: np.ndarray, num_kv_heads: int, obs_window: int) -> np.ndarray:
    """``[B, Hq, q_len, kv_len]`` -> float32 ``[B, Hkv, kv_len]``."""
    B, hq, q_len, kv_len = attn.shape
    w = max(1, min(obs_window, q_len))
    a = attn[:, :, q_len - w:, :].astype(np.float32)
    per_head = a[:, :, 0, :].copy()
    for r in range(1, w):
        per_head = per_head + a[:, :, r, :]
    g = hq // num_kv_heads
    per_head = per_head.reshape(B, num_kv_heads, g, kv_len)
    votes = per_head[:, :, 0, :].copy()
    for i in range(1, g):
        votes = votes + per_head[:, :, i, :]
    return votes.astype(np.float32)


def pool_scores(scores: np.ndarray, kernel, mode: str = "maxpool") -> np.ndarray:
    if kernel is None or kernel <= 1:
        return scores
    if mode not in ("maxpool", "avgpool"):
        raise ValueError(f"unknown pooling: {mode}")
    n = scores.shape[-1]
    pad = kernel // 2
    fill = -np.inf if mode == "maxpool" else 0.0
    padded = np.concatenate([np.full(scores.shape[:-1] + (pad,), fill, np.float32),
                             scores.astype(np.float32),
                             np.full(scores.shape[:-1] + (kernel,), fill, np.float32)], axis=-1)
    out = padded[..., 0:n].copy()
    for t in range(1, kernel):
        win = padded[..., t:t + n]
        out = np.maximum(out, win) if mode == "maxpool" else (out + win).astype(np.float32)
    if mode == "avgpool":
        out = (out / np.float32(kernel)).astype(np.float32)
    return out.astype(np.float32)


def topk_sorted(signal: np.ndarray, k: int) -> np.ndarray:
    """Ascending positions of the k largest (NaN first, equal values: earlier first)."""
    lead = signal.shape[:-1]
    flat = signal.reshape(-1, signal.shape[-1])
    out = np.empty((flat.shape[0], k), np.int64)
    for r in range(flat.shape[0]):
        key = np.where(np.isnan(flat[r]), -np.inf, -flat[r].astype(np.float64))
        order = np.lexsort((np.arange(flat.shape[1]), key))
        out[r] = np.sort(order[:k])
    return out.reshape(lead + (k,))


def select_prompt_indices(attentions, *, prompt_len, num_kv_heads, prefill_keep_ratio,
                          sink_tokens, obs_window, pool_kernel, pooling):
    budget, sink_keep, recent_start, select_k = selection_plan(
        prompt_len, prefill_keep_ratio, sink_tokens, obs_window)
    result = []
    for attn in attentions:
        b = attn.shape[0]
        sink_idx = np.broadcast_to(np.arange(sink_keep), (b, num_kv_heads, sink_keep))
        recent_idx = np.broadcast_to(np.arange(recent_start, prompt_len),
                                     (b, num_kv_heads, prompt_len - recent_start))
        if select_k:
            votes = observation_votes(attn, num_kv_heads, min(obs_window, prompt_len))
            cand = pool_scores(votes[..., sink_keep:recent_start], pool_kernel, pooling)
            top = topk_sorted(cand, select_k) + sink_keep
        else:
            top = np.zeros((b, num_kv_heads, 0), np.int64)
        keep = np.concatenate([sink_idx, top, recent_idx], axis=-1)
        assert keep.shape[-1] == budget
        result.append(np.sort(keep, axis=-1).astype(np.int64))
    return result
