"""Prefill-side prompt selection on the GPU: which prompt positions each kv head keeps.

Mirrors ``select_prompt_indices`` of ``src/phasekv/prompt_tier.py:22-76``: per layer,
observation-window votes over the prefill attention (the last ``obs_window`` query rows,
summed, then summed over each kv head's query heads; ``hetero_cache.py:55-77``), 1-D
pooling of the candidate votes (``hetero_cache.py:80-94``), a per-head top-k
(``hetero_cache.py:147-157``), and the kept positions: the sink tokens, the selected
candidates and the most recent ``obs_window`` tokens, ascending.  Two HIP launches per
layer (``pk_prompt_votes``, ``pk_select_prompt``).  Among exactly equal pooled scores
the earlier position is kept (``torch.topk`` leaves that choice open).
"""
from __future__ import annotations

import torch

from . import _lib

_DTYPE_CODES = {torch.float16: _lib.PK_DTYPE_F16, torch.bfloat16: _lib.PK_DTYPE_BF16,
                torch.float32: _lib.PK_DTYPE_F32}
_POOL_MODES = {"maxpool": 0, "avgpool": 1}


def num_kv_heads_of(model_config) -> int:
    """``hetero_cache.py:48-49``."""
    return getattr(model_config, "num_key_value_heads",
                   getattr(model_config, "num_attention_heads"))


def selection_plan(prompt_len: int, prefill_keep_ratio: float, sink_tokens: int,
                   obs_window: int):
    """(budget, sink_keep, recent_start, select_k) of ``prompt_tier.py:48-53``."""
    sink = min(sink_tokens, prompt_len)
    budget = min(prompt_len, max(1, sink, round(prompt_len * prefill_keep_ratio)))
    sink_keep = min(sink, budget)
    recent_keep = min(obs_window, budget - sink_keep, prompt_len - sink_keep)
    recent_start = prompt_len - recent_keep
    select_k = budget - sink_keep - recent_keep
    return budget, sink_keep, recent_start, select_k


def prompt_votes(attention: torch.Tensor, num_kv_heads: int, obs_window: int) -> torch.Tensor:
    """fp32 ``[B, Hkv, kv_len]`` votes of one layer's attention ``[B, Hq, q_len, kv_len]``."""
    if attention.dim() != 4:
        raise ValueError("attention must be [B, Hq, q_len, kv_len]")
    dev = _lib.require_device(attention)
    if attention.dtype not in _DTYPE_CODES:
        attention = attention.float()
    B, hq, q_len, kv_len = attention.shape
    votes = torch.empty(B, num_kv_heads, kv_len, dtype=torch.float32, device=dev)
    _lib.check(_lib.load().pk_prompt_votes(attention.data_ptr(), _DTYPE_CODES[attention.dtype],
                                           B, hq, q_len, kv_len,
                                           _lib.i64_array(attention.stride()), num_kv_heads,
                                           obs_window, votes.data_ptr(), _lib.stream_ptr(dev)),
               "prompt_votes")
    return votes


def select_prompt_indices(attentions, *, prompt_len: int, model_config,
                          prefill_keep_ratio: float, sink_tokens: int, obs_window: int,
                          pool_kernel: int, pooling: str) -> list:
    """Per layer, ``[B, Hkv, K0]`` int64 kept prompt positions, strictly ascending."""
    if attentions is None or not attentions:
        raise ValueError("prompt selection needs every layer's prefill attention")
    if prompt_len <= 0 or not 0.0 < prefill_keep_ratio <= 1.0:
        raise ValueError("prompt_len and prefill_keep_ratio are invalid")
    if sink_tokens < 0 or obs_window <= 0:
        raise ValueError("sink_tokens must not be negative and obs_window must be positive")
    if pooling not in _POOL_MODES and pool_kernel is not None and pool_kernel > 1:
        raise ValueError(f"unknown pooling: {pooling}; maxpool and avgpool are supported")
    hkv = num_kv_heads_of(model_config)
    budget, sink_keep, recent_start, select_k = selection_plan(prompt_len, prefill_keep_ratio,
                                                               sink_tokens, obs_window)
    k = 1 if pool_kernel is None or pool_kernel <= 1 else int(pool_kernel)
    mode = _POOL_MODES.get(pooling, 0)
    result = []
    lib = _lib.load()
    for attention in attentions:
        if attention is None or attention.shape[-1] != prompt_len:
            raise ValueError("prefill attention is missing or its key length is not prompt_len")
        dev = _lib.require_device(attention)
        B = attention.shape[0]
        votes = prompt_votes(attention, hkv, min(obs_window, prompt_len))
        keep = torch.empty(B, hkv, budget, dtype=torch.int64, device=dev)
        _lib.check(lib.pk_select_prompt(votes.data_ptr(), B * hkv, prompt_len, sink_keep,
                                        recent_start, select_k, k, mode, keep.data_ptr(),
                                        _lib.stream_ptr(dev)), "select_prompt")
        result.append(keep)
    return result
