"""PhaseKV decode attention for transformers' Qwen2 (installed 5.x API) on ROCm.

Mirrors ``src/phasekv/qwen2_attention.py`` of the reference (written for transformers
4.46): ``install_qwen2_phasekv_attention(model)`` wraps every layer's attention so that,
when the layer is called with a ``phasekv_amd.cache.PhaseKVCache``, it projects q/k/v
with the layer's own weights, applies RoPE at the true positions, writes K/V into the
cache and attends over the packed tiers with the HIP decode path
(``qwen2_attention.py:32-109``).  Any other cache goes to the original module.

Differences: transformers 5.x passes ``past_key_values`` and ``position_embeddings``
and expects ``(output, weights)``; a new input chunk is appended in one launch and
attended in one pass by ``fused_phasekv_prompt_chunk_attention`` (the reference loops
token by token, ``:100-106``); a decode step's RoPE, fp16 casts and window append are
one launch (``PhaseKVCache.rope_append_hot``, ``:89-92, 77``).  ``phasekv_prefill`` and ``phasekv_step`` drive
the model the way the reference's usage notes do: prefill with the dense cache and the
eager attention (for the selection votes), then one step per token, then
``finish_decode_step`` / ``finish_prompt_chunk`` after the whole forward pass.
"""
from __future__ import annotations

import torch
from torch import nn

from .cache import PhaseKVCache
from .kernels.attention_triton import (fused_phasekv_decode,
                                       fused_phasekv_prompt_chunk_attention)
from .prompt_tier import select_prompt_indices


class PhaseKVAttention(nn.Module):
    """Reuses the wrapped attention's projections; handles single-token decode and input
    chunks on a ``PhaseKVCache``.  The layer only writes K/V and attends; the caller
    calls ``finish_decode_step`` / ``finish_prompt_chunk`` after the model's forward.
    Subclasses give the model family's RoPE; ``fused_rope`` says it is the rotate_half
    form, which a decode step applies in the window-append launch
    (``PhaseKVCache.rope_append_hot``)."""

    fused_rope = False

    def __init__(self, original: nn.Module):
        super().__init__()
        self.original = original
        self.layer_idx = original.layer_idx
        self.train(original.training)

    @staticmethod
    def rope(q, k, cos, sin):
        raise NotImplementedError

    def check(self) -> None:
        """Model-family conditions of the PhaseKV path."""

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                past_key_values=None, **kwargs):
        if not isinstance(past_key_values, PhaseKVCache):
            return self.original(hidden_states, position_embeddings, attention_mask,
                                 past_key_values=past_key_values, **kwargs)
        batch, q_len, _ = hidden_states.shape
        if batch != 1 or hidden_states.dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("the PhaseKV attention takes batch = 1 in float16 / bfloat16")
        if self.training:
            raise ValueError("PhaseKV decode needs eval()")
        self.check()
        cache = past_key_values
        if cache.prompt_chunk_len:
            if q_len != cache.prompt_chunk_len:
                raise ValueError(f"the open prompt chunk has {cache.prompt_chunk_len} tokens, "
                                 f"got {q_len}")
        elif q_len != 1:
            raise ValueError(f"PhaseKV decode takes q_len = 1, got {q_len}; call "
                             "begin_prompt_chunk(length) for a new input chunk")
        base = self.original
        cfg = base.config
        hq, hkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, base.head_dim
        if position_embeddings is None:
            raise ValueError("position_embeddings (RoPE cos, sin at the true positions) are needed")
        if (self.fused_rope and not cache.prompt_chunk_len
                and position_embeddings[0].dtype == hidden_states.dtype):
            # one launch: q and k rotated, cast to fp16, k and v written into the window
            q = cache.rope_append_hot(self.layer_idx, base.q_proj(hidden_states),
                                      base.k_proj(hidden_states), base.v_proj(hidden_states),
                                      *position_embeddings, hq)
            out = fused_phasekv_decode(q[0], cache.layer_tiers(self.layer_idx), hq)
            out = out.reshape(batch, q_len, hq * hd).to(hidden_states.dtype)
            return base.o_proj(out), None
        q = base.q_proj(hidden_states).view(batch, q_len, hq, hd).transpose(1, 2)
        k = base.k_proj(hidden_states).view(batch, q_len, hkv, hd).transpose(1, 2)
        v = base.v_proj(hidden_states).view(batch, q_len, hkv, hd).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = self.rope(q, k, cos, sin)
        q, k, v = q.to(torch.float16), k.to(torch.float16), v.to(torch.float16)
        tiers = cache.layer_tiers(self.layer_idx)
        if cache.prompt_chunk_len:
            cache.append_prompt_chunk(self.layer_idx, k, v)
            out = fused_phasekv_prompt_chunk_attention(q[0].transpose(0, 1).contiguous(), tiers, hq)
        else:
            cache.append_hot(self.layer_idx, k, v)
            out = fused_phasekv_decode(q[0, :, 0, :], tiers, hq).unsqueeze(0)
        out = out.reshape(batch, q_len, hq * hd).to(hidden_states.dtype)
        return base.o_proj(out), None


class PhaseKVQwen2Attention(PhaseKVAttention):
    """``PhaseKVQwen2Attention`` of ``qwen2_attention.py:19-109``."""

    fused_rope = True

    @staticmethod
    def rope(q, k, cos, sin):
        from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
        return apply_rotary_pos_emb(q, k, cos, sin)


def install_qwen2_phasekv_attention(model) -> int:
    """Wrap every decoder layer's attention of a Qwen2 model; returns the layer count."""
    layers = model.model.layers
    for layer in layers:
        if not isinstance(layer.self_attn, PhaseKVQwen2Attention):
            layer.self_attn = PhaseKVQwen2Attention(layer.self_attn)
    return len(layers)


class _DenseKV:
    """``key_cache`` / ``value_cache`` lists of a transformers 5.x ``DynamicCache``."""

    def __init__(self, cache):
        self.key_cache = [layer.keys for layer in cache.layers]
        self.value_cache = [layer.values for layer in cache.layers]


@torch.no_grad()
def phasekv_prefill(model, input_ids: torch.Tensor, *, prefill_keep_ratio: float = 1.0,
                    sink_tokens: int = 4, obs_window: int = 32, pool_kernel: int = 7,
                    pooling: str = "maxpool", **cache_kwargs):
    """Dense prefill of ``input_ids`` ``[1, S]``, then prompt selection and packing.

    Returns ``(logits of the last position, PhaseKVCache)``.  With
    ``prefill_keep_ratio < 1`` the prefill runs the eager attention so the selection
    can read the observation window's attention rows (``prompt_tier.py:22-76``).
    """
    from transformers import DynamicCache
    S = input_ids.shape[1]
    dense = DynamicCache(config=model.config)
    select = prefill_keep_ratio < 1.0
    out = model(input_ids, past_key_values=dense, use_cache=True, output_attentions=select)
    keep = None
    if select:
        keep = select_prompt_indices(list(out.attentions), prompt_len=S,
                                     model_config=model.config,
                                     prefill_keep_ratio=prefill_keep_ratio,
                                     sink_tokens=sink_tokens, obs_window=obs_window,
                                     pool_kernel=pool_kernel, pooling=pooling)
    cache = PhaseKVCache.from_dense_prefill(_DenseKV(dense), prompt_len=S, keep_indices=keep,
                                            **cache_kwargs)
    return out.logits[:, -1], cache


@torch.no_grad()
def phasekv_step(model, input_ids: torch.Tensor, cache: PhaseKVCache) -> torch.Tensor:
    """One forward over ``input_ids`` ``[1, T]`` on the packed cache: T = 1 is a decode
    step, T > 1 a new input chunk.  Returns the last position's logits."""
    T = input_ids.shape[1]
    if T > 1:
        cache.begin_prompt_chunk(T)
    start = cache.true_seq_length
    pos = torch.arange(start, start + T, device=input_ids.device).unsqueeze(0)
    # a 4-D mask is passed through as is: transformers builds no mask and asks the
    # cache nothing (the PhaseKV attention ignores the mask; causality comes from the
    # append order and the chunk attention)
    mask = torch.zeros(1, 1, T, 1, dtype=torch.bool, device=input_ids.device)
    out = model(input_ids, position_ids=pos, past_key_values=cache, attention_mask=mask,
                use_cache=True)
    if T > 1:
        cache.finish_prompt_chunk()
    else:
        cache.finish_decode_step()
    return out.logits[:, -1]
