"""PhaseKV decode attention for transformers' Llama (installed 5.x API) on ROCm.

Mirrors ``examples/llama_phasekv_adapter.py`` of the reference (transformers 4.46):
``PhaseKVLlamaAttention`` wraps a ``LlamaAttention`` and, on a ``PhaseKVCache``, projects,
applies RoPE, writes K/V and attends over the packed tiers through the HIP decode path
(``llama_phasekv_adapter.py:17-96``); it needs ``pretraining_tp == 1`` as the reference
does (``:60-61``).  ``phasekv_prefill`` / ``phasekv_step`` drive a Llama model as they
drive Qwen2.
"""
from __future__ import annotations

from .qwen2_attention import PhaseKVAttention, phasekv_prefill, phasekv_step  # noqa: F401


class PhaseKVLlamaAttention(PhaseKVAttention):
    fused_rope = True

    @staticmethod
    def rope(q, k, cos, sin):
        from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
        return apply_rotary_pos_emb(q, k, cos, sin)

    def check(self) -> None:
        if getattr(self.original.config, "pretraining_tp", 1) != 1:
            raise ValueError("the PhaseKV Llama path needs pretraining_tp = 1")


def install_llama_phasekv_attention(model) -> int:
    """Wrap every decoder layer's attention of a Llama model; returns the layer count."""
    layers = model.model.layers
    for layer in layers:
        if not isinstance(layer.self_attn, PhaseKVLlamaAttention):
            layer.self_attn = PhaseKVLlamaAttention(layer.self_attn)
    return len(layers)
