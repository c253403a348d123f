"""Three-tier attention semantics on the device (drop-in for the reference's reference.py).

Same names and meaning as ``src/phasekv/kernels/reference.py``: dequantize
every tier to fp16 (HIP ``unpack_dequantize``), concatenate prompt -> cold ->
hot, expand GQA and run fp32 softmax attention with torch on the device.  It
moves the full dequantized KV through HBM, so it is a debugging aid, not the
decode path.  The CPU oracle the tests check against lives outside this
package.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch

from .packing import PackedTensor, unpack_dequantize


@dataclass
class ThreeTierKV:
    """Heterogeneous KV of one layer: packed prompt / cold tiers and an fp16 hot tier.

    Any tier may be None; non-empty tiers are ``[b, Hkv, len, hd]``
    (``reference.py:27-40``).
    """

    prompt_k: Optional[PackedTensor] = None
    prompt_v: Optional[PackedTensor] = None
    cold_k: Optional[PackedTensor] = None
    cold_v: Optional[PackedTensor] = None
    hot_k: Optional[torch.Tensor] = None
    hot_v: Optional[torch.Tensor] = None


def _dequant_concat(kv: ThreeTierKV) -> tuple:
    """Dequantize and concatenate prompt -> cold -> hot on the token axis (``reference.py:43-58``)."""
    ks: List[torch.Tensor] = []
    vs: List[torch.Tensor] = []
    if kv.prompt_k is not None:
        ks.append(unpack_dequantize(kv.prompt_k))
        vs.append(unpack_dequantize(kv.prompt_v))
    if kv.cold_k is not None:
        ks.append(unpack_dequantize(kv.cold_k))
        vs.append(unpack_dequantize(kv.cold_v))
    if kv.hot_k is not None:
        ks.append(kv.hot_k.to(torch.float16))
        vs.append(kv.hot_v.to(torch.float16))
    if not ks:
        raise ValueError("ThreeTierKV has no non-empty tier")
    return torch.cat(ks, dim=-2), torch.cat(vs, dim=-2)


def _expand_gqa(x: torch.Tensor, num_attention_heads: int) -> torch.Tensor:
    """[b, Hkv, S, hd] -> [b, Hq, S, hd]: query head h reads kv head h // (Hq / Hkv)."""
    b, hkv, s, hd = x.shape
    if hkv == num_attention_heads:
        return x
    if num_attention_heads % hkv != 0:
        raise ValueError(f"{num_attention_heads} heads is not a multiple of {hkv} kv heads")
    return x.repeat_interleave(num_attention_heads // hkv, dim=1)


def fused_decode_attention_reference(q: torch.Tensor, kv: ThreeTierKV,
                                     num_attention_heads: int) -> torch.Tensor:
    """softmax(q K^T / sqrt(hd)) V over all tiers in fp32, output fp16 (``reference.py:72-96``)."""
    if q.dim() != 4:
        raise ValueError(f"q must be [b, Hq, q_len, hd], got {tuple(q.shape)}")
    head_dim = q.shape[-1]
    k_all, v_all = _dequant_concat(kv)
    k_all = _expand_gqa(k_all, num_attention_heads).float().contiguous()
    v_all = _expand_gqa(v_all, num_attention_heads).float().contiguous()
    scale = 1.0 / math.sqrt(head_dim)
    scores = torch.matmul(q.float(), k_all.transpose(-1, -2).contiguous()) * scale
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v_all).to(torch.float16)


def dense_fp16_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         num_attention_heads: int) -> torch.Tensor:
    """The same attention over uncompressed fp16 K/V (``reference.py:99-109``)."""
    head_dim = q.shape[-1]
    k = _expand_gqa(k, num_attention_heads).float().contiguous()
    v = _expand_gqa(v, num_attention_heads).float().contiguous()
    scale = 1.0 / math.sqrt(head_dim)
    scores = torch.matmul(q.float(), k.transpose(-1, -2).contiguous()) * scale
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v).to(torch.float16)
