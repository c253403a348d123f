"""Data formats the decode path consumes: one layer's packed segments and FP16 hot window.

Mirrors the duck-typed contract of ``PackedKVSegment`` / ``LayerTiers``
(``src/phasekv/phasekv_cache.py:30-79``) and the cache's K/V packing convention
``_pack_kv`` (``src/phasekv/phasekv_cache.py:101-107``): K is quantized per
channel along tokens (``axis=-2``), V per token along head_dim (``axis=-1``).
The cache's lifecycle (append, cooling, prompt chunks) is ``phasekv_amd.cache``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from .kernels.packing import PackedTensor, quantize_pack


@dataclass
class PackedKVSegment:
    """One packed K/V segment of one layer; ``length`` is the retained token count."""

    key: PackedTensor
    value: PackedTensor

    @property
    def length(self) -> int:
        return self.key.orig_shape[2]

    @property
    def nbytes(self) -> int:
        return self.key.nbytes + self.value.nbytes


@dataclass
class LayerTiers:
    """One layer's cache: read-only prompt, prompt extensions, cold segments, FP16 hot window.

    ``hot_k`` / ``hot_v`` are ``[B, Hkv, capacity, hd]``; the first ``hot_len``
    positions are valid.
    """

    prompt: PackedKVSegment
    prompt_extensions: list = field(default_factory=list)
    cold: list = field(default_factory=list)
    hot_k: Optional[torch.Tensor] = None
    hot_v: Optional[torch.Tensor] = None
    hot_len: int = 0

    @property
    def cold_len(self) -> int:
        return sum(s.length for s in self.cold)

    @property
    def prompt_len(self) -> int:
        return self.prompt.length + sum(s.length for s in self.prompt_extensions)

    @property
    def physical_len(self) -> int:
        return self.prompt_len + self.cold_len + self.hot_len

    def hot_views(self):
        """Views of the written hot positions (strided over the capacity)."""
        if self.hot_k is None or self.hot_v is None:
            raise RuntimeError("hot_k/hot_v are not allocated")
        return self.hot_k[:, :, :self.hot_len, :], self.hot_v[:, :, :self.hot_len, :]


def pack_kv(key: torch.Tensor, value: torch.Tensor, bits: int, group_size: int) -> PackedKVSegment:
    """Pack a non-empty ``[B, Hkv, S, hd]`` K/V pair the way the cache does."""
    return PackedKVSegment(quantize_pack(key, bits, axis=-2, group_size=group_size),
                           quantize_pack(value, bits, axis=-1, group_size=group_size))
