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


def _one_launch(key: torch.Tensor, value: torch.Tensor, bits: int, group_size: int) -> bool:
    """Whether ``pk_quantize_pack_kv`` takes the pair: fp16, contiguous, one shape,
    groups of 32 along S and hd (S and hd multiples of 32), 16-byte aligned, on a GPU."""
    if key.dim() != 4 or key.shape != value.shape or bits not in (2, 4, 8) or group_size != 32:
        return False
    S, D = key.shape[2], key.shape[3]
    return (key.dtype == torch.float16 and value.dtype == torch.float16 and key.is_cuda
            and value.device == key.device and key.is_contiguous() and value.is_contiguous()
            and S > 0 and D > 0 and S % 32 == 0 and D % 32 == 0
            and key.data_ptr() % 16 == 0 and value.data_ptr() % 16 == 0)


def pack_kv(key: torch.Tensor, value: torch.Tensor, bits: int, group_size: int) -> PackedKVSegment:
    """Pack a non-empty ``[B, Hkv, S, hd]`` K/V pair the way the cache does
    (``phasekv_cache.py:101-107``): ``quantize_pack(K, axis=-2)`` and
    ``quantize_pack(V, axis=-1)``.  Pairs ``pk_quantize_pack_kv`` takes are packed in one
    launch into the same tensors, views and values the two calls give."""
    if not _one_launch(key, value, bits, group_size):
        return PackedKVSegment(quantize_pack(key, bits, axis=-2, group_size=group_size),
                               quantize_pack(value, bits, axis=-1, group_size=group_size))
    from . import _lib
    B, H, S, D = key.shape
    vpb, dev = 8 // bits, key.device
    u8, f16 = torch.uint8, torch.float16
    # K: token-major codes and group-major metadata under [B, H, D, *] views
    kp = torch.empty(B, H, S // vpb, D, dtype=u8, device=dev).transpose(-1, -2)
    ks = torch.empty(B, H, S // 32, D, dtype=f16, device=dev).transpose(-1, -2)
    km = torch.empty(B, H, S // 32, D, dtype=f16, device=dev).transpose(-1, -2)
    vp = torch.empty(B, H, S, D // vpb, dtype=u8, device=dev)
    vs = torch.empty(B, H, S, D // 32, dtype=f16, device=dev)
    vm = torch.empty(B, H, S, D // 32, dtype=f16, device=dev)
    _lib.check(_lib.load().pk_quantize_pack_kv(
        key.data_ptr(), value.data_ptr(), B, H, S, D, bits, kp.data_ptr(), ks.data_ptr(),
        km.data_ptr(), vp.data_ptr(), vs.data_ptr(), vm.data_ptr(), _lib.stream_ptr(dev)),
        "quantize_pack_kv")
    shape = (B, H, S, D)
    return PackedKVSegment(
        PackedTensor(packed=kp, scale=ks, mins=km, bits=bits, axis=2, group_size=32,
                     orig_shape=shape, axis_len=S),
        PackedTensor(packed=vp, scale=vs, mins=vm, bits=bits, axis=3, group_size=32,
                     orig_shape=shape, axis_len=D))
