"""The decode-side lifecycle of the packed cache on the GPU: prompt packing at
prefill, one FP16 hot-window append per layer per generated token, and the lazy
cooling of the oldest hot tokens into packed cold segments.

Mirrors ``PhaseKVCache`` of ``src/phasekv/phasekv_cache.py`` for the single-token
decode loop:

* ``from_dense_prefill``   ``phasekv_cache.py:182-263`` (prompt selection by
  ``keep_indices`` and packing)
* ``append_hot``           ``phasekv_cache.py:291-301`` and ``_append_token``
  ``:405-422`` (one HIP launch writes K and V)
* ``rope_append_hot``      the adapters' rotary embedding plus ``append_hot`` of one
  decode token (``qwen2_attention.py:89-92, 77``) in one HIP launch
* ``finish_decode_step``   ``phasekv_cache.py:302-320``
* ``_cool_aged_tokens``    ``phasekv_cache.py:322-340``: one HIP launch ranks the
  aged tokens by value norm, gathers and packs the kept ones into the new cold
  segment and shifts the hot tail (windows too large for one workgroup's LDS:
  a cooling launch, then two ``quantize_pack`` launches)
* accessors ``__len__``, ``layer_tiers``, ``get_seq_length``, ``get_max_cache_shape``,
  ``true_seq_length``, ``physical_nbytes`` (``:265-289``, ``:436-445``)

* multi-turn prompt chunks ``begin_prompt_chunk`` / ``append_prompt_token`` /
  ``finish_prompt_chunk`` (``:342-403``): the chunk borrows the hot window, and is packed
  with ``prompt_bits`` into a prompt extension at its end; ``append_prompt_chunk``
  writes a layer's chunk rows in one launch
* ``reorder_cache`` (``:454-478``): batch reorder of every tier, keeping the transposed
  K storage ``quantize_pack`` gives

``update`` refuses dense use as the reference does (``:447-452``).  The class does not
derive from ``transformers.cache_utils.Cache``: it is driven by the decode loop directly.
"""
from __future__ import annotations

from numbers import Integral, Real
from typing import Optional, Sequence

import torch

from . import _lib
from .kernels.packing import PackedTensor, quantize_pack
from .tiers import LayerTiers, PackedKVSegment, pack_kv

_PACKED_BITS = (2, 4, 8)
_INDEX_DTYPES = (torch.uint8, torch.int8, torch.int16, torch.int32, torch.int64)
COOL_MAX_AGED = 4096   # PK_COOL_MAX_AGED of the C ABI


def _require_positive_int(name: str, value) -> None:
    if isinstance(value, bool) or not isinstance(value, Integral) or value <= 0:
        raise ValueError(f"{name} must be a positive integer, got {value!r}")


def _validate_config(prompt_bits, cold_bits, group_size, recent_window, lazy_g,
                     decode_keep_ratio) -> None:
    """Checks shared by both constructors (``phasekv_cache.py:87-98``)."""
    for name, bits in (("prompt_bits", prompt_bits), ("cold_bits", cold_bits)):
        if isinstance(bits, bool) or not isinstance(bits, Integral) or bits not in _PACKED_BITS:
            raise ValueError(f"{name} must be 2, 4 or 8 for packed storage, got {bits!r}")
    for name, value in (("group_size", group_size), ("recent_window", recent_window),
                        ("lazy_g", lazy_g)):
        _require_positive_int(name, value)
    if (isinstance(decode_keep_ratio, bool) or not isinstance(decode_keep_ratio, Real)
            or not 0.0 < decode_keep_ratio <= 1.0):
        raise ValueError(f"decode_keep_ratio must lie in (0, 1], got {decode_keep_ratio!r}")


def keep_count(aged: int, decode_keep_ratio: float) -> int:
    """Tokens kept out of ``aged`` (``phasekv_cache.py:329``: Python's round)."""
    return max(1, round(decode_keep_ratio * aged))


def cool_hot(hot_k: torch.Tensor, hot_v: torch.Tensor, hot_len: int, aged: int, keep: int,
             with_index: bool = False):
    """One cooling launch over ``[B, Hkv, capacity, hd]`` fp16 hot buffers.

    Returns ``(kept_k, kept_v, index)``: the kept rows ``[B, Hkv, keep, hd]`` in token
    order and, if asked, their token indices ``[B, Hkv, keep]`` (int64).  Rows
    ``[aged, hot_len)`` of the hot buffers move to ``[0, hot_len - aged)``.
    """
    dev = _lib.require_device(hot_k, hot_v)
    if hot_k.dtype != torch.float16 or hot_v.dtype != torch.float16:
        raise ValueError("hot buffers must be float16")
    if hot_k.shape != hot_v.shape or hot_k.stride() != hot_v.stride() or hot_k.ndim != 4:
        raise ValueError("hot_k and hot_v must be [B, Hkv, capacity, hd] with the same strides")
    if hot_k.stride(-1) != 1:
        raise ValueError("hot buffers must have a contiguous head_dim")
    if not 0 < aged <= hot_len <= hot_k.shape[2]:
        raise ValueError(f"need 0 < aged <= hot_len <= capacity, got {aged}, {hot_len}, "
                         f"{hot_k.shape[2]}")
    if aged > COOL_MAX_AGED:
        raise ValueError(f"a cooling step takes at most {COOL_MAX_AGED} tokens, got {aged}")
    if not 0 < keep <= aged:
        raise ValueError(f"keep must lie in [1, aged], got {keep}")
    B, H, _, D = hot_k.shape
    kept_k = torch.empty(B, H, keep, D, dtype=torch.float16, device=dev)
    kept_v = torch.empty_like(kept_k)
    index = torch.empty(B, H, keep, dtype=torch.int64, device=dev) if with_index else None
    lib = _lib.load()
    _lib.check(lib.pk_cool_hot(hot_k.data_ptr(), hot_v.data_ptr(), hot_k.stride(0),
                               hot_k.stride(1), hot_k.stride(2), B, H, D, hot_len, aged, keep,
                               kept_k.data_ptr(), kept_v.data_ptr(),
                               index.data_ptr() if index is not None else None,
                               _lib.stream_ptr(dev)), "cool_hot")
    return kept_k, kept_v, index


def cool_pack_hot(hot_k: torch.Tensor, hot_v: torch.Tensor, hot_len: int, aged: int, keep: int,
                  bits: int, group_size: int, with_index: bool = False):
    """One cooling step and the packing of its cold segment in one launch.

    Returns ``(segment, index)``: a ``PackedKVSegment`` identical to
    ``pack_kv(kept_k, kept_v, bits, group_size)`` over the rows ``cool_hot`` would
    keep (the same tensors, shapes and views ``quantize_pack`` gives), and the kept
    token indices if asked.  Windows the fused launch does not take (see
    ``cool_pack_supported``) go through ``cool_hot`` and two ``quantize_pack``
    launches instead.
    """
    dev = _lib.require_device(hot_k, hot_v)
    B, H, _, D = hot_k.shape
    if not cool_pack_supported(hot_k, hot_v, hot_len, aged, keep, group_size):
        key, value, index = cool_hot(hot_k, hot_v, hot_len, aged, keep, with_index)
        return PackedKVSegment(quantize_pack(key, bits, axis=-2, group_size=group_size),
                               quantize_pack(value, bits, axis=-1, group_size=group_size)), index
    if bits not in _PACKED_BITS:
        raise ValueError(f"bits must be one of {_PACKED_BITS}, got {bits}")
    vpb = 8 // bits
    gsk, gsv = min(group_size, keep), min(group_size, D)
    ngk, nbk = -(-keep // gsk), -(-keep // vpb)
    ngv, nbv = -(-D // gsv), -(-D // vpb)
    u8, f16 = torch.uint8, torch.float16
    # the storage quantize_pack gives K (axis -2: transposed views) and V (axis -1)
    kp = torch.empty(B, H, nbk, D, dtype=u8, device=dev).transpose(-1, -2)
    ks = torch.empty(B, H, ngk, D, dtype=f16, device=dev).transpose(-1, -2)
    km = torch.empty(B, H, ngk, D, dtype=f16, device=dev).transpose(-1, -2)
    vp = torch.empty(B, H, keep, nbv, dtype=u8, device=dev)
    vs = torch.empty(B, H, keep, ngv, dtype=f16, device=dev)
    vm = torch.empty(B, H, keep, ngv, dtype=f16, device=dev)
    index = torch.empty(B, H, keep, dtype=torch.int64, device=dev) if with_index else None
    lib = _lib.load()
    _lib.check(lib.pk_cool_pack_hot(hot_k.data_ptr(), hot_v.data_ptr(), hot_k.stride(0),
                                    hot_k.stride(1), hot_k.stride(2), B, H, D, hot_len, aged,
                                    keep, bits, group_size, kp.data_ptr(), ks.data_ptr(),
                                    km.data_ptr(), vp.data_ptr(), vs.data_ptr(), vm.data_ptr(),
                                    index.data_ptr() if index is not None else None,
                                    _lib.stream_ptr(dev)), "cool_pack_hot")
    shape = (B, H, keep, D)
    key = PackedTensor(packed=kp, scale=ks, mins=km, bits=bits, axis=2, group_size=gsk,
                       orig_shape=shape, axis_len=keep)
    value = PackedTensor(packed=vp, scale=vs, mins=vm, bits=bits, axis=3, group_size=gsv,
                         orig_shape=shape, axis_len=D)
    return PackedKVSegment(key, value), index


def cool_pack_supported(hot_k: torch.Tensor, hot_v: torch.Tensor, hot_len: int, aged: int,
                        keep: int, group_size: int) -> bool:
    """Whether ``cool_pack_hot`` runs as one launch for these buffers and sizes."""
    D = hot_k.shape[-1]
    pieces = all(s % 8 == 0 for s in hot_k.stride()[:3]) and hot_k.stride() == hot_v.stride()
    aligned = hot_k.data_ptr() % 16 == 0 and hot_v.data_ptr() % 16 == 0
    return bool(pieces and aligned and hot_k.stride(-1) == 1 and hot_k.dtype == torch.float16
                and hot_v.dtype == torch.float16
                and _lib.load().pk_cool_pack_supported(hot_len, D, aged, keep, group_size))


class PhaseKVCache:
    """Packed cache of all layers: read-only prompt, frozen cold segments, FP16 hot window.

    ``get_seq_length()`` is the number of tokens a layer holds; ``true_seq_length``
    the number of tokens committed by finished forward passes (the next RoPE
    position).  Within a decode step every layer appends once with ``append_hot``
    and reads ``layer_tiers`` for its attention; ``finish_decode_step`` then cools
    every layer and advances the true length.
    """

    def __init__(self, layers: list, *, seen_tokens: int, prompt_bits: int, cold_bits: int,
                 group_size: int, recent_window: int, lazy_g: int,
                 decode_keep_ratio: float) -> None:
        _validate_config(prompt_bits, cold_bits, group_size, recent_window, lazy_g,
                         decode_keep_ratio)
        _require_positive_int("seen_tokens", seen_tokens)
        if not layers:
            raise ValueError("layers must not be empty: the cache needs at least one layer")
        for layer_idx, layer in enumerate(layers):
            if layer.hot_k is None or layer.hot_v is None:
                raise ValueError(f"layer {layer_idx} has no hot_k/hot_v; build the cache with "
                                 "from_dense_prefill()")
        self.layers = layers
        self._seen_tokens = int(seen_tokens)
        self.prompt_bits = prompt_bits
        self.cold_bits = cold_bits
        self.group_size = group_size
        self.recent_window = recent_window
        self.lazy_g = lazy_g
        self.decode_keep_ratio = decode_keep_ratio
        self._pending_layers: set = set()
        # 0: no prompt chunk open; else its length, and every layer's hot_len at its start
        self._prompt_chunk_len = 0
        self._prompt_chunk_start: list = []

    @classmethod
    @torch.no_grad()
    def from_dense_prefill(cls, dense_cache, *, prompt_len: int,
                           keep_indices: Optional[Sequence[torch.Tensor]] = None,
                           prompt_bits: int = 2, cold_bits: int = 4, group_size: int = 32,
                           recent_window: int = 32, lazy_g: int = 16,
                           decode_keep_ratio: float = 1.0) -> "PhaseKVCache":
        """Select and pack the prefill K/V without modifying ``dense_cache``.

        ``dense_cache`` provides per-layer ``key_cache`` / ``value_cache`` lists of
        ``[B, Hkv, prompt_len, hd]`` float16 or bfloat16 tensors (K with RoPE
        applied).  ``keep_indices[layer]`` are ``[B, Hkv, K0]`` integer positions
        (the same K0 for every layer), or None to keep every token.
        """
        _require_positive_int("prompt_len", prompt_len)
        _validate_config(prompt_bits, cold_bits, group_size, recent_window, lazy_g,
                         decode_keep_ratio)
        if not hasattr(dense_cache, "key_cache") or not hasattr(dense_cache, "value_cache"):
            raise TypeError("dense_cache must provide per-layer key_cache/value_cache")
        keys, values = dense_cache.key_cache, dense_cache.value_cache
        if len(keys) == 0 or len(keys) != len(values):
            raise ValueError(f"prefill K/V need the same non-zero number of layers, got "
                             f"{len(keys)}/{len(values)}")
        if keep_indices is not None and len(keep_indices) != len(keys):
            raise ValueError(f"keep_indices needs {len(keys)} layers, got {len(keep_indices)}")
        capacity = recent_window + lazy_g
        layers = []
        retained = None
        for layer_idx, (key, value) in enumerate(zip(keys, values)):
            context = f"layer {layer_idx} prefill"
            if not isinstance(key, torch.Tensor) or not isinstance(value, torch.Tensor):
                raise TypeError(f"{context} K/V must be tensors")
            if key.ndim != 4 or key.shape != value.shape or any(n == 0 for n in key.shape):
                raise ValueError(f"{context} K/V must be non-empty [B,Hkv,S,hd] of one shape, got "
                                 f"{tuple(key.shape)}/{tuple(value.shape)}")
            if key.dtype not in (torch.float16, torch.bfloat16) or value.dtype != key.dtype:
                raise ValueError(f"{context} K/V must both be float16 or bfloat16, got "
                                 f"{key.dtype}/{value.dtype}")
            if key.device != value.device:
                raise ValueError(f"{context} K/V must be on one device")
            _lib.require_device(key, value)
            if key.shape[2] != prompt_len:
                raise ValueError(f"{context} K/V length should be prompt_len={prompt_len}, got "
                                 f"{key.shape[2]}")
            if keep_indices is not None:
                indices = keep_indices[layer_idx]
                if not isinstance(indices, torch.Tensor) or indices.dtype not in _INDEX_DTYPES:
                    raise ValueError(f"layer {layer_idx} keep_indices must be an integer tensor")
                if indices.ndim != 3 or indices.shape[:2] != key.shape[:2] or indices.shape[2] == 0:
                    raise ValueError(f"layer {layer_idx} keep_indices should be "
                                     f"[{key.shape[0]},{key.shape[1]},K0] with K0>0, got "
                                     f"{tuple(indices.shape)}")
                indices = indices.to(device=key.device, dtype=torch.long).sort(dim=-1).values
                if bool((indices < 0).any()) or bool((indices >= prompt_len).any()):
                    raise ValueError(f"layer {layer_idx} keep_indices must lie in [0, {prompt_len})")
                if bool((indices[..., 1:] == indices[..., :-1]).any()):
                    raise ValueError(f"layer {layer_idx} keep_indices repeat a position")
                gather = indices.unsqueeze(-1).expand(*indices.shape, key.shape[-1])
                key, value = key.gather(2, gather), value.gather(2, gather)
            if retained is not None and key.shape[2] != retained:
                raise ValueError(f"every layer must keep the same number of prompt tokens: layer 0 "
                                 f"keeps {retained}, layer {layer_idx} keeps {key.shape[2]}")
            retained = key.shape[2]
            key, value = key.to(torch.float16), value.to(torch.float16)
            shape = (key.shape[0], key.shape[1], capacity, key.shape[3])
            layers.append(LayerTiers(
                prompt=pack_kv(key, value, prompt_bits, group_size),
                hot_k=torch.empty(shape, dtype=torch.float16, device=key.device),
                hot_v=torch.empty(shape, dtype=torch.float16, device=key.device)))
        return cls(layers, seen_tokens=prompt_len, prompt_bits=prompt_bits,
                   cold_bits=cold_bits, group_size=group_size, recent_window=recent_window,
                   lazy_g=lazy_g, decode_keep_ratio=decode_keep_ratio)

    # ---- accessors ----------------------------------------------------------
    def __len__(self) -> int:
        return len(self.layers)

    def layer_tiers(self, layer_idx: int) -> LayerTiers:
        if (isinstance(layer_idx, bool) or not isinstance(layer_idx, Integral)
                or not 0 <= layer_idx < len(self.layers)):
            raise IndexError(f"layer_idx must be an integer in [0, {len(self.layers)}), got "
                             f"{layer_idx!r}")
        return self.layers[layer_idx]

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self.layer_tiers(0 if layer_idx is None else layer_idx).physical_len

    def get_max_cache_shape(self) -> None:
        """Frozen segments grow without bound: there is no maximum length."""
        return None

    @property
    def true_seq_length(self) -> int:
        return self._seen_tokens

    @property
    def prompt_chunk_len(self) -> int:
        return self._prompt_chunk_len

    def physical_nbytes(self) -> int:
        """Bytes of the KV tensors held, hot capacity included."""
        total = 0
        for layer in self.layers:
            total += layer.prompt.nbytes
            total += sum(s.nbytes for s in layer.prompt_extensions)
            total += sum(s.nbytes for s in layer.cold)
            total += layer.hot_k.numel() * layer.hot_k.element_size()
            total += layer.hot_v.numel() * layer.hot_v.element_size()
        return total

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        raise RuntimeError("PhaseKVCache returns no dense K/V: decode through append_hot() and "
                           "layer_tiers() instead of Cache.update()")

    # ---- decode step --------------------------------------------------------
    @torch.no_grad()
    def append_hot(self, layer_idx: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Write this step's rotated K and its V (``[B, Hkv, 1, hd]`` fp16) for one layer."""
        if self._prompt_chunk_len:
            raise RuntimeError("a prompt chunk is open: append with append_prompt_token() and "
                               "close it with finish_prompt_chunk()")
        layer = self.layer_tiers(layer_idx)
        if layer_idx in self._pending_layers:
            raise RuntimeError(f"layer {layer_idx} already appended in this decode step; call "
                               "finish_decode_step() after the forward pass")
        self._append_token(layer_idx, layer, key, value)
        self._pending_layers.add(layer_idx)

    @torch.no_grad()
    def rope_append_hot(self, layer_idx: int, query: torch.Tensor, key: torch.Tensor,
                        value: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                        num_attention_heads: int) -> torch.Tensor:
        """``apply_rotary_pos_emb`` (rotate_half form), the fp16 casts and ``append_hot``
        of one decode token in one launch; returns the rotated query ``[B, Hq, hd]`` fp16.

        ``query`` / ``key`` / ``value`` are the projections ``[B, 1, H*hd]`` (head_dim
        contiguous) and ``cos`` / ``sin`` ``[B or 1, 1, hd]``, all float16 or all
        bfloat16.  The rotated K and the V go into the window as ``append_hot`` writes
        them, bit-identical to ``x * cos + rotate_half(x) * sin`` on the tensors
        followed by ``.to(torch.float16)`` (``qwen2_attention.py:89-92, 77``).
        """
        if self._prompt_chunk_len:
            raise RuntimeError("a prompt chunk is open: append with append_prompt_token() and "
                               "close it with finish_prompt_chunk()")
        layer = self.layer_tiers(layer_idx)
        if layer_idx in self._pending_layers:
            raise RuntimeError(f"layer {layer_idx} already appended in this decode step; call "
                               "finish_decode_step() after the forward pass")
        hk, hv = layer.hot_k, layer.hot_v
        B, hkv, cap, hd = hk.shape
        hq = int(num_attention_heads)
        tensors = (query, key, value, cos, sin)
        if not all(isinstance(t, torch.Tensor) for t in tensors):
            raise TypeError(f"layer {layer_idx} query / key / value / cos / sin must be tensors")
        dtype = query.dtype
        if dtype not in (torch.float16, torch.bfloat16) or any(t.dtype != dtype for t in tensors):
            raise ValueError(f"layer {layer_idx} query / key / value / cos / sin must be all "
                             "float16 or all bfloat16")
        if hq <= 0 or hq % hkv:
            raise ValueError(f"num_attention_heads {hq} must be a positive multiple of {hkv}")
        if (tuple(query.shape) != (B, 1, hq * hd) or tuple(key.shape) != (B, 1, hkv * hd)
                or key.shape != value.shape):
            raise ValueError(f"layer {layer_idx} projections must be [B, 1, H*hd] = "
                             f"{(B, 1, hq * hd)} / {(B, 1, hkv * hd)}, got {tuple(query.shape)} / "
                             f"{tuple(key.shape)} / {tuple(value.shape)}")
        if cos.shape != sin.shape or cos.dim() != 3 or cos.shape[0] not in (1, B) \
                or tuple(cos.shape[1:]) != (1, hd):
            raise ValueError(f"cos / sin must be [B or 1, 1, {hd}], got {tuple(cos.shape)} / "
                             f"{tuple(sin.shape)}")
        dev = hk.device
        if any(t.device != dev for t in tensors):
            raise ValueError(f"layer {layer_idx} tensors must be on the hot window's device {dev}")
        if layer.hot_len >= cap:
            raise RuntimeError(f"layer {layer_idx} hot window is full: hot_len={layer.hot_len}, "
                               f"capacity={cap}")
        if hk.stride() != hv.stride() or hk.stride(-1) != 1:
            raise ValueError("hot_k and hot_v must share strides with a contiguous head_dim")
        if query.stride(-1) != 1:
            query = query.contiguous()
        if key.stride(-1) != 1 or value.stride(-1) != 1 or key.stride(0) != value.stride(0):
            key, value = key.contiguous(), value.contiguous()
        if cos.stride(-1) != 1 or sin.stride(-1) != 1 or cos.stride(0) != sin.stride(0):
            cos, sin = cos.contiguous(), sin.contiguous()
        q_out = torch.empty(B, hq, hd, dtype=torch.float16, device=dev)
        cs_bstride = cos.stride(0) if cos.shape[0] == B and B > 1 else 0
        q_bstride = query.stride(0) if B > 1 else hq * hd     # unused for one row
        kv_bstride = key.stride(0) if B > 1 else hkv * hd
        _lib.check(_lib.load().pk_rope_append_hot(
            query.data_ptr(), q_bstride, key.data_ptr(), value.data_ptr(), kv_bstride,
            cos.data_ptr(), sin.data_ptr(), cs_bstride,
            _lib.PK_DTYPE_BF16 if dtype == torch.bfloat16 else _lib.PK_DTYPE_F16,
            q_out.data_ptr(), hk.data_ptr(),
            hv.data_ptr(), hk.stride(0), hk.stride(1), hk.stride(2), B, hq, hkv, hd,
            layer.hot_len, cap, _lib.stream_ptr(dev)), "rope_append_hot")
        layer.hot_len += 1
        self._pending_layers.add(layer_idx)
        return q_out

    def _append_token(self, layer_idx: int, layer: LayerTiers, key: torch.Tensor,
                      value: torch.Tensor) -> None:
        """One token into the window (``phasekv_cache.py:405-422``); checks before any write."""
        context = f"layer {layer_idx} new K/V"
        if not isinstance(key, torch.Tensor) or not isinstance(value, torch.Tensor):
            raise TypeError(f"{context} must be tensors")
        expected = (*layer.hot_k.shape[:2], 1, layer.hot_k.shape[-1])
        if tuple(key.shape) != expected or tuple(value.shape) != expected:
            raise ValueError(f"{context} must be one token of shape {expected}, got "
                             f"{tuple(key.shape)}/{tuple(value.shape)}")
        if key.dtype != torch.float16 or value.dtype != torch.float16:
            raise ValueError(f"{context} must be float16, got {key.dtype}/{value.dtype}")
        if key.device != layer.hot_k.device or value.device != layer.hot_v.device:
            raise ValueError(f"{context} must be on the hot window's device {layer.hot_k.device}")
        if layer.hot_len >= layer.hot_k.shape[2]:
            raise RuntimeError(f"layer {layer_idx} hot window is full: hot_len={layer.hot_len}, "
                               f"capacity={layer.hot_k.shape[2]}")
        if key.stride(-1) != 1 or value.stride(-1) != 1:
            key, value = key.contiguous(), value.contiguous()
        hk, hv = layer.hot_k, layer.hot_v
        if hk.stride() != hv.stride() or hk.stride(-1) != 1:
            raise ValueError("hot_k and hot_v must share strides with a contiguous head_dim")
        lib = _lib.load()
        _lib.check(lib.pk_append_hot(key.data_ptr(), value.data_ptr(), key.stride(0),
                                     key.stride(1), value.stride(0), value.stride(1),
                                     hk.data_ptr(), hv.data_ptr(), hk.stride(0), hk.stride(1),
                                     hk.stride(2), hk.shape[0], hk.shape[1], hk.shape[3],
                                     layer.hot_len, hk.shape[2], _lib.stream_ptr(hk.device)),
                   "append_hot")
        layer.hot_len += 1

    @torch.no_grad()
    def finish_decode_step(self) -> None:
        """After the forward pass of one token: cool every layer, advance the true length."""
        if self._prompt_chunk_len:
            raise RuntimeError("a prompt chunk is open: call finish_prompt_chunk(), not "
                               "finish_decode_step()")
        missing = sorted(set(range(len(self.layers))) - self._pending_layers)
        if missing:
            raise RuntimeError(f"finish_decode_step() needs one appended token per layer; "
                               f"missing layers {missing}")
        lengths = [(layer.physical_len, layer.hot_len) for layer in self.layers]
        if len(set(lengths)) != 1:
            raise RuntimeError(f"layers disagree on (physical length, hot length) before cooling: "
                               f"{lengths}")
        for layer in self.layers:
            self._cool_aged_tokens(layer)
        self._seen_tokens += 1
        self._pending_layers.clear()

    def _cool_aged_tokens(self, layer: LayerTiers) -> None:
        """Move the oldest batch of hot tokens into a cold segment once ``lazy_g`` have aged."""
        aged = layer.hot_len - self.recent_window
        if aged < self.lazy_g:
            return
        keep = keep_count(aged, self.decode_keep_ratio)
        segment, _ = cool_pack_hot(layer.hot_k, layer.hot_v, layer.hot_len, aged, keep,
                                   self.cold_bits, self.group_size)
        layer.cold.append(segment)
        layer.hot_len -= aged

    # ---- multi-turn prompt chunks -------------------------------------------
    def _require_idle(self, operation: str) -> None:
        if self._prompt_chunk_len:
            raise RuntimeError(f"{operation} cannot run inside a prompt chunk; call "
                               "finish_prompt_chunk() first")
        if self._pending_layers:
            raise RuntimeError(f"{operation} cannot run inside a decode step; layers "
                               f"{sorted(self._pending_layers)} appended, call finish_decode_step()")

    @staticmethod
    def _empty_hot(layer: LayerTiers, capacity: int):
        shape = (*layer.hot_k.shape[:2], capacity, layer.hot_k.shape[-1])
        return layer.hot_k.new_empty(shape), layer.hot_v.new_empty(shape)

    @torch.no_grad()
    def begin_prompt_chunk(self, length: int) -> None:
        """Reserve window rows for a new input chunk of ``length`` tokens (between steps)."""
        _require_positive_int("length", length)
        self._require_idle("begin_prompt_chunk()")
        for layer in self.layers:
            needed = layer.hot_len + length
            if needed <= layer.hot_k.shape[2]:
                continue
            new_k, new_v = self._empty_hot(layer, needed)
            new_k[:, :, :layer.hot_len].copy_(layer.hot_k[:, :, :layer.hot_len])
            new_v[:, :, :layer.hot_len].copy_(layer.hot_v[:, :, :layer.hot_len])
            layer.hot_k, layer.hot_v = new_k, new_v
        self._prompt_chunk_start = [layer.hot_len for layer in self.layers]
        self._prompt_chunk_len = length

    @torch.no_grad()
    def append_prompt_token(self, layer_idx: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """One chunk token for one layer; its attention then sees no later chunk token."""
        if not self._prompt_chunk_len:
            raise RuntimeError("no prompt chunk is open; call begin_prompt_chunk(length) first")
        layer = self.layer_tiers(layer_idx)
        written = layer.hot_len - self._prompt_chunk_start[layer_idx]
        if written >= self._prompt_chunk_len:
            raise RuntimeError(f"layer {layer_idx} already holds the chunk's "
                               f"{self._prompt_chunk_len} tokens")
        self._append_token(layer_idx, layer, key, value)

    @torch.no_grad()
    def append_prompt_chunk(self, layer_idx: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """The next ``T`` chunk tokens of one layer (``[B, Hkv, T, hd]`` fp16) in one launch:
        the window rows equal ``T`` calls of ``append_prompt_token``
        (``qwen2_attention.py:100-106``).  Causality comes from the chunk attention's
        per-row lengths, as with the per-token appends."""
        if not self._prompt_chunk_len:
            raise RuntimeError("no prompt chunk is open; call begin_prompt_chunk(length) first")
        layer = self.layer_tiers(layer_idx)
        context = f"layer {layer_idx} chunk K/V"
        if not isinstance(key, torch.Tensor) or not isinstance(value, torch.Tensor):
            raise TypeError(f"{context} must be tensors")
        hk, hv = layer.hot_k, layer.hot_v
        B, hkv, cap, hd = hk.shape
        if key.dim() != 4 or key.shape != value.shape or tuple(key.shape[:2]) != (B, hkv) \
                or key.shape[3] != hd or key.shape[2] <= 0:
            raise ValueError(f"{context} must be [B, Hkv, T, hd] = [{B}, {hkv}, T, {hd}], got "
                             f"{tuple(key.shape)}/{tuple(value.shape)}")
        if key.dtype != torch.float16 or value.dtype != torch.float16:
            raise ValueError(f"{context} must be float16, got {key.dtype}/{value.dtype}")
        if key.device != hk.device or value.device != hv.device:
            raise ValueError(f"{context} must be on the hot window's device {hk.device}")
        count = key.shape[2]
        written = layer.hot_len - self._prompt_chunk_start[layer_idx]
        if written + count > self._prompt_chunk_len:
            raise RuntimeError(f"layer {layer_idx} holds {written} of the chunk's "
                               f"{self._prompt_chunk_len} tokens; {count} more do not fit")
        if hk.stride() != hv.stride() or hk.stride(-1) != 1:
            raise ValueError("hot_k and hot_v must share strides with a contiguous head_dim")
        if key.stride(-1) != 1:
            key = key.contiguous()
        if value.stride(-1) != 1:
            value = value.contiguous()
        _lib.check(_lib.load().pk_append_hot_rows(
            key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1), key.stride(2),
            value.stride(0), value.stride(1), value.stride(2), hk.data_ptr(), hv.data_ptr(),
            hk.stride(0), hk.stride(1), hk.stride(2), B, hkv, hd, layer.hot_len, count, cap,
            _lib.stream_ptr(hk.device)), "append_hot_rows")
        layer.hot_len += count

    @torch.no_grad()
    def finish_prompt_chunk(self) -> None:
        """Pack every chunk token with ``prompt_bits`` into a new prompt extension.

        The generated tokens that were in the window before the chunk stay there as
        FP16; their cooling is still decided by ``finish_decode_step``.
        """
        if not self._prompt_chunk_len:
            raise RuntimeError("no prompt chunk is open; call begin_prompt_chunk(length) first")
        for layer_idx, (layer, start) in enumerate(zip(self.layers, self._prompt_chunk_start)):
            written = layer.hot_len - start
            if written != self._prompt_chunk_len:
                raise RuntimeError(f"layer {layer_idx} holds {written} of the chunk's "
                                   f"{self._prompt_chunk_len} tokens")
        for layer, start in zip(self.layers, self._prompt_chunk_start):
            segment = pack_kv(layer.hot_k[:, :, start:layer.hot_len],
                              layer.hot_v[:, :, start:layer.hot_len],
                              self.prompt_bits, self.group_size)
            hot_k, hot_v = self._empty_hot(layer, self.recent_window + self.lazy_g)
            hot_k[:, :, :start].copy_(layer.hot_k[:, :, :start])
            hot_v[:, :, :start].copy_(layer.hot_v[:, :, :start])
            layer.prompt_extensions.append(segment)
            layer.hot_k, layer.hot_v = hot_k, hot_v
            layer.hot_len = start
        self._seen_tokens += self._prompt_chunk_len
        self._prompt_chunk_len = 0
        self._prompt_chunk_start = []

    # ---- beam reorder ---------------------------------------------------------
    @torch.no_grad()
    def reorder_cache(self, beam_idx: torch.Tensor) -> None:
        """Reorder the batch of every tier between steps (``phasekv_cache.py:454-478``)."""
        self._require_idle("reorder_cache()")
        if (not isinstance(beam_idx, torch.Tensor) or beam_idx.ndim != 1
                or beam_idx.dtype != torch.long or beam_idx.numel() == 0):
            raise ValueError("beam_idx must be a non-empty 1-D torch.long tensor")
        for layer_idx, layer in enumerate(self.layers):
            if bool((beam_idx < 0).any()) or bool((beam_idx >= layer.hot_k.shape[0]).any()):
                raise ValueError(f"beam_idx outside layer {layer_idx}'s batch range "
                                 f"[0, {layer.hot_k.shape[0]})")

        def select(t: torch.Tensor) -> torch.Tensor:
            index = beam_idx.to(t.device)
            base = t.transpose(-1, -2)
            if t.dim() >= 2 and not t.is_contiguous() and base.is_contiguous():
                # the transposed storage of per-channel K: reorder it and view it back
                return base.index_select(0, index).transpose(-1, -2)
            return t.index_select(0, index)

        def reorder(pt: PackedTensor) -> PackedTensor:
            return PackedTensor(packed=select(pt.packed), scale=select(pt.scale),
                                mins=select(pt.mins), bits=pt.bits, axis=pt.axis,
                                group_size=pt.group_size,
                                orig_shape=(beam_idx.numel(), *tuple(pt.orig_shape)[1:]),
                                axis_len=pt.axis_len)

        def reorder_segment(seg: PackedKVSegment) -> PackedKVSegment:
            return PackedKVSegment(reorder(seg.key), reorder(seg.value))

        for layer in self.layers:
            layer.prompt = reorder_segment(layer.prompt)
            layer.prompt_extensions = [reorder_segment(s) for s in layer.prompt_extensions]
            layer.cold = [reorder_segment(s) for s in layer.cold]
            layer.hot_k = layer.hot_k.index_select(0, beam_idx.to(layer.hot_k.device))
            layer.hot_v = layer.hot_v.index_select(0, beam_idx.to(layer.hot_v.device))
