"""Sub-byte packing and KIVI quantization on MI355X (drop-in for the reference's packing.py).

Same names, signatures, dataclass and error behaviour as
``src/phasekv/kernels/packing.py`` of the reference; the work runs in the HIP
kernels of ``libphasekv_hip.so`` (``pk_pack_low_bits``, ``pk_unpack_low_bits``,
``pk_quantize_pack``, ``pk_unpack_dequantize``).  Outputs are bit-identical to
the reference.  Tensors must be on a ROCm device: there is no CPU path.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import torch

from .. import _lib

_BITS_PER_BYTE = 8
_PACKABLE_BITS = (2, 4, 8)
#: Compact metadata bytes per quantization group (fp16 scale + fp16 min).
SCALE_MIN_BYTES = 4

_DTYPE_CODES = {
    torch.float16: _lib.PK_DTYPE_F16,
    torch.bfloat16: _lib.PK_DTYPE_BF16,
    torch.float32: _lib.PK_DTYPE_F32,
}


def _vals_per_byte(bits: int) -> int:
    """Codes per byte; ``packing.py:32-35``."""
    if bits not in _PACKABLE_BITS:
        raise ValueError(f"packable bit widths are {_PACKABLE_BITS}, got {bits}")
    return _BITS_PER_BYTE // bits


def pack_low_bits(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack uint8 codes in [0, 2**bits) along the last dim, LSB first (``packing.py:41-64``).

    Returns uint8 with last dim ``ceil(L / (8 // bits))``; tail codes padded with 0.
    """
    if codes.dtype != torch.uint8:
        raise ValueError(f"codes must be uint8, got {codes.dtype}")
    vpb = _vals_per_byte(bits)
    if bits == _BITS_PER_BYTE:
        return codes.contiguous()
    dev = _lib.require_device(codes)
    src = codes.contiguous()
    length = src.shape[-1] if src.dim() else 1
    n_bytes = -(-length // vpb)
    out = torch.empty(*src.shape[:-1], n_bytes, dtype=torch.uint8, device=dev)
    rows = src.numel() // length if length else 0
    if out.numel():
        lib = _lib.load()
        _lib.check(lib.pk_pack_low_bits(src.data_ptr(), rows, length, bits, out.data_ptr(),
                                        _lib.stream_ptr(dev)), "pack_low_bits")
    return out


def unpack_low_bits(packed: torch.Tensor, bits: int, length: int) -> torch.Tensor:
    """Inverse of ``pack_low_bits``: the first ``length`` codes (``packing.py:67-79``)."""
    if packed.dtype != torch.uint8:
        raise ValueError(f"packed must be uint8, got {packed.dtype}")
    vpb = _vals_per_byte(bits)
    if bits == _BITS_PER_BYTE:
        return packed[..., :length].contiguous()
    dev = _lib.require_device(packed)
    src = packed.contiguous()
    packed_len = src.shape[-1]
    length = min(int(length), packed_len * vpb)
    out = torch.empty(*src.shape[:-1], length, dtype=torch.uint8, device=dev)
    rows = src.numel() // packed_len if packed_len else 0
    if out.numel():
        lib = _lib.load()
        _lib.check(lib.pk_unpack_low_bits(src.data_ptr(), rows, packed_len, bits, length,
                                          out.data_ptr(), _lib.stream_ptr(dev)),
                   "unpack_low_bits")
    return out


@dataclass
class PackedTensor:
    """Low-bit packed K or V block as it lives in HBM (``packing.py:85-112``).

    packed     : uint8 codes, quantized axis moved last and packed.
    scale, mins: fp16 per-group parameters, shape ``[..., n_groups]`` (axis last).
    bits       : 2, 4 or 8.
    axis       : quantized axis of the original tensor (non-negative).
    group_size : group length (clipped to the axis length).
    orig_shape : shape of the original tensor.
    axis_len   : true length of the quantized axis.
    """

    packed: torch.Tensor
    scale: torch.Tensor
    mins: torch.Tensor
    bits: int
    axis: int
    group_size: int
    orig_shape: Tuple[int, ...]
    axis_len: int

    @property
    def nbytes(self) -> int:
        """Physical bytes: packed codes plus fp16 scale and min."""
        data = self.packed.numel()
        meta = self.scale.numel() + self.mins.numel()
        return int(data + meta * 2)


def quantize_pack(x: torch.Tensor, bits: int, axis: int, group_size: int) -> PackedTensor:
    """Grouped asymmetric min/max quantization along ``axis`` plus packing (``packing.py:115-155``).

    One HIP launch reads ``x`` in place through its strides (no transpose copy
    for the per-channel K layout) and writes the packed codes and fp16
    scale/min.  ``scale = max(max - min, 1e-8) / qmax`` and
    ``code = round_half_even((x - min) / scale)`` in IEEE float32, exactly as the
    reference.

    For ``axis == -2`` (the cache's per-channel K layout) ``packed``, ``scale`` and
    ``mins`` keep the reference's shapes ``[..., D, n_bytes]`` / ``[..., D, n_groups]``
    but are transposed views of ``[..., n_bytes, D]`` / ``[..., n_groups, D]``
    storage: a few consecutive tokens of every channel then sit together, which
    is how the decode kernels read them.  Values are identical; code that needs
    the reference's contiguous layout calls ``.contiguous()``.
    """
    if bits not in _PACKABLE_BITS:
        raise ValueError(f"bits must be one of {_PACKABLE_BITS}, got {bits}")
    dev = _lib.require_device(x)
    orig_shape = tuple(x.shape)
    if x.dim() == 0:
        raise ValueError("x must have at least one dimension")
    axis = axis % x.dim()
    length = orig_shape[axis]
    if length == 0:
        raise ValueError("the quantized axis must not be empty")
    gs = length if group_size is None or group_size <= 0 else min(group_size, length)
    if x.dtype not in _DTYPE_CODES:
        x = x.float()
    moved_prefix = tuple(s for i, s in enumerate(orig_shape) if i != axis)
    vpb = _BITS_PER_BYTE // bits
    n_bytes = -(-length // vpb)
    n_groups = -(-length // gs)
    group_major = x.dim() >= 2 and axis == x.dim() - 2
    if group_major:
        # [..., n_bytes, D] / [..., n_groups, D] storage seen as [..., D, n_bytes] / [..., D, n_groups]
        d_last = moved_prefix[-1]
        packed = torch.empty(*moved_prefix[:-1], n_bytes, d_last, dtype=torch.uint8,
                             device=dev).transpose(-1, -2)
        meta_shape = (*moved_prefix[:-1], n_groups, d_last)
        scale = torch.empty(*meta_shape, dtype=torch.float16, device=dev).transpose(-1, -2)
        mins = torch.empty(*meta_shape, dtype=torch.float16, device=dev).transpose(-1, -2)
    else:
        packed = torch.empty(*moved_prefix, n_bytes, dtype=torch.uint8, device=dev)
        scale = torch.empty(*moved_prefix, n_groups, dtype=torch.float16, device=dev)
        mins = torch.empty(*moved_prefix, n_groups, dtype=torch.float16, device=dev)
    if packed.numel():
        lib = _lib.load()
        shape = _lib.i64_array(orig_shape)
        strides = _lib.i64_array(x.stride())
        _lib.check(lib.pk_quantize_pack(x.data_ptr(), _DTYPE_CODES[x.dtype], x.dim(), shape,
                                        strides, axis, bits, gs, packed.data_ptr(),
                                        scale.data_ptr(), mins.data_ptr(),
                                        (_lib.PK_LAYOUT_META_TRANSPOSED
                                         | _lib.PK_LAYOUT_CODES_TRANSPOSED) if group_major else 0,
                                        _lib.stream_ptr(dev)), "quantize_pack")
    return PackedTensor(packed=packed, scale=scale, mins=mins, bits=bits, axis=axis,
                        group_size=gs, orig_shape=orig_shape, axis_len=length)


def unpack_dequantize(pt: PackedTensor) -> torch.Tensor:
    """Inverse of ``quantize_pack`` back to fp16 in the original layout (``packing.py:158-175``).

    ``code * scale + min`` as a float32 multiply then a float32 add, rounded to fp16.
    """
    _vals_per_byte(pt.bits)
    dev = _lib.require_device(pt.packed, pt.scale, pt.mins)
    out = torch.empty(pt.orig_shape, dtype=torch.float16, device=dev)
    if out.numel():
        packed = pt.packed.contiguous()
        scale = pt.scale.contiguous()
        mins = pt.mins.contiguous()
        lib = _lib.load()
        shape = _lib.i64_array(pt.orig_shape)
        _lib.check(lib.pk_unpack_dequantize(packed.data_ptr(), scale.data_ptr(), mins.data_ptr(),
                                            len(pt.orig_shape), shape, pt.axis, pt.bits,
                                            pt.group_size, pt.scale.shape[-1], out.data_ptr(),
                                            _lib.stream_ptr(dev)), "unpack_dequantize")
    return out
