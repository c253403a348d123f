"""numpy restatement of the reference's sub-byte packing and KIVI quantization.

Test infrastructure only (see ``oracle/__init__.py``).

Every operation is done in IEEE float32 in the same order as the reference, so
the outputs are expected to be bit-identical to ``packing.py`` run by torch on
the CPU:

* ``pack_low_bits``     follows ``src/phasekv/kernels/packing.py:41-64``
* ``unpack_low_bits``   follows ``src/phasekv/kernels/packing.py:67-79``
* ``quantize_pack``     follows ``src/phasekv/kernels/packing.py:115-155``
* ``unpack_dequantize`` follows ``src/phasekv/kernels/packing.py:158-175``
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import numpy as np

BITS_PER_BYTE = 8
PACKABLE_BITS = (2, 4, 8)
SCALE_MIN_BYTES = 4


def vals_per_byte(bits: int) -> int:
    """Codes per byte (``packing.py:32-35``)."""
    if bits not in PACKABLE_BITS:
        raise ValueError(f"bits must be one of {PACKABLE_BITS}, got {bits}")
    return BITS_PER_BYTE // bits


def pack_low_bits(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack along the last axis, code j of byte k at bits [j*b, (j+1)*b) (LSB first).

    Tail codes that do not fill a byte are padded with zero codes
    (``packing.py:56-64``); 8-bit is a pass-through (``packing.py:54-55``).
    """
    if codes.dtype != np.uint8:
        raise ValueError("codes must be uint8")
    vpb = vals_per_byte(bits)
    if bits == 8:
        return np.ascontiguousarray(codes)
    length = codes.shape[-1]
    pad = (-length) % vpb
    if pad:
        codes = np.concatenate(
            [codes, np.zeros(codes.shape[:-1] + (pad,), np.uint8)], axis=-1)
    grouped = codes.reshape(codes.shape[:-1] + (codes.shape[-1] // vpb, vpb)).astype(np.int32)
    shifts = np.arange(vpb, dtype=np.int32) * bits
    return (grouped << shifts).sum(axis=-1).astype(np.uint8)


def unpack_low_bits(packed: np.ndarray, bits: int, length: int) -> np.ndarray:
    """Inverse of ``pack_low_bits``, truncated to ``length`` codes (``packing.py:67-79``)."""
    if packed.dtype != np.uint8:
        raise ValueError("packed must be uint8")
    vpb = vals_per_byte(bits)
    if bits == 8:
        return np.ascontiguousarray(packed[..., :length])
    mask = (1 << bits) - 1
    p = packed.astype(np.int32)[..., None]
    shifts = np.arange(vpb, dtype=np.int32) * bits
    vals = (p >> shifts) & mask
    vals = vals.reshape(packed.shape[:-1] + (packed.shape[-1] * vpb,))
    return np.ascontiguousarray(vals[..., :length].astype(np.uint8))


@dataclass
class PackedArrays:
    """Host mirror of ``PackedTensor`` (``packing.py:85-112``)."""

    packed: np.ndarray   # uint8, quantized axis moved last, packed
    scale: np.ndarray    # float16, [..., n_groups]
    mins: np.ndarray     # float16, [..., n_groups]
    bits: int
    axis: int
    group_size: int
    orig_shape: Tuple[int, ...]
    axis_len: int

    @property
    def nbytes(self) -> int:
        return int(self.packed.size + 2 * (self.scale.size + self.mins.size))


def _group_min_max(xg: np.ndarray):
    """Per-group ``amin`` / ``amax`` over the last axis (``packing.py:141-142``).

    A left-to-right fold that takes the new element only when it compares
    strictly smaller (larger) or is NaN.  This fixes the two results IEEE
    comparison leaves open: a NaN anywhere gives NaN, and among equal values the
    first one is kept, which decides the sign of a zero min/max when a group
    holds both +0.0 and -0.0 (torch's CPU reduction over groups this short keeps
    the first as well).
    """
    mn = xg[..., 0:1].copy()
    mx = mn.copy()
    for i in range(1, xg.shape[-1]):
        v = xg[..., i:i + 1]
        nan = np.isnan(v)
        mn = np.where((v < mn) | nan, v, mn)
        mx = np.where((v > mx) | nan, v, mx)
    return mn, mx


def quantize_pack(x: np.ndarray, bits: int, axis: int, group_size) -> PackedArrays:
    """Grouped asymmetric min/max quantization along ``axis`` (``packing.py:115-155``).

    Steps, all in float32: move ``axis`` last; replicate-pad the tail to a
    multiple of ``gs = min(group_size, len)``; per group ``min``/``max``;
    ``scale = max(max - min, 1e-8) / qmax``; ``code = clip(rint((x - min) /
    scale), 0, qmax)`` (round half to even); drop the padded codes; pack; store
    the float32 scale and min rounded to float16.
    """
    if bits not in PACKABLE_BITS:
        raise ValueError(f"bits must be one of {PACKABLE_BITS}, got {bits}")
    qmax = (1 << bits) - 1
    orig_shape = tuple(x.shape)
    axis = axis % x.ndim
    xf = np.ascontiguousarray(np.moveaxis(x.astype(np.float32), axis, -1))
    moved_shape = xf.shape
    length = moved_shape[-1]
    gs = length if group_size is None or group_size <= 0 else min(group_size, length)
    pad = (-length) % gs
    if pad:
        tail = np.broadcast_to(xf[..., -1:], xf.shape[:-1] + (pad,))
        xf = np.concatenate([xf, tail], axis=-1)
    padded = xf.shape[-1]
    n_groups = padded // gs
    xg = xf.reshape(xf.shape[:-1] + (n_groups, gs))
    g_min, g_max = _group_min_max(xg)
    scale = np.maximum(g_max - g_min, np.float32(1e-8)).astype(np.float32) / np.float32(qmax)
    scale = scale.astype(np.float32)
    q = np.rint((xg - g_min) / scale).astype(np.float32)
    codes_g = np.clip(q, 0, qmax).astype(np.uint8)
    codes = np.ascontiguousarray(codes_g.reshape(moved_shape[:-1] + (padded,))[..., :length])
    return PackedArrays(
        packed=pack_low_bits(codes, bits),
        scale=scale[..., 0].astype(np.float16),
        mins=g_min[..., 0].astype(np.float16),
        bits=bits, axis=axis, group_size=gs, orig_shape=orig_shape, axis_len=length,
    )


def unpack_dequantize(pt: PackedArrays) -> np.ndarray:
    """``codes * scale + min`` in float32 (separate multiply and add), then float16.

    Follows ``packing.py:158-175``: the codes are zero-padded to whole groups,
    dequantized, truncated to ``axis_len`` and the axis is moved back.
    """
    gs = pt.group_size
    n_groups = pt.scale.shape[-1]
    padded = n_groups * gs
    codes = unpack_low_bits(pt.packed, pt.bits, pt.axis_len).astype(np.float32)
    if pt.axis_len < padded:
        codes = np.concatenate(
            [codes, np.zeros(codes.shape[:-1] + (padded - pt.axis_len,), np.float32)], axis=-1)
    prefix = codes.shape[:-1]
    codes_g = codes.reshape(prefix + (n_groups, gs))
    scale = pt.scale.astype(np.float32)[..., None]
    mins = pt.mins.astype(np.float32)[..., None]
    prod = (codes_g * scale).astype(np.float32)
    deq = (prod + mins).astype(np.float32).reshape(prefix + (padded,))[..., :pt.axis_len]
    deq = np.moveaxis(deq, -1, pt.axis)
    return np.ascontiguousarray(deq.astype(np.float16))


def dequantize_float(pt: PackedArrays) -> np.ndarray:
    """float32 dequantization without the final float16 rounding.

    This is the ``dense_float`` helper of the reference's CUDA test
    (``tests/test_phasekv_launch_config.py:57-61``): codes times the float16
    scale plus the float16 min, kept in float32.
    """
    codes = unpack_low_bits(pt.packed, pt.bits, pt.axis_len).astype(np.float32)
    groups = np.arange(pt.axis_len) // pt.group_size
    out = codes * pt.scale.astype(np.float32)[..., groups] + pt.mins.astype(np.float32)[..., groups]
    return np.moveaxis(out, -1, pt.axis)
