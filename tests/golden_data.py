"""Loader of the committed golden vectors written by tests/golden/make_packing_golden.py."""
from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load():
    z = np.load(os.path.join(HERE, "packing_golden.npz"))
    with open(os.path.join(HERE, "packing_golden.json")) as f:
        manifest = json.load(f)
    return z, manifest


def input_as_float32(z, case) -> np.ndarray:
    """The case's input as float32 values (bf16 inputs are stored as raw bits)."""
    x = z[case["input"]]
    if case["dtype"] == "bfloat16":
        return (x.astype(np.uint16).astype(np.uint32) << 16).view(np.float32)
    return x.astype(np.float32) if x.dtype != np.float32 else x


def same_min_bits(a, b) -> bool:
    """Bitwise equality of two float16 min (or max) arrays, where +0.0 and -0.0 match.

    A group holding both signed zeros has a zero min whose sign IEEE comparison
    leaves open: torch's CPU reduction keeps the first element for short groups
    and follows its vector lanes for long ones (group size 32 gives +0.0 for a
    group that starts with -0.0).  The stored sign is invisible after
    dequantization (``code * scale + min`` with ``code * scale >= +0.0``), so the
    parity checks accept either sign there and stay bitwise everywhere else,
    NaN payloads included.
    """
    a16 = np.asarray(a).view(np.uint16)
    b16 = np.asarray(b).view(np.uint16)
    if a16.shape != b16.shape:
        return False
    zero = ((a16 & 0x7FFF) == 0) & ((b16 & 0x7FFF) == 0)
    return bool(np.all((a16 == b16) | zero))
