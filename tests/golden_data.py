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
