"""Write golden input/output vectors for quantize_pack / unpack_dequantize / pack_low_bits.

Run in the build container only (it needs the reference checkout):

    python tests/golden/make_packing_golden.py /root/reference

It loads ``src/phasekv/kernels/packing.py`` of the reference by file path (that
module depends on torch and the standard library only), runs it on the CPU on
seeded and constructed inputs, and stores inputs and outputs as plain arrays in
``tests/golden/packing_golden.npz`` plus the case list in
``tests/golden/packing_golden.json``.  The fixture holds data only.
"""
from __future__ import annotations

import importlib.util
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference_packing(ref_root: str):
    path = os.path.join(ref_root, "src", "phasekv", "kernels", "packing.py")
    spec = importlib.util.spec_from_file_location("reference_packing_module", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod   # dataclasses look the module up by name
    spec.loader.exec_module(mod)
    return mod


def constructed_inputs():
    """Inputs whose quantization has a closed form or sits on a rounding edge."""
    cases = {}
    # Constant groups: scale = fp32(1e-8)/qmax, all codes 0, dequant == min.
    cases["constant"] = np.full((1, 2, 40, 8), 0.3125, np.float16)
    # Two-valued groups: codes are exactly {0, qmax}.
    tv = np.where(np.arange(40)[None, None, :, None] % 3 == 0, -1.5, 2.25) * np.ones((1, 2, 40, 8))
    cases["two_valued"] = tv.astype(np.float16)
    # Exact ties: values min + (k + 1/2) * (max-min)/qmax for 2-bit (qmax = 3).
    row = np.array([0.0, 0.5, 1.5, 2.5, 3.0, 1.0, 2.0, 0.5], np.float32)
    cases["ties"] = np.broadcast_to(row, (1, 2, 8, 8)).astype(np.float16).copy()
    # Many groups with small ranges (scale rounding to fp16 matters).
    g = torch.Generator().manual_seed(11)
    small = (torch.randn(1, 2, 33, 16, generator=g) * 1e-3 + 5.0).to(torch.float16)
    cases["narrow_range"] = small.numpy()
    # Heavy tails with outlier channels.
    heavy = torch.randn(1, 2, 48, 32, generator=g)
    heavy[..., 5] *= 40
    heavy[..., 17] *= -25
    cases["outliers"] = heavy.to(torch.float16).numpy()
    # IEEE specials: groups holding a NaN, +inf, -inf, both infinities, signed zeros only,
    # and a NaN beside an infinity, next to ordinary groups (how amin / amax, the scale's
    # clamp, round and the uint8 cast treat them fixes codes, scales and mins)
    sp = torch.randn(1, 2, 40, 8, generator=g)
    sp[0, 0, 3, 1] = float("nan")
    sp[0, 0, 12, 2] = float("inf")
    sp[0, 1, 20, 3] = float("-inf")
    sp[0, 1, 33, 4] = float("inf")
    sp[0, 1, 34, 4] = float("-inf")
    sp[0, 0, 32:40, 5] = 0.0
    sp[0, 0, 32:40:2, 5] = -0.0
    sp[0, 1, 6, 6] = float("nan")
    sp[0, 1, 7, 6] = float("inf")
    cases["specials"] = sp.to(torch.float16).numpy()
    return cases


def main(ref_root: str) -> None:
    ref = load_reference_packing(ref_root)
    arrays = {}
    manifest = {"quantize": [], "pack": []}

    gen = torch.Generator().manual_seed(1234)
    random_inputs = {
        "r_1x2x37x8": torch.randn(1, 2, 37, 8, generator=gen).to(torch.float16),
        "r_1x2x8x37": torch.randn(1, 2, 8, 37, generator=gen).to(torch.float16),
        "r_2x2x45x16": torch.randn(2, 2, 45, 16, generator=gen).to(torch.float16),
        "r_1x1x1x8": torch.randn(1, 1, 1, 8, generator=gen).to(torch.float16),
        "r_bf16_1x2x19x8": torch.randn(1, 2, 19, 8, generator=gen).to(torch.bfloat16),
        "r_f32_1x2x21x8": torch.randn(1, 2, 21, 8, generator=gen).to(torch.float32),
    }
    inputs = {k: v for k, v in random_inputs.items()}
    for name, arr in constructed_inputs().items():
        inputs["c_" + name] = torch.from_numpy(arr)

    idx = 0
    for name, x in inputs.items():
        if x.dtype == torch.bfloat16:
            arrays[f"x_{name}"] = x.view(torch.int16).numpy()   # raw bf16 bits
            dtype_name = "bfloat16"
        else:
            arrays[f"x_{name}"] = x.numpy()
            dtype_name = str(x.dtype).replace("torch.", "")
        for bits in (2, 4, 8):
            for axis in (-1, -2):
                for gs in (32, 4, 1, 5, 0):
                    if gs in (1, 5) and name not in ("r_1x2x37x8", "c_ties", "c_constant"):
                        continue
                    if gs == 0 and name not in ("r_1x2x8x37", "r_2x2x45x16"):
                        continue
                    pt = ref.quantize_pack(x, bits, axis, gs)
                    deq = ref.unpack_dequantize(pt)
                    key = f"q{idx}"
                    arrays[f"{key}_packed"] = pt.packed.numpy()
                    arrays[f"{key}_scale"] = pt.scale.numpy()
                    arrays[f"{key}_mins"] = pt.mins.numpy()
                    arrays[f"{key}_deq"] = deq.numpy()
                    manifest["quantize"].append({
                        "key": key, "input": f"x_{name}", "dtype": dtype_name,
                        "shape": list(x.shape), "bits": bits, "axis": axis, "group_size": gs,
                        "out_axis": pt.axis, "out_group_size": pt.group_size,
                        "axis_len": pt.axis_len, "orig_shape": list(pt.orig_shape),
                    })
                    idx += 1

    gen = torch.Generator().manual_seed(99)
    pidx = 0
    for bits in (2, 4, 8):
        for length in (1, 2, 3, 4, 5, 7, 8, 9, 31, 32, 33):
            codes = torch.randint(0, 1 << bits, (3, length), generator=gen, dtype=torch.int64)
            codes = codes.to(torch.uint8)
            packed = ref.pack_low_bits(codes, bits)
            unpacked = ref.unpack_low_bits(packed, bits, length)
            key = f"p{pidx}"
            arrays[f"{key}_codes"] = codes.numpy()
            arrays[f"{key}_packed"] = packed.numpy()
            arrays[f"{key}_unpacked"] = unpacked.numpy()
            manifest["pack"].append({"key": key, "bits": bits, "length": length})
            pidx += 1

    np.savez_compressed(os.path.join(HERE, "packing_golden.npz"), **arrays)
    with open(os.path.join(HERE, "packing_golden.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print(f"wrote {idx} quantize cases and {pidx} pack cases")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
