"""Pins the packing oracle: golden vectors of the reference, brute force, closed forms.

The oracle restates src/phasekv/kernels/packing.py; these checks do not retype
its formulas: the golden vectors come from the reference module itself, the
brute-force checks build bytes bit by bit, and the planted-mistake checks show
that each plausible slip (fp16 scale for codes, rounding mode, bit order,
a min/max that skips NaN) fails at least one golden vector.
"""
import numpy as np
import pytest

from oracle import packing_oracle as po
from tests import golden_data


@pytest.fixture(scope="module")
def golden():
    return golden_data.load()


def _quant_matches(pt, z, key):
    return (np.array_equal(pt.packed, z[key + "_packed"])
            and np.array_equal(pt.scale.view(np.uint16), z[key + "_scale"].view(np.uint16))
            and golden_data.same_min_bits(pt.mins, z[key + "_mins"]))


def test_oracle_quantize_matches_reference_golden(golden):
    z, man = golden
    assert len(man["quantize"]) >= 150
    for case in man["quantize"]:
        x = golden_data.input_as_float32(z, case)
        pt = po.quantize_pack(x, case["bits"], case["axis"], case["group_size"])
        assert pt.axis == case["out_axis"] and pt.group_size == case["out_group_size"]
        assert pt.axis_len == case["axis_len"] and list(pt.orig_shape) == case["orig_shape"]
        assert _quant_matches(pt, z, case["key"]), case
        deq = po.unpack_dequantize(pt)
        assert np.array_equal(deq.view(np.uint16), z[case["key"] + "_deq"].view(np.uint16)), case


def test_oracle_pack_matches_reference_golden(golden):
    z, man = golden
    for case in man["pack"]:
        k = case["key"]
        packed = po.pack_low_bits(z[k + "_codes"], case["bits"])
        assert np.array_equal(packed, z[k + "_packed"])
        assert np.array_equal(po.unpack_low_bits(packed, case["bits"], case["length"]),
                              z[k + "_unpacked"])


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_bit_by_bit_brute_force(bits):
    rng = np.random.default_rng(5)
    vpb = 8 // bits
    for length in range(1, 34):
        codes = rng.integers(0, 1 << bits, size=(3, length), dtype=np.uint8)
        packed = po.pack_low_bits(codes, bits)
        assert packed.shape == (3, -(-length // vpb))
        for r in range(3):
            for k in range(packed.shape[1]):
                want = 0
                for j in range(vpb):
                    pos = k * vpb + j
                    if pos < length:
                        for bit in range(bits):
                            if (int(codes[r, pos]) >> bit) & 1:
                                want |= 1 << (j * bits + bit)
                assert int(packed[r, k]) == want
        assert np.array_equal(po.unpack_low_bits(packed, bits, length), codes)


@pytest.mark.parametrize("bits", [2, 4])
def test_every_byte_value_round_trips(bits):
    vpb = 8 // bits
    allbytes = np.arange(256, dtype=np.uint8)[None, :]
    codes = po.unpack_low_bits(allbytes, bits, 256 * vpb)
    assert np.array_equal(po.pack_low_bits(codes, bits), allbytes)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_constant_group_closed_form(bits):
    qmax = (1 << bits) - 1
    x = np.full((2, 3, 40), 0.3125, np.float16)
    pt = po.quantize_pack(x, bits, -1, 32)
    assert np.all(po.unpack_low_bits(pt.packed, bits, 40) == 0)
    want_scale = np.float16(np.float32(1e-8) / np.float32(qmax))
    assert np.all(pt.scale == want_scale)
    assert np.all(pt.mins == np.float16(0.3125))
    assert np.array_equal(po.unpack_dequantize(pt), x)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_two_valued_group_codes_are_extremes(bits):
    qmax = (1 << bits) - 1
    x = np.where(np.arange(64) % 3 == 0, -1.5, 2.25).astype(np.float16)[None]
    pt = po.quantize_pack(x, bits, -1, 32)
    codes = po.unpack_low_bits(pt.packed, bits, 64)[0]
    assert np.array_equal(codes, np.where(np.arange(64) % 3 == 0, 0, qmax))


def test_exact_ties_round_half_to_even():
    # min 0, max 3, 2-bit: scale is exactly 1.0, so x = k + 1/2 is an exact tie
    x = np.array([[0.0, 0.5, 1.5, 2.5, 3.0, 1.0, 2.0, 0.5]], np.float16)
    pt = po.quantize_pack(x, 2, -1, 8)
    codes = po.unpack_low_bits(pt.packed, 2, 8)[0].tolist()
    assert codes == [0, 0, 2, 2, 3, 1, 2, 0]


def test_group_size_one_and_tail_groups():
    x = np.array([[1.0, -2.0, 3.5, 0.25, 7.0]], np.float16)
    pt = po.quantize_pack(x, 4, -1, 1)
    assert pt.scale.shape == (1, 5) and np.array_equal(pt.mins[0], x[0])
    assert np.array_equal(po.unpack_dequantize(pt), x)
    pt = po.quantize_pack(x, 2, -1, 2)     # groups [0,1], [2,3], tail [4]
    assert pt.scale.shape == (1, 3)
    assert pt.mins[0, 2] == np.float16(7.0)


# ---------------------------------------------------------------------------
# planted mistakes: each variant must fail at least one golden vector
# ---------------------------------------------------------------------------
def _mutant_quantize(x, bits, axis, group_size, mutation):
    qmax = (1 << bits) - 1
    axis = axis % x.ndim
    xf = np.ascontiguousarray(np.moveaxis(x.astype(np.float32), axis, -1))
    length = xf.shape[-1]
    gs = length if group_size is None or group_size <= 0 else min(group_size, length)
    pad = (-length) % gs
    if pad:
        xf = np.concatenate([xf, np.broadcast_to(xf[..., -1:], xf.shape[:-1] + (pad,))], -1)
    xg = xf.reshape(xf.shape[:-1] + (xf.shape[-1] // gs, gs))
    if mutation == "nan_skipping":
        with np.errstate(invalid="ignore"):
            mn = np.fmin.reduce(xg, axis=-1, keepdims=True)
            mx = np.fmax.reduce(xg, axis=-1, keepdims=True)
    else:
        mn = xg.min(-1, keepdims=True)
        mx = xg.max(-1, keepdims=True)
    scale = (np.maximum(mx - mn, np.float32(1e-8)) / np.float32(qmax)).astype(np.float32)
    use = scale
    if mutation == "fp16_scale":
        use = scale.astype(np.float16).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = (xg - mn) / use
    if mutation == "round_half_up":
        q = np.floor(q + np.float32(0.5))
    else:
        q = np.rint(q)
    with np.errstate(invalid="ignore"):
        codes = np.clip(np.nan_to_num(q), 0, qmax).astype(np.uint8).reshape(xf.shape)[..., :length]
    if mutation == "msb_first" and bits < 8:
        vpb = 8 // bits
        padn = (-length) % vpb
        c = np.concatenate([codes, np.zeros(codes.shape[:-1] + (padn,), np.uint8)], -1)
        c = c.reshape(c.shape[:-1] + (c.shape[-1] // vpb, vpb)).astype(np.int32)
        shifts = (vpb - 1 - np.arange(vpb)) * bits
        packed = (c << shifts).sum(-1).astype(np.uint8)
    else:
        packed = po.pack_low_bits(np.ascontiguousarray(codes), bits)
    return packed, scale[..., 0].astype(np.float16), mn[..., 0].astype(np.float16)


@pytest.mark.parametrize("mutation", ["fp16_scale", "round_half_up", "msb_first", "nan_skipping"])
def test_planted_quantize_mistakes_fail_golden(golden, mutation):
    z, man = golden
    failures = 0
    for case in man["quantize"]:
        x = golden_data.input_as_float32(z, case)
        packed, scale, mins = _mutant_quantize(x, case["bits"], case["axis"],
                                               case["group_size"], mutation)
        k = case["key"]
        if not (np.array_equal(packed, z[k + "_packed"])
                and np.array_equal(scale.view(np.uint16), z[k + "_scale"].view(np.uint16))
                and golden_data.same_min_bits(mins, z[k + "_mins"])):
            failures += 1
    assert failures > 0, f"golden vectors do not detect the '{mutation}' mistake"


def test_dequant_matches_exact_arithmetic():
    """unpack_dequantize == fp16(fp32(c*s + m)) computed exactly in float64.

    A code (<= 8 bits) times an fp16 scale (11 significant bits) is exact in
    float32, so the float32 multiply never rounds and only the add does: a
    fused multiply-add and packing.py:173's separate multiply then add give the
    same bits.  The float64 sum below is exact for these magnitudes.
    """
    rng = np.random.default_rng(3)
    n = 4096
    codes = rng.integers(0, 256, size=(n, 1)).astype(np.uint8)
    scale = rng.uniform(1e-4, 4.0, size=(n, 1)).astype(np.float16)
    mins = rng.uniform(-16.0, 16.0, size=(n, 1)).astype(np.float16)
    pt = po.PackedArrays(packed=po.pack_low_bits(codes, 8), scale=scale, mins=mins, bits=8,
                         axis=1, group_size=1, orig_shape=(n, 1), axis_len=1)
    got = po.unpack_dequantize(pt)
    exact = codes.astype(np.float64) * scale.astype(np.float64) + mins.astype(np.float64)
    want = exact.astype(np.float32).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
