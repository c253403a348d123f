"""HIP pack / unpack / quantize / dequantize vs the oracle: bit-exact."""
import numpy as np
import pytest
import torch

from oracle import packing_oracle as po
from tests import golden_data

pytestmark = pytest.mark.gpu


def _to_torch(x_np, case, device):
    if case["dtype"] == "bfloat16":
        return torch.from_numpy(x_np.astype(np.int16)).view(torch.bfloat16).to(device)
    return torch.from_numpy(x_np).to(device)


def _u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def test_golden_vectors_through_hip(gpu):
    from phasekv_amd.kernels import packing
    z, man = golden_data.load()
    for case in man["quantize"]:
        x = _to_torch(z[case["input"]], case, gpu)
        pt = packing.quantize_pack(x, case["bits"], case["axis"], case["group_size"])
        k = case["key"]
        assert pt.axis == case["out_axis"] and pt.group_size == case["out_group_size"], case
        assert np.array_equal(pt.packed.cpu().numpy(), z[k + "_packed"]), case
        assert np.array_equal(_u16(pt.scale), z[k + "_scale"].view(np.int16)), case
        assert golden_data.same_min_bits(pt.mins.cpu().numpy(), z[k + "_mins"]), case
        deq = packing.unpack_dequantize(pt)
        assert np.array_equal(_u16(deq), z[k + "_deq"].view(np.int16)), case
    for case in man["pack"]:
        k = case["key"]
        codes = torch.from_numpy(z[k + "_codes"]).to(gpu)
        packed = packing.pack_low_bits(codes, case["bits"])
        assert np.array_equal(packed.cpu().numpy(), z[k + "_packed"])
        un = packing.unpack_low_bits(packed, case["bits"], case["length"])
        assert np.array_equal(un.cpu().numpy(), z[k + "_unpacked"])


@pytest.mark.parametrize("shape,axis,gs", [
    ((2, 3, 97, 16), -2, 32), ((2, 3, 97, 16), -1, 32), ((1, 4, 64, 128), -2, 32),
    ((1, 4, 64, 128), -1, 32), ((3, 5, 7), 0, 2), ((1, 2, 33, 8), -2, 5), ((1, 2, 8, 33), -1, 7),
    ((4, 1, 1, 8), -2, 1), ((1, 1, 300), -1, 1000),
])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_random_shapes_bit_exact(gpu, shape, axis, gs, bits):
    from phasekv_amd.kernels import packing
    g = torch.Generator().manual_seed(hash((shape, axis, gs, bits)) % 10000)
    x = (torch.randn(*shape, generator=g) * 3).to(torch.float16)
    pt = packing.quantize_pack(x.to(gpu), bits, axis, gs)
    ref = po.quantize_pack(x.numpy(), bits, axis, gs)
    assert pt.group_size == ref.group_size and pt.axis == ref.axis
    assert np.array_equal(pt.packed.cpu().numpy(), ref.packed)
    assert np.array_equal(_u16(pt.scale), ref.scale.view(np.int16))
    assert np.array_equal(_u16(pt.mins), ref.mins.view(np.int16))
    assert np.array_equal(_u16(packing.unpack_dequantize(pt)),
                          po.unpack_dequantize(ref).view(np.int16))


def test_strided_input_is_read_in_place(gpu):
    from phasekv_amd.kernels import packing
    g = torch.Generator().manual_seed(7)
    base = torch.randn(2, 64, 3, 40, generator=g).to(torch.float16)
    x = base.permute(0, 2, 1, 3)[:, :, 5:50]          # [2, 3, 45, 40] non-contiguous
    xd = base.to(gpu).permute(0, 2, 1, 3)[:, :, 5:50]
    assert not xd.is_contiguous()
    for axis in (-1, -2):
        pt = packing.quantize_pack(xd, 4, axis, 32)
        ref = po.quantize_pack(x.contiguous().numpy(), 4, axis, 32)
        assert np.array_equal(pt.packed.cpu().numpy(), ref.packed)
        assert np.array_equal(_u16(pt.scale), ref.scale.view(np.int16))


def test_bf16_and_fp32_inputs(gpu):
    from phasekv_amd.kernels import packing
    g = torch.Generator().manual_seed(9)
    x32 = torch.randn(1, 2, 70, 16, generator=g)
    for x in (x32, x32.to(torch.bfloat16)):
        pt = packing.quantize_pack(x.to(gpu), 2, -2, 32)
        ref = po.quantize_pack(x.float().numpy(), 2, -2, 32)
        assert np.array_equal(pt.packed.cpu().numpy(), ref.packed)
        assert np.array_equal(_u16(pt.scale), ref.scale.view(np.int16))


def test_prefill_pack_block_full_size(gpu):
    """C4 prefill: an 8192 x 4 x 128 fp16 K/V block packed to 2 bits, bit-exact."""
    from phasekv_amd.kernels import packing
    g = torch.Generator().manual_seed(1234)
    k = torch.randn(1, 4, 8192, 128, generator=g).to(torch.float16)
    v = torch.randn(1, 4, 8192, 128, generator=g).to(torch.float16)
    kd, vd = k.to(gpu), v.to(gpu)
    pk = packing.quantize_pack(kd, 2, -2, 32)
    pv = packing.quantize_pack(vd, 2, -1, 32)
    rk = po.quantize_pack(k.numpy(), 2, -2, 32)
    rv = po.quantize_pack(v.numpy(), 2, -1, 32)
    assert tuple(pk.packed.shape) == (1, 4, 128, 2048) and tuple(pv.packed.shape) == (1, 4, 8192, 32)
    for pt, ref in ((pk, rk), (pv, rv)):
        assert np.array_equal(pt.packed.cpu().numpy(), ref.packed)
        assert np.array_equal(_u16(pt.scale), ref.scale.view(np.int16))
        assert np.array_equal(_u16(pt.mins), ref.mins.view(np.int16))
    # size-independent property: unpack(pack(codes)) == codes
    codes = packing.unpack_low_bits(pk.packed, 2, 8192)
    assert torch.equal(packing.pack_low_bits(codes, 2), pk.packed)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_fast_path_rounding_ties_bit_exact(gpu, bits):
    """Rounding ties in the fp16 group-of-32 kernels: groups whose values sit exactly on
    k + 1/2 scales (scale 1 and 0.5 with half-integer values at several offsets, fp16
    values spaced 1/64 apart over random ranges) round half to even exactly as the
    reference's round() does."""
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(bits)
    qmax = (1 << bits) - 1
    rows = []
    for step in (1.0, 0.5):
        # min = offset, max = offset + qmax * step: scale = step, and values
        # offset + (k + 1/2) * step are exact ties (offset 0 takes the exact
        # statistics path, the others the fast one)
        grid = torch.arange(0, 2 * qmax + 1, dtype=torch.float32) * (step / 2)
        for offset in (0.0, 4.0, -8.0, 64.0):
            for _ in range(16):
                vals = grid[torch.randint(0, grid.numel(), (32,), generator=g)]
                vals[0], vals[1] = 0.0, qmax * step
                rows.append(vals + offset)
    for _ in range(128):
        lo = float(torch.randint(-64, 64, (1,), generator=g)) / 8
        span = float(torch.randint(1, 512, (1,), generator=g)) / 64
        vals = lo + torch.randint(0, int(span * 64) + 1, (32,), generator=g).float() / 64
        rows.append(vals)
    x = torch.stack(rows).to(torch.float16)                       # [R, 32] groups
    n = x.shape[0] // 4 * 4
    block = x[:n].reshape(1, n // 4, 4, 32).permute(0, 2, 1, 3).reshape(1, 4, n // 4 * 32 // 32, 32)
    for axis, data in ((-1, x[:n].reshape(1, 4, n // 4, 32)),           # V: groups along head_dim
                       (-2, block.transpose(-1, -2).contiguous())):    # K: groups along tokens
        pt = quantize_pack(data.to(gpu), bits, axis, 32)
        ref = po.quantize_pack(data.numpy(), bits, axis, 32)
        assert np.array_equal(pt.packed.cpu().numpy(), ref.packed), axis
        assert np.array_equal(_u16(pt.scale), ref.scale.view(np.int16)), axis
        assert np.array_equal(_u16(pt.mins), ref.mins.view(np.int16)), axis


def test_errors_are_value_errors(gpu):
    from phasekv_amd.kernels import packing
    x = torch.zeros(1, 2, 8, 8, dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError):
        packing.quantize_pack(x, 3, -1, 4)
    with pytest.raises(ValueError):
        packing.quantize_pack(x[:, :, :0], 2, -2, 4)
    with pytest.raises(ValueError):
        packing.unpack_low_bits(torch.zeros(4, dtype=torch.int32, device=gpu), 2, 4)


@pytest.mark.parametrize("shape,bits", [((1, 4, 8192, 128), 2), ((2, 3, 64, 64), 4),
                                        ((1, 2, 96, 128), 8), ((3, 1, 32, 32), 2)])
def test_pack_kv_one_launch_matches_two_quantize_packs(gpu, shape, bits):
    """``pack_kv``'s one-launch path (``pk_quantize_pack_kv``) gives the tensors, views,
    fields and bits of ``quantize_pack(K, axis=-2)`` and ``quantize_pack(V, axis=-1)``,
    with signed zeros, infinities and NaNs among the inputs."""
    from phasekv_amd.kernels.packing import quantize_pack
    from phasekv_amd.tiers import _one_launch, pack_kv
    print(f"case shape={shape} bits={bits}", flush=True)
    g = torch.Generator().manual_seed(sum(shape) + bits)
    k = torch.randn(*shape, generator=g) * 3
    v = torch.randn(*shape, generator=g)
    flat = k.view(-1)
    idx = torch.randint(0, flat.numel(), (64,), generator=g)
    flat[idx[:16]] = 0.0
    flat[idx[16:32]] = -0.0
    flat[idx[32:40]] = float("inf")
    flat[idx[40:44]] = float("nan")
    v.view(-1)[idx[44:60] % v.numel()] = -0.0
    k, v = k.to(torch.float16).to(gpu), v.to(torch.float16).to(gpu)
    assert _one_launch(k, v, bits, 32)
    got = pack_kv(k, v, bits, 32)
    want_k, want_v = quantize_pack(k, bits, axis=-2, group_size=32), \
        quantize_pack(v, bits, axis=-1, group_size=32)
    for a, b in ((got.key, want_k), (got.value, want_v)):
        assert (a.bits, a.axis, a.group_size, tuple(a.orig_shape), a.axis_len) == \
            (b.bits, b.axis, b.group_size, tuple(b.orig_shape), b.axis_len)
        for x, y in ((a.packed, b.packed), (a.scale, b.scale), (a.mins, b.mins)):
            assert x.shape == y.shape and x.stride() == y.stride()
            assert torch.equal(x.contiguous().flatten().view(torch.uint8),
                               y.contiguous().flatten().view(torch.uint8))
