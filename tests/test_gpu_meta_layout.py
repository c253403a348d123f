"""K code and scale/min storage: quantize_pack keeps the reference's shapes and values
for the per-channel K layout (axis -2) but stores the transposes; the decode kernels must
give bit-identical results for every mix of that storage and the reference's contiguous
layout."""
import dataclasses

import numpy as np
import pytest
import torch

from oracle import packing_oracle as po

pytestmark = pytest.mark.gpu


def _contiguous_meta(pt):
    return dataclasses.replace(pt, scale=pt.scale.contiguous(), mins=pt.mins.contiguous())


def _contiguous_codes(pt):
    return dataclasses.replace(pt, packed=pt.packed.contiguous())


def _layout_variants(pt):
    """(codes token major, meta group major) x both: the four storages of one K segment."""
    return {(1, 1): pt, (0, 1): _contiguous_codes(pt), (1, 0): _contiguous_meta(pt),
            (0, 0): _contiguous_codes(_contiguous_meta(pt))}


def test_quantize_pack_k_metadata_is_group_major_view_with_reference_values(gpu):
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(7)
    x = torch.randn(2, 3, 200, 64, generator=g).to(torch.float16)
    pt = quantize_pack(x.to(gpu), 2, -2, 32)
    want = po.quantize_pack(x.numpy(), 2, -2, 32)
    assert tuple(pt.scale.shape) == want.scale.shape == (2, 3, 64, 7)
    assert pt.scale.stride(-2) == 1 and pt.scale.stride(-1) == 64      # [.., groups, D] storage
    assert tuple(pt.packed.shape) == want.packed.shape == (2, 3, 64, 50)
    assert pt.packed.stride(-2) == 1 and pt.packed.stride(-1) == 64     # [.., bytes, D] storage
    np.testing.assert_array_equal(pt.scale.cpu().numpy(), want.scale)
    np.testing.assert_array_equal(pt.mins.cpu().numpy(), want.mins)
    np.testing.assert_array_equal(pt.packed.cpu().numpy(), want.packed)
    # V (per token along head_dim) keeps the contiguous layout
    pv = quantize_pack(x.to(gpu), 2, -1, 32)
    assert pv.scale.is_contiguous()


@pytest.mark.parametrize("generic", [False, True])
@pytest.mark.parametrize("lengths", [(4096, 256), (1000, 37), (384, 128, 33), (4000, 200, 96)])
def test_decode_identical_for_both_metadata_layouts(gpu, generic, lengths):
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case generic={generic} lengths={lengths}", flush=True)
    g = torch.Generator().manual_seed(sum(lengths))
    hq, hkv, hd = 28, 4, 128
    q = torch.randn(1, hq, hd, generator=g).to(torch.float16).to(gpu)
    segs = {key: [] for key in ((1, 1), (0, 1), (1, 0), (0, 0))}
    for i, length in enumerate(lengths):
        bits = (2, 4, 8)[i % 3]
        k = torch.randn(1, hkv, length, hd, generator=g).to(torch.float16).to(gpu)
        v = torch.randn(1, hkv, length, hd, generator=g).to(torch.float16).to(gpu)
        pk, pv = quantize_pack(k, bits, -2, 32), quantize_pack(v, bits, -1, 32)
        for key, variant in _layout_variants(pk).items():
            seg = dec.packed_segment(variant, pv, batched=True)
            assert (seg.desc.k_data_layout, seg.desc.k_meta_layout) == key
            segs[key].append(seg)
    ref = dec.fused_decode(dec.Problem(q, segs[(0, 0)], hq, generic_kernel=generic))
    pref = dec.decode_partials(dec.Problem(q, segs[(0, 0)], hq, generic_kernel=generic))
    for key in ((1, 1), (0, 1), (1, 0)):
        out = dec.fused_decode(dec.Problem(q, segs[key], hq, generic_kernel=generic))
        assert torch.equal(out, ref), key
        part = dec.decode_partials(dec.Problem(q, segs[key], hq, generic_kernel=generic))
        assert all(torch.equal(a, b) for a, b in zip(part, pref)), key


def test_ragged_batch_identical_for_both_metadata_layouts(gpu):
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(3)
    b, hq, hkv, hd, length = 3, 8, 2, 128, 1024
    q = torch.randn(b, hq, hd, generator=g).to(torch.float16).to(gpu)
    k = torch.randn(b, hkv, length, hd, generator=g).to(torch.float16).to(gpu)
    v = torch.randn(b, hkv, length, hd, generator=g).to(torch.float16).to(gpu)
    lens = torch.tensor([1024, 700, 129], dtype=torch.int32, device=gpu)
    pk, pv = quantize_pack(k, 2, -2, 32), quantize_pack(v, 2, -1, 32)
    outs = [dec.fused_decode(dec.Problem(q, [dec.packed_segment(variant, pv, batched=True,
                                                                seq_lens=lens)], hq))
            for variant in _layout_variants(pk).values()]
    assert all(torch.equal(o, outs[0]) for o in outs[1:])


def test_unpack_dequantize_reads_group_major_metadata(gpu):
    from phasekv_amd.kernels.packing import quantize_pack, unpack_dequantize
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, 2, 96, 128, generator=g).to(torch.float16)
    pt = quantize_pack(x.to(gpu), 4, -2, 32)
    want = po.unpack_dequantize(po.quantize_pack(x.numpy(), 4, -2, 32))
    np.testing.assert_array_equal(unpack_dequantize(pt).cpu().numpy(), want)
