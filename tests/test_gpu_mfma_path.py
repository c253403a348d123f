"""The MFMA decode kernel against the generic kernel and the oracle, over every K/V bit
width pair, head_dim 64 / 128, GQA group sizes, head slabs, ragged batches and tails."""
import numpy as np
import pytest
import torch

from oracle import attention_oracle as ao
from oracle import packing_oracle as po

pytestmark = pytest.mark.gpu


def _np_pt(pt):
    return po.PackedArrays(pt.packed.cpu().numpy(), pt.scale.cpu().numpy(), pt.mins.cpu().numpy(),
                           pt.bits, pt.axis, pt.group_size, tuple(pt.orig_shape), pt.axis_len)


def _run(q, segs, hq, generic):
    from phasekv_amd import decode as dec
    return dec.fused_decode(dec.Problem(q, segs, hq, generic_kernel=generic))


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("kb,vb", [(2, 2), (2, 4), (2, 8), (4, 2), (4, 4), (4, 8), (8, 2),
                                   (8, 4), (8, 8)])
def test_mfma_matches_generic_and_oracle(gpu, hd, kb, vb):
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case hd={hd} bits={kb},{vb}", flush=True)
    g = torch.Generator().manual_seed(kb * 10 + vb + hd)
    hq, hkv = 28, 4
    q = torch.randn(1, hq, hd, generator=g).to(torch.float16)
    parts, segs = [], []
    for length in (700, 64, 33, 5):          # tails inside a tile, one group, tiny segments
        kd = (torch.randn(1, hkv, length, hd, generator=g) * 2).to(torch.float16)
        vd = torch.randn(1, hkv, length, hd, generator=g).to(torch.float16)
        pk = quantize_pack(kd.to(gpu), kb, -2, 32)
        pv = quantize_pack(vd.to(gpu), vb, -1, 32)
        segs.append(dec.packed_segment(pk, pv, batched=True))
        strip = lambda pt: po.PackedArrays(*(x[0] for x in (pt.packed.cpu().numpy(),
                                             pt.scale.cpu().numpy(), pt.mins.cpu().numpy())),
                                           pt.bits, pt.axis - 1, pt.group_size,
                                           tuple(pt.orig_shape[1:]), pt.axis_len)
        parts.append(ao.segment_partial(q[0].numpy(), strip(pk), strip(pv), hq))
    hk = torch.randn(1, hkv, 40, hd, generator=g).to(torch.float16)
    hv = torch.randn(1, hkv, 40, hd, generator=g).to(torch.float16)
    segs.append(dec.fp16_segment(hk.to(gpu), hv.to(gpu), batched=True))
    parts.append(ao.fp16_layer_partial(q[0].numpy(), hk[0].numpy(), hv[0].numpy(), hq))
    want = ao.merge_partials(parts, out_dtype=None)
    fast = _run(q.to(gpu), segs, hq, False)[0].float().cpu().numpy()
    slow = _run(q.to(gpu), segs, hq, True)[0].float().cpu().numpy()
    np.testing.assert_allclose(fast, want, atol=2e-3, rtol=1e-2)
    np.testing.assert_allclose(slow, want, atol=2e-3, rtol=1e-2)
    np.testing.assert_allclose(fast, slow, atol=1e-3, rtol=1e-2)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("kb,vb", [(2, 2), (2, 4), (2, 8), (4, 2), (4, 4), (4, 8), (8, 2),
                                   (8, 4), (8, 8)])
def test_mfma_whole_segment_in_one_chunk(gpu, hd, kb, vb):
    """One chunk per head group: a workgroup runs all 12 stages of the segment through
    both LDS stage buffers (prologue, steady loop, tail, ragged last stage).  The launch
    holds only this width pair, so its stage buffers are sized for exactly this layout."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case hd={hd} bits={kb},{vb}", flush=True)
    g = torch.Generator().manual_seed(kb * 100 + vb + hd)
    hq, hkv, length = 8, 2, 1500
    q = torch.randn(1, hq, hd, generator=g).to(torch.float16)
    kd = (torch.randn(1, hkv, length, hd, generator=g) * 2).to(torch.float16)
    vd = torch.randn(1, hkv, length, hd, generator=g).to(torch.float16)
    pk = quantize_pack(kd.to(gpu), kb, -2, 32)
    pv = quantize_pack(vd.to(gpu), vb, -1, 32)
    seg = dec.packed_segment(pk, pv, batched=True, splits=1)
    fast = _run(q.to(gpu), [seg], hq, False)[0].float().cpu().numpy()
    slow = _run(q.to(gpu), [seg], hq, True)[0].float().cpu().numpy()
    deq_k = po.dequantize_float(_np_pt(pk))[0]
    deq_v = po.dequantize_float(_np_pt(pv))[0]
    want = ao.segments_attention(q[0].numpy(), [(deq_k, deq_v)], hq)
    np.testing.assert_allclose(fast, want, atol=2e-3, rtol=1e-2)
    np.testing.assert_allclose(fast, slow, atol=1e-3, rtol=1e-2)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (16, 1), (28, 4), (32, 1), (40, 2)])
def test_mfma_gqa_groups_and_head_slabs(gpu, hq, hkv):
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(hq + hkv)
    hd, b, length = 128, 2, 1000
    q = torch.randn(b, hq, hd, generator=g).to(torch.float16)
    kd = torch.randn(b, hkv, length, hd, generator=g).to(torch.float16)
    vd = torch.randn(b, hkv, length, hd, generator=g).to(torch.float16)
    pk = quantize_pack(kd.to(gpu), 2, -2, 32)
    pv = quantize_pack(vd.to(gpu), 2, -1, 32)
    lens = torch.tensor([1000, 613], dtype=torch.int32, device=gpu)
    seg = dec.packed_segment(pk, pv, batched=True, seq_lens=lens)
    fast = _run(q.to(gpu), [seg], hq, False).float().cpu().numpy()
    slow = _run(q.to(gpu), [seg], hq, True).float().cpu().numpy()
    np.testing.assert_allclose(fast, slow, atol=1e-3, rtol=1e-2)
    # row 1 stops at 613 valid tokens: compare with the oracle on the truncated row
    pkn, pvn = _np_pt(pk), _np_pt(pv)
    deq_k = po.dequantize_float(pkn)[1, :, :613]
    deq_v = po.dequantize_float(pvn)[1, :, :613]
    want = ao.segments_attention(q[1].numpy(), [(deq_k, deq_v)], hq)
    np.testing.assert_allclose(fast[1], want, atol=2e-3, rtol=1e-2)


def test_mfma_fp16_dense_long(gpu):
    from phasekv_amd.kernels.attention_triton import dense_fp16_decode
    g = torch.Generator().manual_seed(3)
    hq, hkv, hd, s = 28, 4, 128, 5000
    q = torch.randn(hq, hd, generator=g).to(torch.float16)
    k = torch.randn(hkv, s, hd, generator=g).to(torch.float16)
    v = torch.randn(hkv, s, hd, generator=g).to(torch.float16)
    out = dense_fp16_decode(q.to(gpu), k.to(gpu), v.to(gpu), hq).float().cpu().numpy()
    want = ao.segments_attention(q.numpy(), [(k.numpy(), v.numpy())], hq)
    np.testing.assert_allclose(out, want, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("length", [896, 1024, 1056, 1100, 1184, 1311, 1408])
def test_mfma_long_wave_runs(gpu, hd, length):
    """One chunk per head group of a 2/2-bit segment: every wave runs 7 to 11 groups, so
    the waves take the pipelined group loop (8 or more groups) or the one-group-at-a-time
    loop, with full and ragged last groups on either side of the steady-loop bounds."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case hd={hd} length={length}", flush=True)
    g = torch.Generator().manual_seed(length + hd)
    hq, hkv = 8, 2
    q = torch.randn(1, hq, hd, generator=g).to(torch.float16)
    kd = (torch.randn(1, hkv, length, hd, generator=g) * 2).to(torch.float16)
    vd = torch.randn(1, hkv, length, hd, generator=g).to(torch.float16)
    pk = quantize_pack(kd.to(gpu), 2, -2, 32)
    pv = quantize_pack(vd.to(gpu), 2, -1, 32)
    seg = dec.packed_segment(pk, pv, batched=True, splits=1)
    fast = _run(q.to(gpu), [seg], hq, False)[0].float().cpu().numpy()
    slow = _run(q.to(gpu), [seg], hq, True)[0].float().cpu().numpy()
    deq_k = po.dequantize_float(_np_pt(pk))[0]
    deq_v = po.dequantize_float(_np_pt(pv))[0]
    want = ao.segments_attention(q[0].numpy(), [(deq_k, deq_v)], hq)
    np.testing.assert_allclose(fast, want, atol=2e-3, rtol=1e-2)
    np.testing.assert_allclose(fast, slow, atol=1e-3, rtol=1e-2)
