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


def _ramp_tiers(gpu, g, hq, hkv, hd, length, kb, vb, v_range, big_q):
    """Scores that climb along the segment (so the running maximum keeps lagging the
    group maxima by up to the lazy bound) over V rows whose channel groups span
    ``v_range``.  With ``big_q``, q channel 5 is large and K channel 5 spans a range whose
    scale times that q is beyond fp16 in one group (tokens 320..351, which then holds the
    largest scores) and below it everywhere else."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    q = torch.randn(1, hq, hd, generator=g)
    k = torch.randn(1, hkv, length, hd, generator=g)
    # k . q grows along the tokens: a component along each head group's mean q direction
    dirs = q[0].view(hkv, hq // hkv, hd).mean(1)
    dirs = dirs / dirs.norm(dim=-1, keepdim=True)
    ramp = torch.linspace(0.0, 60.0, length)
    k += ramp[None, None, :, None] * dirs[None, :, None, :]
    if big_q:
        # (q, range of the special group, range elsewhere) per K width: q * scale is about
        # 3e5 (9e4 at 8 bits) in the special group and at most 5e4 elsewhere.  In the
        # special group token 330 alone takes the top code of channel 5, so it holds
        # the largest score by far (a well-conditioned one-hot softmax)
        qv, r_s, r_o = {2: (300.0, 3000.0, 500.0), 4: (300.0, 15000.0, 2500.0),
                        8: (2000.0, 12000.0, 1500.0)}[kb]
        q[..., 5] = qv
        u = torch.rand(1, hkv, length, generator=g) - 0.5
        k[..., 5] = u * r_o
        k[..., 320:352, 5] = (u[..., 320:352] - 0.5) * (r_s / 2)
        k[..., 321, 5] = -r_s / 2
        k[..., 330, 5] = r_s / 2
    v = torch.randn(1, hkv, length, hd, generator=g)
    v[..., ::3, :32] *= v_range / 6.0          # wide channel groups on every third token
    v = v.clamp(-65000.0, 65000.0)
    q, k, v = (x.to(torch.float16) for x in (q, k, v))
    pk = quantize_pack(k.to(gpu), kb, -2, 32)
    pv = quantize_pack(v.to(gpu), vb, -1, 32)
    # one chunk per head group: every wave runs many groups, so the lagging maximum
    # lets p reach the lazy bound
    return q, pk, pv, dec.packed_segment(pk, pv, batched=True, splits=1)


@pytest.mark.parametrize("kb,vb", [(2, 2), (2, 4), (4, 4), (2, 8), (8, 8)])
@pytest.mark.parametrize("case", ["wide_v", "big_q_times_k_scale"])
def test_wide_ranges_stay_finite(gpu, kb, vb, case):
    """Operands the MFMA path rounds to fp16 (q times the K scale, p times the V scale)
    must not overflow: V groups whose scale is far above 2^8 with the lagging softmax
    maximum, and a q channel times a K scale beyond 65504.  Against the oracle, which
    computes in float64, at the north-star tolerance applied to the data rescaled to unit
    range (the absolute bound scales with the largest |V|)."""
    print(f"case {case} bits={kb},{vb}", flush=True)
    g = torch.Generator().manual_seed(kb * 7 + vb)
    hq, hkv, hd, length = 8, 2, 128, 1400
    v_range = {2: 6000.0, 4: 40000.0, 8: 120000.0}[vb] if case == "wide_v" else 4.0
    q, pk, pv, seg = _ramp_tiers(gpu, g, hq, hkv, hd, length, kb, vb, v_range,
                                 case != "wide_v")
    deq_k = po.dequantize_float(_np_pt(pk))[0]
    deq_v = po.dequantize_float(_np_pt(pv))[0]
    want = ao.segments_attention(q[0].numpy(), [(deq_k, deq_v)], hq)
    assert np.isfinite(want).all()
    fast = _run(q.to(gpu), [seg], hq, False)[0].float().cpu().numpy()
    assert np.isfinite(fast).all(), "the MFMA path overflowed"
    scale = max(1.0, float(np.abs(deq_v).max()))
    np.testing.assert_allclose(fast, want, atol=2e-3 * scale, rtol=1e-2)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("kind,kb,vb", [("kivi", 2, 2), ("kivi", 2, 4), ("kivi", 4, 4),
                                        ("token", 2, 2), ("token", 4, 2), ("token", 4, 4)])
def test_eight_wave_workgroups(gpu, hd, kind, kb, vb):
    """Launches of at most one workgroup per CU with long chunks run eight waves per
    workgroup (two per SIMD): one chunk per row here, 8.5 groups per wave, ragged rows and a
    tail inside a group, against the four-wave kernel and the oracle."""
    import os
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case hd={hd} {kind} bits={kb},{vb}", flush=True)
    g = torch.Generator().manual_seed(hd + 7 * kb + vb + (50 if kind == "token" else 0))
    B, hq, hkv, S = 2, 28, 4, 2170
    q = torch.randn(B, hq, hd, generator=g).to(torch.float16)
    kd = torch.randn(B, hkv, S, hd, generator=g).to(torch.float16)
    vd = torch.randn(B, hkv, S, hd, generator=g).to(torch.float16)
    k_axis = -2 if kind == "kivi" else -1
    pk = quantize_pack(kd.to(gpu), kb, k_axis, 32)
    pv = quantize_pack(vd.to(gpu), vb, -1, 32)
    # ragged rows for per-token K only: a KIVI row cut inside a K group would need the
    # oracle to quantize that group over the tokens beyond the row's length as well
    lens = [S, 1517] if kind == "token" else [S, S]
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=gpu)
    seg = dec.packed_segment(pk, pv, batched=True, splits=1, seq_lens=seq_lens)
    outs = {}
    for w8 in ("1", "0"):
        os.environ["PK_WAVES8"] = w8
        try:
            outs[w8] = dec.fused_decode(dec.Problem(q.to(gpu), [seg], hq, require_mfma=True))
        finally:
            os.environ.pop("PK_WAVES8", None)
    torch.cuda.synchronize()
    for b, L in enumerate(lens):
        kq = po.quantize_pack(kd[b, :, :L].float().numpy(), kb, k_axis, 32)
        vq = po.quantize_pack(vd[b, :, :L].float().numpy(), vb, -1, 32)
        want = ao.merge_partials([ao.segment_partial(q[b].numpy(), kq, vq, hq)], out_dtype=None)
        for w8, out in outs.items():
            err = np.abs(out[b].float().cpu().numpy() - want).max()
            print(f"  row {b} waves8={w8} max abs err {err:.2e}", flush=True)
            np.testing.assert_allclose(out[b].float().cpu().numpy(), want, atol=2e-3, rtol=1e-2)
    np.testing.assert_allclose(outs["1"].float().cpu().numpy(), outs["0"].float().cpu().numpy(),
                               atol=1e-3, rtol=1e-2)
