"""The MFMA kernel on per-token K segments (the reference's legacy layout,
src/phasekv/kernels/attention_triton.py:145-282): against the generic kernel and the
oracle over every K/V bit width pair, head_dim 64 / 128, GQA groups and head slabs,
ragged batches, the reference's split counts, three tiers, and the published shapes
(Hq 28, Hkv 4, hd 128, S up to 32K, scripts/bench_decode_kernel.py:66-130).

Every fast-path call passes require_mfma, so a silent fall to the generic kernel
fails the test instead of passing on it.
"""
import numpy as np
import pytest
import torch

from oracle import attention_oracle as ao
from oracle import packing_oracle as po

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _np_pt(pt):
    return po.PackedArrays(pt.packed.cpu().numpy(), pt.scale.cpu().numpy(), pt.mins.cpu().numpy(),
                           pt.bits, pt.axis, pt.group_size, tuple(pt.orig_shape), pt.axis_len)


def _strip(pt):
    """Oracle arrays of row 0 of a batched [1, Hkv, S, hd] PackedTensor."""
    return po.PackedArrays(pt.packed[0].cpu().numpy(), pt.scale[0].cpu().numpy(),
                           pt.mins[0].cpu().numpy(), pt.bits, pt.axis - 1, pt.group_size,
                           tuple(pt.orig_shape[1:]), pt.axis_len)


def _run(q, segs, hq, generic=False):
    from phasekv_amd import decode as dec
    return dec.fused_decode(dec.Problem(q, segs, hq, generic_kernel=generic,
                                        require_mfma=not generic))


def _close(got, want, atol=ATOL, rtol=RTOL):
    got = got.float().cpu().numpy() if torch.is_tensor(got) else got
    np.testing.assert_allclose(got.astype(np.float64), want, atol=atol, rtol=rtol)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("kb,vb", [(2, 2), (2, 4), (2, 8), (4, 2), (4, 4), (4, 8), (8, 2),
                                   (8, 4), (8, 8)])
def test_token_mfma_matches_generic_and_oracle(gpu, hd, kb, vb):
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case hd={hd} bits={kb},{vb}", flush=True)
    g = torch.Generator().manual_seed(100 + kb * 10 + vb + hd)
    hq, hkv = 28, 4
    q = torch.randn(1, hq, hd, generator=g).to(torch.float16)
    parts, segs = [], []
    for length in (700, 64, 33, 5):          # tails inside a group, one group, tiny segments
        kd = (torch.randn(1, hkv, length, hd, generator=g) * 2).to(torch.float16)
        vd = torch.randn(1, hkv, length, hd, generator=g).to(torch.float16)
        pk = quantize_pack(kd.to(gpu), kb, -1, 32)
        pv = quantize_pack(vd.to(gpu), vb, -1, 32)
        segs.append(dec.packed_segment(pk, pv, batched=True))
        parts.append(ao.segment_partial(q[0].numpy(), _strip(pk), _strip(pv), hq))
    hk = torch.randn(1, hkv, 40, hd, generator=g).to(torch.float16)
    hv = torch.randn(1, hkv, 40, hd, generator=g).to(torch.float16)
    segs.append(dec.fp16_segment(hk.to(gpu), hv.to(gpu), batched=True))
    parts.append(ao.fp16_layer_partial(q[0].numpy(), hk[0].numpy(), hv[0].numpy(), hq))
    want = ao.merge_partials(parts, out_dtype=None)
    fast = _run(q.to(gpu), segs, hq)[0].float().cpu().numpy()
    slow = _run(q.to(gpu), segs, hq, generic=True)[0].float().cpu().numpy()
    _close(fast, want)
    _close(slow, want)
    _close(fast, slow, atol=1e-3, rtol=1e-2)


@pytest.mark.parametrize("hq,hkv", [(28, 4), (32, 8), (16, 16), (64, 2), (40, 2)])
def test_token_mfma_gqa_groups_and_head_slabs(gpu, hq, hkv):
    """Group sizes 7, 4, 1, 32 (two head slabs) and 20 (a partial second slab)."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case hq={hq} hkv={hkv}", flush=True)
    g = torch.Generator().manual_seed(hq * 7 + hkv)
    hd = 128
    q = torch.randn(1, hq, hd, generator=g).to(torch.float16)
    kd = torch.randn(1, hkv, 517, hd, generator=g).to(torch.float16)
    vd = torch.randn(1, hkv, 517, hd, generator=g).to(torch.float16)
    pk = quantize_pack(kd.to(gpu), 4, -1, 32)
    pv = quantize_pack(vd.to(gpu), 2, -1, 32)
    want = ao.merge_partials([ao.segment_partial(q[0].numpy(), _strip(pk), _strip(pv), hq)],
                             out_dtype=None)
    _close(_run(q.to(gpu), [dec.packed_segment(pk, pv, batched=True)], hq)[0], want)


def test_token_mfma_batched_ragged(gpu):
    """Batch 3 with per-row valid lengths (one row ends inside a group, one row at 1 token)."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(77)
    B, hq, hkv, hd, S = 3, 28, 4, 128, 1000
    q = torch.randn(B, hq, hd, generator=g).to(torch.float16)
    kd = torch.randn(B, hkv, S, hd, generator=g).to(torch.float16)
    vd = torch.randn(B, hkv, S, hd, generator=g).to(torch.float16)
    pk = quantize_pack(kd.to(gpu), 2, -1, 32)
    pv = quantize_pack(vd.to(gpu), 4, -1, 32)
    lens = [1000, 613, 1]
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=gpu)
    out = _run(q.to(gpu), [dec.packed_segment(pk, pv, batched=True, seq_lens=seq_lens)], hq)
    for b, L in enumerate(lens):
        print(f"  row {b} length {L}", flush=True)
        kb = po.quantize_pack(kd[b, :, :L].float().numpy(), 2, -1, 32)
        vb = po.quantize_pack(vd[b, :, :L].float().numpy(), 4, -1, 32)
        want = ao.merge_partials([ao.segment_partial(q[b].numpy(), kb, vb, hq)], out_dtype=None)
        _close(out[b], want)


def test_token_mfma_reference_split_counts(gpu):
    """decode_attention_packed_splitk at the reference's split grid (8 .. 128 splits of a
    4K prompt): every count whose split length is whole 32-token groups runs on the MFMA
    kernel, and all agree with the oracle; the per-split partials of 64 splits match the
    oracle's split partials."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels import attention_triton as at
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(9)
    hq, hkv, hd, S = 28, 4, 128, 4096
    q = torch.randn(hq, hd, generator=g).to(torch.float16)
    kd = torch.randn(hkv, S, hd, generator=g).to(torch.float16)
    vd = torch.randn(hkv, S, hd, generator=g).to(torch.float16)
    pk = quantize_pack(kd.to(gpu), 2, -1, 32)
    pv = quantize_pack(vd.to(gpu), 2, -1, 32)
    part = ao.segment_partial(q.numpy(), _np_pt(pk), _np_pt(pv), hq)
    want = part[2] / part[1][:, None]
    for ns in (8, 16, 32, 64, 128):
        print(f"  splits {ns}", flush=True)
        seg = dec.packed_segment(pk, pv, batched=False, splits=ns, split_len=-(-S // ns))
        _close(_run(q.to(gpu), [seg], hq)[0], want)
        _close(at.decode_attention_packed_splitk(q.to(gpu), pk, pv, hq, num_splits=ns), want)
    pm, pl, pacc = at._packed_split_launch(q.to(gpu), pk, pv, hq, 64, 64)
    ref_pm, ref_pl, ref_pacc = ao.split_partials(
        q.numpy(), po.dequantize_float(_np_pt(pk)), po.dequantize_float(_np_pt(pv)), hq, 64)
    np.testing.assert_allclose(pm.cpu().numpy(), ref_pm, atol=1e-4)
    np.testing.assert_allclose(pl.cpu().numpy(), ref_pl, rtol=1e-3)
    # each split's output acc / l at the attention bar (acc itself is a sum of up to 64
    # unnormalized terms)
    _close(pacc.cpu().numpy() / pl.cpu().numpy()[..., None], ref_pacc / ref_pl[..., None])


def test_token_mfma_three_tiers(gpu):
    """fused_three_tier_decode over a per-token prompt, a per-token cold tier and an fp16
    hot tier: one MFMA launch for the three."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels import attention_triton as at
    from phasekv_amd.kernels.packing import quantize_pack
    from phasekv_amd.kernels.reference import ThreeTierKV
    g = torch.Generator().manual_seed(21)
    hq, hkv, hd = 28, 4, 128
    q = torch.randn(hq, hd, generator=g).to(torch.float16)
    pk = quantize_pack(torch.randn(hkv, 2048, hd, generator=g).half().to(gpu), 2, -1, 32)
    pv = quantize_pack(torch.randn(hkv, 2048, hd, generator=g).half().to(gpu), 2, -1, 32)
    ck = quantize_pack(torch.randn(hkv, 512, hd, generator=g).half().to(gpu), 4, -1, 32)
    cv = quantize_pack(torch.randn(hkv, 512, hd, generator=g).half().to(gpu), 4, -1, 32)
    hk = torch.randn(hkv, 100, hd, generator=g).half()
    hv = torch.randn(hkv, 100, hd, generator=g).half()
    kv = ThreeTierKV(pk, pv, ck, cv, hk.to(gpu), hv.to(gpu))
    parts = [ao.segment_partial(q.numpy(), _np_pt(pk), _np_pt(pv), hq),
             ao.segment_partial(q.numpy(), _np_pt(ck), _np_pt(cv), hq),
             ao.fp16_layer_partial(q.numpy(), hk.numpy(), hv.numpy(), hq)]
    want = ao.merge_partials(parts, out_dtype=None)
    segs = [dec.packed_segment(pk, pv, batched=False), dec.packed_segment(ck, cv, batched=False),
            dec.fp16_segment(hk.to(gpu), hv.to(gpu), batched=False)]
    _close(_run(q.to(gpu), segs, hq)[0], want)
    _close(at.fused_three_tier_decode(q.to(gpu), kv, hq), want)


def test_token_mfma_refuses_kivi_in_the_same_launch(gpu):
    """KIVI and per-token K segments take different kernels: one problem holding both runs
    on the generic kernel, and require_mfma says so."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(3)
    hq, hkv, hd = 8, 2, 128
    q = torch.randn(hq, hd, generator=g).half().to(gpu)
    x = lambda n: torch.randn(hkv, n, hd, generator=g).half().to(gpu)
    tok = dec.packed_segment(quantize_pack(x(64), 2, -1, 32), quantize_pack(x(64), 2, -1, 32),
                             batched=False)
    kivi = dec.packed_segment(quantize_pack(x(64), 2, -2, 32), quantize_pack(x(64), 2, -1, 32),
                              batched=False)
    with pytest.raises(ValueError, match="MFMA kernel does not apply"):
        _run(q, [tok, kivi], hq)
    out = _run(q, [tok, kivi], hq, generic=True)
    assert torch.isfinite(out).all()


@pytest.mark.parametrize("bits", [2, 4])
def test_published_shape_32k_matches_oracle(gpu, bits):
    """The reference's published legacy shape at its longest context: Hq 28, Hkv 4, hd 128,
    S = 32768, K and V packed per token at `bits` (results/kernel_decode_bench.md:9-16),
    through the planner and through the reference's best split count (128)."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels import attention_triton as at
    from phasekv_amd.kernels.packing import quantize_pack
    print(f"case S=32768 bits={bits}", flush=True)
    g = torch.Generator().manual_seed(1234 + bits)
    hq, hkv, hd, S = 28, 4, 128, 32768
    q = torch.randn(hq, hd, generator=g).to(torch.float16)
    kd = torch.randn(hkv, S, hd, generator=g).to(torch.float16)
    vd = torch.randn(hkv, S, hd, generator=g).to(torch.float16)
    pk = quantize_pack(kd.to(gpu), bits, -1, 32)
    pv = quantize_pack(vd.to(gpu), bits, -1, 32)
    part = ao.segment_partial(q.numpy(), _np_pt(pk), _np_pt(pv), hq)
    want = part[2] / part[1][:, None]
    auto = _run(q.to(gpu), [dec.packed_segment(pk, pv, batched=False)], hq)[0]
    ref128 = at.decode_attention_packed_splitk(q.to(gpu), pk, pv, hq, num_splits=128)
    for got in (auto, ref128):
        err = np.abs(got.float().cpu().numpy() - want).max()
        print(f"  max abs err {err:.2e} (max |out| {np.abs(want).max():.2e})", flush=True)
        # the reference's own bar for its fp32 kernel (tests/test_phasekv_launch_config.py:79)
        _close(got, want, atol=3e-4, rtol=1e-3)
