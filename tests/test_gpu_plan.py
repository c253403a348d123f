"""The automatic decode plan: the weighted chunk plan (per-segment chunk lengths, chunk-major
launch order), the uniform chunk plan and a forced small chunk all give the oracle's result
on a mix of 2/4/8-bit segments, an FP16 window and a ragged batch."""
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


def _problem(gpu, seed):
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels.packing import quantize_pack
    g = torch.Generator().manual_seed(seed)
    b, hq, hkv, hd = 2, 28, 4, 128
    q = torch.randn(b, hq, hd, generator=g).to(torch.float16)
    lens = torch.tensor([3000, 1713], dtype=torch.int32)
    segs, dense = [], [[] for _ in range(b)]
    for length, kb, vb, ragged in ((3000, 2, 2, True), (700, 8, 8, False), (300, 4, 2, False),
                                   (96, 2, 8, False)):
        k = (torch.randn(b, hkv, length, hd, generator=g) * 2).to(torch.float16)
        v = torch.randn(b, hkv, length, hd, generator=g).to(torch.float16)
        pk, pv = quantize_pack(k.to(gpu), kb, -2, 32), quantize_pack(v.to(gpu), vb, -1, 32)
        segs.append(dec.packed_segment(pk, pv, batched=True,
                                       seq_lens=lens.to(gpu) if ragged else None))
        dk, dv = po.dequantize_float(_np_pt(pk)), po.dequantize_float(_np_pt(pv))
        for i in range(b):
            n = int(lens[i]) if ragged else length
            dense[i].append((dk[i, :, :n], dv[i, :, :n]))
    hk = torch.randn(b, hkv, 77, hd, generator=g).to(torch.float16)
    hv = torch.randn(b, hkv, 77, hd, generator=g).to(torch.float16)
    segs.append(dec.fp16_segment(hk.to(gpu), hv.to(gpu), batched=True))
    for i in range(b):
        dense[i].append((hk[i].numpy(), hv[i].numpy()))
    want = np.stack([ao.segments_attention(q[i].numpy(), dense[i], hq) for i in range(b)])
    return dec.Problem(q.to(gpu), segs, hq), want


@pytest.mark.parametrize("seed", [1, 2])
def test_plans_agree_with_the_oracle(gpu, monkeypatch, seed):
    from phasekv_amd import decode as dec
    prob, want = _problem(gpu, seed)
    outs, splits = {}, {}
    for name, env in (("weighted", {}), ("uniform", {"PK_WEIGHTED_PLAN": "0"}),
                      ("chunk128", {"PK_CHUNK_TOKENS": "128"})):
        for key in ("PK_WEIGHTED_PLAN", "PK_CHUNK_TOKENS"):
            monkeypatch.delenv(key, raising=False)
        for key, val in env.items():
            monkeypatch.setenv(key, val)
        print(f"case seed={seed} plan={name}", flush=True)
        splits[name] = prob.workspace_size()[1]
        outs[name] = dec.fused_decode(prob).float().cpu().numpy()
        np.testing.assert_allclose(outs[name], want, atol=ATOL, rtol=RTOL)
    # the plans differ, and agree with each other more tightly than with the oracle
    assert len(set(splits.values())) > 1, splits
    np.testing.assert_allclose(outs["weighted"], outs["uniform"], atol=1e-3, rtol=1e-2)
    np.testing.assert_allclose(outs["weighted"], outs["chunk128"], atol=1e-3, rtol=1e-2)


def test_weighted_plan_graph_replay(gpu):
    """Chunk-major launch order under a captured graph: every replay equals the eager result."""
    from phasekv_amd import decode as dec
    prob, want = _problem(gpu, 5)
    eager = dec.fused_decode(prob)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        dec.fused_decode(prob)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = dec.fused_decode(prob)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        dec.fused_decode(prob)   # eager work between replays
        torch.cuda.synchronize()
    np.testing.assert_allclose(eager.float().cpu().numpy(), want, atol=ATOL, rtol=RTOL)
