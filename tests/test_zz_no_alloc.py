"""pk_fused_decode_noalloc through the C ABI: the same output as pk_fused_decode with a
caller workspace, bit for bit, on two calls in a row (the second problem smaller, so the
scratch array still holds the first call's partials), and a clear error for a problem
whose workspace exceeds the array."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import attention_oracle as ao
from oracle import packing_oracle as po

pytestmark = pytest.mark.gpu


def _problem(cfg_name, gpu):
    from phasekv_amd import workloads
    from phasekv_amd.kernels.attention_triton import phasekv_problem
    wl = workloads.make_workload(workloads.CONFIGS[cfg_name], gpu)
    return wl, phasekv_problem(wl.q[0], wl.tiers, wl.cfg.hq)


def _noalloc(problem):
    from phasekv_amd import _lib
    out = torch.empty(problem.batch, problem.hq, problem.hd, dtype=torch.float16,
                      device=problem.device)
    _lib.check(_lib.load().pk_fused_decode_noalloc(ctypes.byref(problem.c), out.data_ptr(),
                                                   _lib.stream_ptr(problem.device)),
               "fused_decode_noalloc")
    return out


def _with_workspace(problem):
    from phasekv_amd import _lib
    nbytes, _ = problem.workspace_size()
    ws = torch.empty(nbytes, dtype=torch.uint8, device=problem.device)
    out = torch.empty(problem.batch, problem.hq, problem.hd, dtype=torch.float16,
                      device=problem.device)
    _lib.check(_lib.load().pk_fused_decode(ctypes.byref(problem.c), ws.data_ptr(), ws.numel(),
                                           out.data_ptr(), _lib.stream_ptr(problem.device)),
               "fused_decode")
    return out


def _np_pt(pt):
    return po.PackedArrays(pt.packed.cpu().numpy(), pt.scale.cpu().numpy(), pt.mins.cpu().numpy(),
                           pt.bits, pt.axis, pt.group_size, tuple(pt.orig_shape), pt.axis_len)


def test_noalloc_matches_workspace_entry_point_twice(gpu):
    # C2 (28 heads, 4480 tokens) then C1 (14 heads, 544 tokens): the second call reuses
    # the array the first one filled
    for name in ("C2", "C1"):
        print(f"case {name}", flush=True)
        wl, problem = _problem(name, gpu)
        got = _noalloc(problem)
        want = _with_workspace(problem)
        torch.cuda.synchronize()
        assert torch.equal(got, want), name
        hk, hv = wl.tiers.hot_views()
        seg = lambda s: ao.SegmentArrays(_np_pt(s.key), _np_pt(s.value))
        tiers = ao.LayerTiersArrays(seg(wl.tiers.prompt), [], [seg(s) for s in wl.tiers.cold],
                                    hk.cpu().numpy(), hv.cpu().numpy())
        ref = ao.layer_tiers_attention(wl.q[0].cpu().numpy(), tiers, wl.cfg.hq)
        np.testing.assert_allclose(got[0].float().cpu().numpy(), ref, atol=2e-3, rtol=1e-2)


def test_noalloc_refuses_a_workspace_beyond_the_array(gpu):
    from phasekv_amd import _lib
    from phasekv_amd import decode as dec
    # batch 64 x 32 heads over an fp16 segment cut into 32 splits: the partials exceed
    # 16 MiB.  The tensors are never read: the size check fails before any launch.
    q = torch.empty(64, 32, 128, dtype=torch.float16, device=gpu)
    kv = torch.empty(64, 8, 8192, 128, dtype=torch.float16, device=gpu)
    problem = dec.Problem(q, [dec.fp16_segment(kv, kv, batched=True, splits=32)], 32)
    nbytes, _ = problem.workspace_size()
    assert nbytes > _lib.PK_NOALLOC_SCRATCH_BYTES
    out = torch.empty(64, 32, 128, dtype=torch.float16, device=gpu)
    rc = _lib.load().pk_fused_decode_noalloc(ctypes.byref(problem.c), out.data_ptr(),
                                             _lib.stream_ptr(gpu))
    assert rc == _lib.PK_ERR_INVALID
    assert b"workspace" in _lib.load().pk_last_error()
