"""Benchmark of the PhaseKV Stage-B decode attention on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config C2] [--no-sweep] [--no-cpu]
                    [--no-dense] [--copy-probe-mib M] [--lifecycle] [--prefill] [--e2e]

A step is one decode-attention call (one layer, one query token) over the
packed prompt tier, the cold tier and the FP16 hot window of the workload.
Steps are captured into a HIP graph and replayed back to back; each step reads
a different copy of the tiers, and the copies together exceed twice the
256 MB MALL, so the timed bytes come from HBM.  ``value`` is the achieved
algorithmic HBM bandwidth (packed K/V codes + fp16 scale/min + fp16 hot
window + q + output per step) divided by the measured step time.

``roofline`` is the partials kernel (``pk::decode_mfma_kernel``, which reads
every KV byte; the combine launch reads only the small workspace) timed on its
own the same way: algorithmic bytes per launch / its average launch time, and
``traffic``, the HBM bytes per launch that rocprofv3's FETCH_SIZE + WRITE_SIZE
counters read for it, from the committed PMC summary.

Prints ONE JSON line (rank 0).  Extra fields: ``us_per_step``, the FP16 dense
GQA-aware comparator on the same tokens, and ``sweep``: the same measurement
for the context sweep (C3), the batched configurations (C4, C5), C4's
prefill-side quantize + pack of an 8192 x 4 x 128 K/V block, the hot window
lifecycle (append per step, one cooling event) at the C2 and C5 cache shapes, and
the causal attention of a 16/64/256-token input chunk at the C2 cache against the
loop of one decode call per chunk token, and the prefill prompt selection of an
8192-token prompt.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

METRIC = "decode-attn µs/step + HBM GB/s (% of peak), 7B shape, ctx 4K–32K, 1 GPU"
HBM_PEAK_GBS = 8000.0
CACHE_DEFEAT_BYTES = 2 * 256 * 1024 * 1024      # twice the MI355X MALL


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _copies_for(bytes_per_set: int, cap: int = 1024) -> int:
    return max(2, min(cap, math.ceil(CACHE_DEFEAT_BYTES / max(1, bytes_per_set))))


_FLUSH = {}


def _flush_caches(device) -> None:
    """Write a buffer of twice the MALL so that nothing read before stays in L2 or the MALL."""
    buf = _FLUSH.get(device)
    if buf is None:
        buf = _FLUSH[device] = torch.empty(CACHE_DEFEAT_BYTES // 4, dtype=torch.float32,
                                           device=device)
    buf.fill_(1.0)


def _time_graph(fns, steps: int, warmup: int, stream) -> float:
    """Seconds per step of ``steps`` calls captured in one graph, call i reading copy i mod
    len(fns).  The graph is replayed ``warmup`` steps' worth untimed; then the caches are
    flushed (a write of twice the MALL), so the timed replay reads its copies from HBM even
    when it touches fewer copies than the caches hold."""
    with torch.cuda.stream(stream):
        for f in fns:
            f()       # warm workspaces and build every copy's problem outside the capture
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                fns[i % len(fns)]()
        torch.cuda.synchronize()
        for _ in range(max(1, math.ceil(warmup / steps))):
            graph.replay()
        _flush_caches(stream.device)
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        end.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


def _bench_config(cfg, device, steps, warmup, stream, with_dense=True):
    """Step time (partials + combine) and the partials kernel's own time on rotating copies."""
    from phasekv_amd import decode as dec
    from phasekv_amd import workloads
    from phasekv_amd.kernels.attention_triton import (fused_phasekv_decode,
                                                      fused_phasekv_decode_batched,
                                                      phasekv_problem)
    wl = workloads.make_workload(cfg, device, keep_dense=with_dense)
    nbytes = wl.bytes
    copies = _copies_for(nbytes)
    tiers = [wl.tiers] + [workloads.clone_tiers(wl.tiers) for _ in range(copies - 1)]
    q = wl.q
    if cfg.batch == 1:
        fns = [lambda t=t: fused_phasekv_decode(q[0], t, cfg.hq) for t in tiers]
        probs = [phasekv_problem(q[0], t, cfg.hq) for t in tiers]
    else:
        fns = [lambda t=t: fused_phasekv_decode_batched(q, t, cfg.hq, wl.prompt_lens) for t in tiers]
        probs = [phasekv_problem(q, t, cfg.hq, batched=True, prompt_lens=wl.prompt_lens)
                 for t in tiers]
    sec = _time_graph(fns, steps, warmup, stream)
    # the dominant kernel alone: the same steps without the combine launch
    ksec = _time_graph([lambda pr=pr: dec.launch_partials(pr) for pr in probs], steps, warmup,
                       stream)
    # one eager call on one kept tiers object (the decode problem is built on the first
    # call and reused, as in a decode loop), host call to completion, median of 50
    lat = []
    with torch.cuda.stream(stream):
        for i in range(60):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fns[0]()
            torch.cuda.synchronize()
            lat.append(time.perf_counter() - t0)
    single = sorted(lat[10:])[len(lat[10:]) // 2]
    res = {"config": cfg.name, "tokens": cfg.tokens, "bytes": nbytes, "copies": copies,
           "timed_distinct_bytes": min(steps, copies) * nbytes,
           "us_per_step": sec * 1e6, "gbs": nbytes / sec / 1e9,
           "partials_us": ksec * 1e6, "partials_gbs": nbytes / ksec / 1e9,
           "single_call_us": single * 1e6}
    res["frac"] = res["gbs"] / HBM_PEAK_GBS
    del tiers, fns, probs
    if with_dense:
        # uncompressed fp16 K/V of the same tokens (prompt rows at their ragged lengths),
        # read by the same GQA-aware kernel as the hot window: no expanded copies
        dense = [(k.to(device), v.to(device)) for k, v in zip(wl.dense_k, wl.dense_v)
                 if k is not None]
        dbytes = workloads.fp16_dense_bytes(cfg, wl.prompt_lens_list if cfg.ragged_min else None)
        dcopies = _copies_for(dbytes, 64)
        sets = [dense] + [[(k.clone(), v.clone()) for k, v in dense] for _ in range(dcopies - 1)]
        probs = []
        for kv in sets:
            segs = [dec.fp16_segment(k, v, batched=True,
                                     seq_lens=wl.prompt_lens if (i == 0 and cfg.ragged_min) else None)
                    for i, (k, v) in enumerate(kv)]
            probs.append(dec.Problem(q, segs, cfg.hq))
        dfns = [lambda pr=pr: dec.fused_decode(pr) for pr in probs]
        dsec = _time_graph(dfns, steps, warmup, stream)
        res["fp16_dense_us"] = dsec * 1e6
        res["fp16_dense_gbs"] = dbytes / dsec / 1e9
        res["speedup_vs_fp16"] = dsec / sec
        del sets, probs, dfns, dense
    torch.cuda.empty_cache()
    return res, wl


def _bench_long_generation(device, steps, warmup, stream, generated=1056):
    """C2's cache after ``generated`` decode tokens with lazy cooling (lazy_g 16, keep all,
    4-bit cold): 64 cold segments of 16 tokens beside the prompt, C2's cold tier and a
    40-token window.  The decode attends the cold segments from the device segment table
    (one partials launch), timed beside the same segments as one list of launches of up to
    8 segments each."""
    from phasekv_amd import decode as dec
    from phasekv_amd import workloads
    from phasekv_amd.kernels.attention_triton import _reused_problem, fused_phasekv_decode
    base = workloads.CONFIGS["C2"]
    wl = workloads.make_long_generation(base, generated, device)
    cfg = wl.cfg
    nbytes = workloads.tiers_algorithmic_bytes(wl.tiers, cfg.hq)
    copies = _copies_for(nbytes, 96)
    tiers = [wl.tiers] + [workloads.clone_tiers(wl.tiers) for _ in range(copies - 1)]
    q = wl.q[0]
    sec = _time_graph([lambda t=t: fused_phasekv_decode(q, t, cfg.hq) for t in tiers], steps,
                      warmup, stream)
    probs = [_reused_problem(q, t, cfg.hq) for t in tiers]
    listed = [dec.Problem(q, [pr.segments[0], *pr.segments[1:-1], *pr.table.segments,
                              pr.segments[-1]], cfg.hq) for pr in probs]
    lsec = _time_graph([lambda pr=pr: dec.fused_decode(pr) for pr in listed], steps, warmup,
                       stream)
    ksec = _time_graph([lambda pr=pr: dec.launch_partials(pr) for pr in probs], steps, warmup,
                       stream)
    n_list = len(listed[0].segments)
    res = {"config": cfg.name, "generated_tokens": generated,
           "cold_segments": len(wl.tiers.cold), "table_entries": probs[0].table.count,
           "tokens": cfg.prompt + cfg.cold + cfg.hot, "bytes": nbytes, "copies": copies,
           "timed_distinct_bytes": min(steps, copies) * nbytes,
           "us_per_step": sec * 1e6, "gbs": nbytes / sec / 1e9, "partials_launches": 1,
           "partials_us": ksec * 1e6,
           "listed_us_per_step": lsec * 1e6,
           "listed_partials_launches": -(-n_list // 8),
           "speedup_vs_listed": lsec / sec}
    del tiers, probs, listed
    torch.cuda.empty_cache()
    return res


# The reference's published legacy numbers (RTX 4080 SUPER, split-K kernel at its best
# split count, ms; results/kernel_decode_bench.md:9-16), keyed by (S, bits).
LEGACY_PUBLISHED_MS = {(4096, 2): 0.1321, (4096, 4): 0.24576, (8192, 2): 0.22323,
                       (8192, 4): 0.29082, (16384, 2): 0.40346, (16384, 4): 0.54374,
                       (32768, 2): 0.76595, (32768, 4): 1.05165}


def _bench_legacy(device, S, bits, steps, warmup, stream, with_dense=True, with_grid=True):
    """The reference's legacy per-token layout at its published shape (Hq 28, Hkv 4, hd 128,
    group 32, prompt only, K and V packed per token at ``bits``; seeded N(0,1) K/V/q as
    scripts/bench_decode_kernel.py:66-84): the planner's launch, the reference's split grid
    (8 .. 128 splits, best), the partials kernel alone, and the GQA-aware FP16 kernel over the
    same tokens."""
    from phasekv_amd import decode as dec
    from phasekv_amd.kernels import attention_triton as at
    from phasekv_amd.kernels.packing import quantize_pack
    hq, hkv, hd = 28, 4, 128
    g = torch.Generator().manual_seed(1234)
    K = torch.randn(hkv, S, hd, generator=g).to(torch.float16).to(device)
    V = torch.randn(hkv, S, hd, generator=g).to(torch.float16).to(device)
    q = torch.randn(hq, hd, generator=g).to(torch.float16).to(device)
    pk = quantize_pack(K, bits, -1, 32)
    pv = quantize_pack(V, bits, -1, 32)
    kv_bytes = sum(t.numel() * t.element_size() for pt in (pk, pv)
                   for t in (pt.packed, pt.scale, pt.mins))
    nbytes = kv_bytes + 2 * 2 * hq * hd
    copies = _copies_for(nbytes)
    clone = lambda pt: type(pt)(pt.packed.clone(), pt.scale.clone(), pt.mins.clone(), pt.bits,
                                pt.axis, pt.group_size, pt.orig_shape, pt.axis_len)
    sets = [(pk, pv)] + [(clone(pk), clone(pv)) for _ in range(copies - 1)]
    probs = [dec.Problem(q, [dec.packed_segment(a, b, batched=False)], hq, require_mfma=True)
             for a, b in sets]
    sec = _time_graph([lambda pr=pr: dec.fused_decode(pr) for pr in probs], steps, warmup, stream)
    ksec = _time_graph([lambda pr=pr: dec.launch_partials(pr) for pr in probs], steps, warmup,
                       stream)
    grid = {}
    for ns in ((8, 16, 32, 64, 128) if with_grid else ()):
        grid[ns] = _time_graph([lambda a=a, b=b: at.decode_attention_packed_splitk(
            q, a, b, hq, num_splits=ns) for a, b in sets], steps, warmup, stream)
    best_ns = min(grid, key=grid.get) if grid else None
    ref_ms = LEGACY_PUBLISHED_MS.get((S, bits))
    res = {"config": f"legacy-S{S}-{bits}b", "shape": "Hq28/Hkv4/hd128, per-token K and V",
           "S": S, "bits": bits, "bytes": nbytes, "copies": copies,
           "timed_distinct_bytes": min(steps, copies) * nbytes,
           "us_per_step": sec * 1e6, "gbs": nbytes / sec / 1e9,
           "partials_us": ksec * 1e6, "partials_gbs": nbytes / ksec / 1e9,
           "splitk_grid_us": {str(k): round(v * 1e6, 3) for k, v in grid.items()},
           "splitk_best_us": grid[best_ns] * 1e6 if grid else None, "splitk_best_splits": best_ns,
           "ref_published_splitk_us": ref_ms * 1e3 if ref_ms else None}
    res["frac"] = res["gbs"] / HBM_PEAK_GBS
    res["partials_frac"] = res["partials_gbs"] / HBM_PEAK_GBS
    if ref_ms:
        res["speedup_vs_ref_published"] = ref_ms * 1e-3 / sec
    del sets, probs
    if with_dense:
        dbytes = 2 * hkv * S * hd * 2 + 2 * 2 * hq * hd
        dcopies = _copies_for(dbytes, 64)
        dsets = [(K, V)] + [(K.clone(), V.clone()) for _ in range(dcopies - 1)]
        dprobs = [dec.Problem(q, [dec.fp16_segment(k, v, batched=False)], hq) for k, v in dsets]
        dsec = _time_graph([lambda pr=pr: dec.fused_decode(pr) for pr in dprobs], steps, warmup,
                           stream)
        res["fp16_dense_us"] = dsec * 1e6
        res["fp16_dense_gbs"] = dbytes / dsec / 1e9
        res["speedup_vs_fp16"] = dsec / sec
        del dsets, dprobs
    torch.cuda.empty_cache()
    return res


def _legacy_rows(device, steps, warmup, stream, with_dense=True, with_grid=True,
                 lengths=(4096, 8192, 16384, 32768), widths=(2, 4)):
    rows = []
    for S in lengths:
        for bits in widths:
            r = _bench_legacy(device, S, bits, steps, warmup, stream, with_dense, with_grid)
            _log(f"bench: legacy {r}")
            rows.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
    return rows


def _bench_prefill_pack(device, steps, warmup, stream):
    """C4's prefill side: an 8192 x 4 x 128 fp16 K/V block packed to the 2-bit prompt tier.

    K is quantized per channel along tokens (axis -2), V per token along head_dim
    (axis -1), groups of 32 (``phasekv_cache.py:101-107``), by the cache's ``pack_kv``
    (one launch for both); ``two_launch_us`` times the two ``quantize_pack`` calls.
    Algorithmic bytes: the fp16 block read once, packed codes and fp16 scale/min
    written once.
    """
    from phasekv_amd.kernels.packing import quantize_pack
    from phasekv_amd.tiers import pack_kv
    gen = torch.Generator().manual_seed(1234)
    shape = (1, 4, 8192, 128)
    k = torch.randn(*shape, generator=gen).to(torch.float16).to(device)
    v = torch.randn(*shape, generator=gen).to(torch.float16).to(device)
    elems = k.numel()
    nbytes = 2 * (2 * elems) + 2 * (elems // 4) + 2 * 2 * 2 * (elems // 32)
    copies = _copies_for(2 * 2 * elems, 64)
    sets = [(k, v)] + [(k.clone(), v.clone()) for _ in range(copies - 1)]
    fns = [lambda kv=kv: pack_kv(kv[0], kv[1], 2, 32) for kv in sets]
    sec = _time_graph(fns, steps, warmup, stream)
    fns = [lambda kv=kv: (quantize_pack(kv[0], 2, -2, 32), quantize_pack(kv[1], 2, -1, 32))
           for kv in sets]
    sec2 = _time_graph(fns, steps, warmup, stream)
    del sets, fns
    torch.cuda.empty_cache()
    return {"config": "C4-prefill-pack", "shape": list(shape), "bits": 2, "bytes": nbytes,
            "copies": copies, "us_per_step": sec * 1e6, "two_launch_us": sec2 * 1e6, "gbs": nbytes / sec / 1e9,
            "frac": nbytes / sec / 1e9 / HBM_PEAK_GBS}


def _bench_lifecycle(cfg, device, steps, warmup, stream, ratio, with_cpu):
    """The hot window lifecycle of one layer at ``cfg``'s cache shape (recent window 32,
    lazy_g 16, 4-bit cold segments: ``phasekv_cache.py:185-196`` defaults): the
    ``append_hot`` launch of every decode step, and one cooling event (one launch
    that ranks, gathers and packs the new segment and shifts the window; the
    three-launch form, cooling then two ``quantize_pack``, is timed beside it),
    which fires once every lazy_g steps.  Both are latency-bound: a cooling event moves
    ``B * Hkv * 48`` rows of ``hd`` fp16 values.
    """
    from phasekv_amd import _lib
    from phasekv_amd.cache import cool_hot, cool_pack_hot, cool_pack_supported, keep_count
    from phasekv_amd.kernels.packing import quantize_pack
    window, lazy_g, bits = 32, 16, 4
    cap = window + lazy_g
    B, H, D = cfg.batch, cfg.hkv, cfg.hd
    gen = torch.Generator().manual_seed(1234)
    hot_k = torch.randn(B, H, cap, D, generator=gen).to(torch.float16).to(device)
    hot_v = torch.randn(B, H, cap, D, generator=gen).to(torch.float16).to(device)
    tok = torch.randn(B, H, 1, D, generator=gen).to(torch.float16).to(device)
    keep = keep_count(lazy_g, ratio)
    lib = _lib.load()

    def append():
        _lib.check(lib.pk_append_hot(tok.data_ptr(), tok.data_ptr(), tok.stride(0), tok.stride(1),
                                     tok.stride(0), tok.stride(1), hot_k.data_ptr(),
                                     hot_v.data_ptr(), hot_k.stride(0), hot_k.stride(1),
                                     hot_k.stride(2), B, H, D, cap - 1, cap,
                                     _lib.stream_ptr(device)), "append_hot")

    def cool():
        cool_pack_hot(hot_k, hot_v, cap, lazy_g, keep, bits, 32)

    def cool_unfused():
        k, v, _ = cool_hot(hot_k, hot_v, cap, lazy_g, keep)
        quantize_pack(k, bits, -2, 32)
        quantize_pack(v, bits, -1, 32)

    a_sec = _time_graph([append], steps, warmup, stream)
    c_sec = _time_graph([cool], steps, warmup, stream)
    u_sec = _time_graph([cool_unfused], steps, warmup, stream)
    res = {"config": f"{cfg.name}-lifecycle", "shape": [B, H, cap, D], "recent_window": window,
           "lazy_g": lazy_g, "decode_keep_ratio": ratio, "cold_bits": bits,
           "append_us": a_sec * 1e6, "cooling_us": c_sec * 1e6,
           "cooling_three_launches_us": u_sec * 1e6, "fused": cool_pack_supported(
               hot_k, hot_v, cap, lazy_g, keep, 32),
           "us_per_layer_step": (a_sec + c_sec / lazy_g) * 1e6}
    if with_cpu:
        # the numpy oracle of the same event on the host: the reference's CPU path
        from oracle import cache_oracle as co
        hk, hv = hot_k.cpu().numpy(), hot_v.cpu().numpy()
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 1.0:
            co.cool_aged_tokens(hk.copy(), hv.copy(), cap, window, lazy_g, ratio, bits, 32)
            n += 1
        res["cpu_cooling_us"] = (time.perf_counter() - t0) / n * 1e6
    del hot_k, hot_v
    torch.cuda.empty_cache()
    return res


def _bench_prompt_chunk(cfg, device, T, steps, warmup, stream):
    """A T-token input chunk at ``cfg``'s cache (its packed tiers, 128 generated hot rows
    and the chunk as the window's last T rows): the one-pass causal chunk attention
    against the reference adapter's loop of T decode calls (one per chunk token)."""
    import dataclasses
    from phasekv_amd import workloads
    from phasekv_amd.kernels.attention_triton import (fused_phasekv_decode,
                                                      fused_phasekv_prompt_chunk_attention)
    wl = workloads.make_workload(cfg, device)
    gen = torch.Generator().manual_seed(77)
    shape = (1, cfg.hkv, cfg.hot + T, cfg.hd)
    hk = torch.randn(*shape, generator=gen).to(torch.float16).to(device)
    hv = torch.randn(*shape, generator=gen).to(torch.float16).to(device)
    tiers = dataclasses.replace(wl.tiers, hot_k=hk, hot_v=hv, hot_len=cfg.hot + T)
    q = torch.randn(T, cfg.hq, cfg.hd, generator=gen).to(torch.float16).to(device)
    one = _time_graph([lambda: fused_phasekv_prompt_chunk_attention(q, tiers, cfg.hq)], steps,
                      warmup, stream)
    by = {m: _time_graph([lambda m=m: fused_phasekv_prompt_chunk_attention(q, tiers, cfg.hq, m)],
                         steps, warmup, stream) for m in ("heads", "batch")}
    views = [dataclasses.replace(tiers, hot_len=cfg.hot + t + 1) for t in range(T)]

    def loop():
        for t in range(T):
            fused_phasekv_decode(q[t], views[t], cfg.hq)

    lsec = _time_graph([loop], max(2, steps // 8), max(2, warmup // 8), stream)
    del wl, tiers, views
    torch.cuda.empty_cache()
    return {"config": f"{cfg.name}-prompt-chunk", "chunk_tokens": T, "chunk_us": one * 1e6,
            "us_per_chunk_token": one * 1e6 / T, "heads_us": by["heads"] * 1e6,
            "batch_us": by["batch"] * 1e6, "per_token_loop_us": lsec * 1e6,
            "speedup_vs_loop": lsec / one}


def _bench_prompt_select(device, steps, warmup, stream, with_cpu):
    """C4's prefill side, selection: one layer's prompt selection over an 8192-token
    prompt (Hq 28 / Hkv 4, observation window 64, keep 25 %, 4 sinks, max pooling over
    7): the votes read the window's 64 rows of every query head's attention (fp16, the
    only rows the selection reads), then the per-kv-head pooling and top-k."""
    from phasekv_amd.prompt_tier import select_prompt_indices

    class Cfg:
        num_key_value_heads, num_attention_heads = 4, 28

    L, w = 8192, 64
    gen = torch.Generator().manual_seed(1234)
    attn = torch.softmax(torch.randn(1, 28, w, L, generator=gen) * 3, dim=-1).to(torch.float16)
    kw = dict(prompt_len=L, model_config=Cfg, prefill_keep_ratio=0.25, sink_tokens=4,
              obs_window=w, pool_kernel=7, pooling="maxpool")
    nbytes = attn.numel() * 2
    # rotating copies of the attention rows, so that the votes read HBM as a prefill does
    dev_attn = attn.to(device)
    sets = [dev_attn] + [dev_attn.clone() for _ in range(_copies_for(nbytes) - 1)]
    sec = _time_graph([lambda a=a: select_prompt_indices([a], **kw) for a in sets], steps,
                      warmup, stream)
    res = {"config": "C4-prefill-select", "prompt_len": L, "obs_window": w, "us": sec * 1e6,
           "copies": len(sets), "votes_bytes": nbytes, "gbs": nbytes / sec / 1e9}
    if with_cpu:
        from oracle import select_oracle as so
        a = attn.float().numpy()
        t0 = time.perf_counter()
        so.select_prompt_indices([a], num_kv_heads=4, **{k: v for k, v in kw.items()
                                                         if k != "model_config"})
        res["cpu_us"] = (time.perf_counter() - t0) * 1e6
    del dev_attn, sets
    torch.cuda.empty_cache()
    return res


def _bench_e2e(device, prompt_len, layers, steps):
    """Time per output token of a random-weight Qwen2.5-7B-shaped model (``layers`` of its
    28 decoder layers, fp16) decoding after a ``prompt_len``-token prefill: the PhaseKV
    adapter (2-bit prompt, 4-bit cold, FP16 window of 32 + 16) against the model's own
    dense DynamicCache decode with SDPA, both in eager mode (the same Python overhead)."""
    from transformers import DynamicCache, Qwen2Config, Qwen2ForCausalLM
    from phasekv_amd.qwen2_attention import (install_qwen2_phasekv_attention, phasekv_prefill,
                                             phasekv_step)
    cfg = Qwen2Config(vocab_size=152064, hidden_size=3584, intermediate_size=18944,
                      num_hidden_layers=layers, num_attention_heads=28, num_key_value_heads=4,
                      max_position_embeddings=32768, attn_implementation="sdpa")
    torch.manual_seed(0)
    with torch.device(device):
        model = Qwen2ForCausalLM(cfg).half().eval()
    install_qwen2_phasekv_attention(model)
    gen = torch.Generator().manual_seed(1234)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=gen).to(device)
    toks = torch.randint(0, cfg.vocab_size, (steps + 8, 1), generator=gen).to(device)
    with torch.no_grad():
        _, cache = phasekv_prefill(model, prompt, prompt_bits=2, cold_bits=4)
        dense = DynamicCache(config=cfg)
        model(prompt, past_key_values=dense, use_cache=True)
        for i in range(8):
            phasekv_step(model, toks[i:i + 1], cache)
            model(toks[i:i + 1], past_key_values=dense, use_cache=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(8, 8 + steps):
            phasekv_step(model, toks[i:i + 1], cache)
        torch.cuda.synchronize()
        pk = (time.perf_counter() - t0) / steps
        t0 = time.perf_counter()
        for i in range(8, 8 + steps):
            model(toks[i:i + 1], past_key_values=dense, use_cache=True)
        torch.cuda.synchronize()
        dn = (time.perf_counter() - t0) / steps
        # a new input chunk of 64 tokens (a follow-up turn), 4 in a row: the adapter appends,
        # attends in one chunk launch per layer and packs the chunk into a prompt extension
        chunk_t, chunks = 64, 4
        cids = torch.randint(0, cfg.vocab_size, (chunks + 1, chunk_t), generator=gen).to(device)
        phasekv_step(model, cids[:1], cache)                       # untimed first chunk
        model(cids[:1], past_key_values=dense, use_cache=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(1, chunks + 1):
            phasekv_step(model, cids[i:i + 1], cache)
        torch.cuda.synchronize()
        pk_chunk = (time.perf_counter() - t0) / chunks
        t0 = time.perf_counter()
        for i in range(1, chunks + 1):
            model(cids[i:i + 1], past_key_values=dense, use_cache=True)
        torch.cuda.synchronize()
        dn_chunk = (time.perf_counter() - t0) / chunks
    del model, cache, dense
    torch.cuda.empty_cache()
    return {"config": f"e2e-qwen2.5-7b-shape-{layers}L", "prompt_len": prompt_len,
            "phasekv_ms_per_token": pk * 1e3, "dense_ms_per_token": dn * 1e3,
            "speedup_vs_dense": dn / pk, "chunk_tokens": chunk_t,
            "phasekv_ms_per_chunk": pk_chunk * 1e3, "dense_ms_per_chunk": dn_chunk * 1e3,
            "chunk_speedup_vs_dense": dn_chunk / pk_chunk}


def _cpu_baseline(cfg_name: str, budget_s: float = 10.0):
    """The oracle (reference.py semantics in numpy) on host cores, bounded sample."""
    import numpy as np
    from threadpoolctl import threadpool_limits
    from oracle import attention_oracle as ao
    from oracle import packing_oracle as po
    from phasekv_amd import workloads
    cfg = workloads.CONFIGS[cfg_name]
    threads = min(16, os.cpu_count() or 1)
    gen = torch.Generator().manual_seed(1234)
    q = torch.randn(1, cfg.hq, 1, cfg.hd, generator=gen).to(torch.float16).numpy()
    rnd = lambda n: torch.randn(1, cfg.hkv, n, cfg.hd, generator=gen).to(torch.float16).numpy()
    kv = ao.ThreeTierArrays(
        po.quantize_pack(rnd(cfg.prompt), cfg.prompt_bits, -2, 32),
        po.quantize_pack(rnd(cfg.prompt), cfg.prompt_bits, -1, 32),
        po.quantize_pack(rnd(cfg.cold), cfg.cold_bits, -2, 32) if cfg.cold else None,
        po.quantize_pack(rnd(cfg.cold), cfg.cold_bits, -1, 32) if cfg.cold else None,
        rnd(cfg.hot), rnd(cfg.hot))
    times = []
    with threadpool_limits(limits=threads):
        ao.fused_decode_attention_reference(q, kv, cfg.hq)
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            ao.fused_decode_attention_reference(q, kv, cfg.hq)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    nbytes = workloads.algorithmic_bytes(cfg)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_step": med * 1e3,
            "sample": f"{len(times)} {cfg_name} decode steps of the numpy oracle "
                      "(dequantize every tier, concat, GQA expand, fp32 softmax attention), median"}


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def _measured_traffic(cfg_name: str):
    """HBM bytes per partials launch from the committed rocprofv3 PMC summary, if any.

    ``profiles/decode_mfma_<config>.md`` holds a line ``traffic_bytes_per_launch <config>
    <bytes>``: FETCH_SIZE + WRITE_SIZE per dispatch of the partials kernel, each scaled by
    what the same counter reads for a copy of known size (``--copy-probe-mib``).
    """
    try:
        with open(os.path.join(PROFILES, f"decode_mfma_{cfg_name}.md")) as fh:
            for line in fh:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == cfg_name:
                    return int(parts[2])
    except OSError:
        pass
    return None


def _copy_probe(mib: int, device) -> None:
    """Three plain device copies of ``mib`` MiB: the calibration dispatches of a PMC run."""
    src = torch.ones(mib << 19, dtype=torch.float16, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    _log(f"bench: copy probe {mib} MiB read + {mib} MiB written per dispatch, 3 dispatches")
    del src, dst
    torch.cuda.empty_cache()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=512)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-dense", action="store_true", help="skip the FP16 dense comparator")
    ap.add_argument("--e2e", action="store_true",
                    help="time per output token of the Qwen2 adapter against the dense cache")
    ap.add_argument("--prefill", action="store_true",
                    help="time only the prefill side (C4 pack, prompt selection) and print its line")
    ap.add_argument("--long-generation", action="store_true",
                    help="time only the C2 cache after 1056 generated tokens (64 cold segments)")
    ap.add_argument("--legacy", action="store_true",
                    help="time only the legacy per-token layout at the reference's published "
                         "shape and print its line")
    ap.add_argument("--legacy-lengths", type=int, nargs="+", default=[4096, 8192, 16384, 32768])
    ap.add_argument("--legacy-bits", type=int, nargs="+", default=[2, 4])
    ap.add_argument("--no-grid", action="store_true",
                    help="legacy rows without the reference's split-count grid")
    ap.add_argument("--lifecycle", action="store_true",
                    help="time only the hot window lifecycle (append, cooling) and print its line")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run plain copies of this size (PMC calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the decode path "
              "runs on one GPU and multi-GPU sharding is design-only", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    from phasekv_amd import _lib, workloads
    _lib.load()
    device = torch.device("cuda:0")
    stream = torch.cuda.Stream(device)
    cfg = workloads.CONFIGS[args.config]
    if args.copy_probe_mib > 0:
        _copy_probe(args.copy_probe_mib, device)
    if args.e2e:
        rows = [_bench_e2e(device, L, 4, 32) for L in (4096, 16384, 32768)]
        rows = [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
                for r in rows]
        print(json.dumps({"metric": "time per output token, Qwen2.5-7B-shaped random-weight "
                                    "model (4 of 28 layers), PhaseKV adapter vs dense cache",
                          "value": rows[0]["phasekv_ms_per_token"], "unit": "ms",
                          "higher_is_better": False, "n_gpus": 1,
                          "config": {"workload": "Qwen2.5-7B shape, 4 layers, fp16"},
                          "rows": rows}), flush=True)
        return 0
    if args.prefill:
        rows = [_bench_prefill_pack(device, min(args.steps, 128), min(args.warmup, 128), stream),
                _bench_prompt_select(device, 64, 64, stream, not args.no_cpu)]
        rows = [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
                for r in rows]
        print(json.dumps({"metric": "prefill side: C4 pack µs and prompt selection µs per layer",
                          "value": rows[1]["us"], "unit": "µs", "higher_is_better": False,
                          "n_gpus": 1, "config": {"workload": "C4 prefill"}, "rows": rows}),
              flush=True)
        return 0
    if args.long_generation:
        r = _bench_long_generation(device, min(args.steps, 256), min(args.warmup, 256), stream)
        r = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
        print(json.dumps({"metric": "decode-attn µs/step, C2 cache after 1056 generated tokens",
                          "value": r["us_per_step"], "unit": "µs", "higher_is_better": False,
                          "n_gpus": 1, "config": {"workload": r["config"]}, "rows": [r]}),
              flush=True)
        return 0
    if args.legacy:
        rows = _legacy_rows(device, min(args.steps, 256), min(args.warmup, 256), stream,
                            not args.no_dense, not args.no_grid, args.legacy_lengths,
                            args.legacy_bits)
        print(json.dumps({"metric": "legacy per-token layout decode-attn µs/step, Hq28/Hkv4/"
                                    "hd128, prompt only, S 4K-32K, 2/4-bit",
                          "value": rows[-1]["us_per_step"], "unit": "µs",
                          "higher_is_better": False, "n_gpus": 1,
                          "config": {"workload": rows[-1]["config"]}, "rows": rows}), flush=True)
        return 0
    if args.lifecycle:
        rows = []
        for name, ratio in (("C2", 1.0), ("C2", 0.5), ("C5", 0.5)):
            r = _bench_lifecycle(workloads.CONFIGS[name], device, min(args.steps, 128),
                                 min(args.warmup, 128), stream, ratio, not args.no_cpu)
            rows.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
        print(json.dumps({"metric": "hot window lifecycle: µs per layer-step (append + cooling "
                                    "event / lazy_g)", "value": rows[0]["us_per_layer_step"],
                          "unit": "µs", "higher_is_better": False, "n_gpus": 1,
                          "config": {"workload": "C2 cache shape, keep all"}, "rows": rows}),
              flush=True)
        return 0
    _log(f"bench: {cfg} steps={args.steps} warmup={args.warmup}")
    main_res, _ = _bench_config(cfg, device, args.steps, args.warmup, stream,
                                with_dense=not args.no_dense)
    _log(f"bench: {cfg.name} {main_res}")
    sweep = []
    if not args.no_sweep:
        for name in ("C1", "C3-4K", "C3-8K", "C3-16K", "C3-32K", "C4", "C5"):
            steps = min(args.steps, 256) if workloads.CONFIGS[name].batch == 1 else 32
            r, _ = _bench_config(workloads.CONFIGS[name], device, steps, min(args.warmup, steps),
                                 stream, with_dense=not args.no_dense)
            if name == "C1" and not args.no_cpu:
                # the CPU reference path at the Qwen2.5-0.5B shape
                r["cpu_baseline"] = _cpu_baseline("C1", min(args.cpu_seconds, 5.0))
            _log(f"bench: {name} {r}")
            sweep.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
        sweep.extend(_legacy_rows(device, min(args.steps, 256), min(args.warmup, 256), stream,
                                  not args.no_dense))
        r = _bench_long_generation(device, min(args.steps, 256), min(args.warmup, 256), stream)
        _log(f"bench: long generation {r}")
        sweep.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
        r = _bench_prefill_pack(device, min(args.steps, 128), min(args.warmup, 128), stream)
        _log(f"bench: C4-prefill-pack {r}")
        sweep.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
        for name, ratio in (("C2", 1.0), ("C2", 0.5), ("C5", 0.5)):
            r = _bench_lifecycle(workloads.CONFIGS[name], device, min(args.steps, 128),
                                 min(args.warmup, 128), stream, ratio, not args.no_cpu)
            _log(f"bench: lifecycle {r}")
            sweep.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
        r = _bench_prompt_select(device, 64, 64, stream, not args.no_cpu)
        _log(f"bench: prompt select {r}")
        sweep.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
        for T in (16, 64, 256):
            r = _bench_prompt_chunk(workloads.CONFIGS["C2"], device, T, 32, 32, stream)
            _log(f"bench: prompt chunk {r}")
            sweep.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
    cpu = None
    if not args.no_cpu:
        cpu = _cpu_baseline(cfg.name if cfg.batch == 1 else "C2", args.cpu_seconds)
        _log(f"bench: cpu baseline {cpu}")
    line = {
        "metric": METRIC,
        "value": round(main_res["gbs"], 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_res["us_per_step"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded N(0,1) K/V with 4 outlier K channels per kv head x8",
        "config": {"workload": f"{cfg.name}: Qwen2.5-7B decode attention, Hq{cfg.hq}/Hkv{cfg.hkv}/"
                               f"hd{cfg.hd}, prompt {cfg.prompt}@{cfg.prompt_bits}b, cold "
                               f"{cfg.cold}@{cfg.cold_bits}b, hot {cfg.hot} fp16, batch {cfg.batch}",
                   "global_batch": cfg.batch, "seq_len": cfg.tokens, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "pk::decode_mfma_kernel",
                     "achieved": round(main_res["partials_gbs"], 3), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(main_res["partials_gbs"] / HBM_PEAK_GBS, 5),
                     "traffic": _measured_traffic(cfg.name),
                     "bytes_per_launch": main_res["bytes"],
                     "launch_us": round(main_res["partials_us"], 3)},
        "cpu_baseline": cpu,
        "us_per_step": round(main_res["us_per_step"], 3),
        "single_call_us": round(main_res["single_call_us"], 3),
        "fp16_dense_us": round(main_res.get("fp16_dense_us", float("nan")), 3),
        "speedup_vs_fp16": round(main_res.get("speedup_vs_fp16", float("nan")), 4),
        "rotating_copies": main_res["copies"],
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
