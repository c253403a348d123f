"""Fused mixed-precision decode attention on MI355X (drop-in for the reference's attention_triton.py).

The module keeps the reference's name and public functions so callers
(``phasekv_cache``, the Qwen2 / Llama adapters, benches and tests) run
unchanged, but nothing here is Triton: every function launches the
hand-written HIP kernels of ``libphasekv_hip.so`` through its C ABI.

Differences in *how*, not *what*:

* ``fused_phasekv_decode`` covers the prompt segment, every prompt extension,
  every cold segment and the FP16 hot window in ONE partials launch (per 8
  segments) plus ONE log-sum-exp combine launch, instead of one Triton launch
  per segment plus ~25 torch ops (``attention_triton.py:643-669``).
* One workgroup serves all query heads of a GQA group, so each packed K/V byte
  is read once per kv head, not once per query head (``attention_triton.py:534``).
* ``num_splits`` / ``block_n`` / ``num_warps`` are validated exactly as the
  reference's ``plan_kivi_decode`` does; when any is given, the split
  boundaries follow that plan, otherwise the library's MI355X planner chooses.
  ``num_warps`` has no other effect (workgroups are 256 threads).
"""
from __future__ import annotations

from dataclasses import replace
from functools import lru_cache

import torch

from .. import _lib
from .. import decode as _dec
from .launch_config import plan_kivi_decode
from .packing import PackedTensor, _vals_per_byte


@lru_cache(maxsize=32)
def _device_sm_count(device: torch.device) -> int:
    """Compute units of the device (``attention_triton.py:599-601``)."""
    return _lib.device_cu_count(device)


def _override_plan(seq_len, num_heads, head_dim, device, num_splits, block_n, num_warps):
    """(splits, split_len) for a segment: the reference plan if any override is given."""
    if num_splits is None and block_n is None and num_warps is None:
        return 0, 0
    cfg = plan_kivi_decode(seq_len, num_heads, head_dim, _device_sm_count(device),
                           num_splits, block_n, num_warps)
    return cfg.num_splits, cfg.split_len


# ---------------------------------------------------------------------------
# legacy per-token packed path (attention_triton.py:24-282)
# ---------------------------------------------------------------------------
def decode_attention_packed(q: torch.Tensor, packed_k: PackedTensor, packed_v: PackedTensor,
                            num_attention_heads: int, block_n: int = 64) -> torch.Tensor:
    """Packed-KV decode attention, K and V both per-token packed (``attention_triton.py:95-142``).

    q ``[Hq, hd]`` fp16; packed_k/packed_v from ``quantize_pack(x, bits, -1, gs)`` over
    ``[Hkv, S, hd]``.  Returns ``[Hq, hd]`` fp16.
    """
    hkv, s_len, hd = packed_k.orig_shape
    if q.shape != (num_attention_heads, hd):
        raise ValueError(f"q must be [Hq={num_attention_heads}, hd={hd}], got {tuple(q.shape)}")
    if num_attention_heads % hkv != 0:
        raise ValueError(f"Hq {num_attention_heads} is not a multiple of Hkv {hkv}")
    vpb = _vals_per_byte(packed_k.bits)
    gs = packed_k.group_size
    if hd % vpb != 0 or hd % gs != 0:
        raise ValueError(f"head_dim ({hd}) must be divisible by vpb ({vpb}) and group_size ({gs})")
    seg = _dec.packed_segment(packed_k, packed_v, batched=False)
    return _dec.fused_decode(_dec.Problem(q, [seg], num_attention_heads))[0]


def _packed_split_launch(q: torch.Tensor, packed_k: PackedTensor, packed_v: PackedTensor,
                         num_attention_heads: int, num_splits: int, block_n: int):
    """Split-K partials (pm, pl, pacc) ``[Hq, num_splits(, hd)]`` (``attention_triton.py:216-254``).

    ``num_splits = max(1, min(num_splits, S))`` splits of ``ceil(S / num_splits)``
    tokens; trailing splits may be empty (m = -inf, l = 0, acc = 0).
    """
    hkv, s_len, hd = packed_k.orig_shape
    if q.shape != (num_attention_heads, hd):
        raise ValueError(f"q must be [Hq={num_attention_heads}, hd={hd}], got {tuple(q.shape)}")
    num_splits = max(1, min(int(num_splits), s_len))
    split_len = -(-s_len // num_splits)
    seg = _dec.packed_segment(packed_k, packed_v, batched=False, splits=num_splits,
                              split_len=split_len)
    return _dec.decode_partials(_dec.Problem(q, [seg], num_attention_heads))


def _reduce_splits(pm, pl, pacc):
    """Merge split partials into one unnormalized (m, l, acc) (``attention_triton.py:257-266``)."""
    return _dec.merge_partials(pm, pl, pacc, normalize=False)


def decode_attention_packed_splitk(q: torch.Tensor, packed_k: PackedTensor,
                                   packed_v: PackedTensor, num_attention_heads: int,
                                   num_splits: int = 8, block_n: int = 64) -> torch.Tensor:
    """Split-K packed decode (``attention_triton.py:269-276``), partials merged in the same launch."""
    hkv, s_len, hd = packed_k.orig_shape
    if q.shape != (num_attention_heads, hd):
        raise ValueError(f"q must be [Hq={num_attention_heads}, hd={hd}], got {tuple(q.shape)}")
    num_splits = max(1, min(int(num_splits), s_len))
    split_len = -(-s_len // num_splits)
    seg = _dec.packed_segment(packed_k, packed_v, batched=False, splits=num_splits,
                              split_len=split_len)
    return _dec.fused_decode(_dec.Problem(q, [seg], num_attention_heads))[0]


def _packed_layer_partial(q, packed_k, packed_v, num_attention_heads, num_splits, block_n):
    """(m, l, acc) of one per-token packed tier (``attention_triton.py:279-282``)."""
    pm, pl, pacc = _packed_split_launch(q, packed_k, packed_v, num_attention_heads, num_splits,
                                        block_n)
    return _reduce_splits(pm, pl, pacc)


def _fp16_layer_partial(q, hot_k, hot_v, num_attention_heads):
    """(m, l, acc) of the FP16 hot tier ``[Hkv, hot, hd]`` (``attention_triton.py:285-297``).

    The hot views are read in place through their strides (no GQA-expanded copies).
    """
    seg = _dec.fp16_segment(hot_k, hot_v, batched=False)
    return _dec.decode_mlacc(_dec.Problem(q, [seg], num_attention_heads))


def _merge_partials(partials):
    """Cross-segment merge of (m, l, acc) partials -> ``[Hq, hd]`` fp16 (``attention_triton.py:300-307``)."""
    if not partials:
        raise ValueError("no partials to merge")
    ms = torch.stack([p[0] for p in partials], dim=1)
    ls = torch.stack([p[1] for p in partials], dim=1)
    accs = torch.stack([p[2] for p in partials], dim=1)
    return _dec.merge_partials(ms, ls, accs, normalize=True)


# ---------------------------------------------------------------------------
# three tiers in the legacy layout (attention_triton.py:310-511)
# ---------------------------------------------------------------------------
def _three_tier_segments(kv, num_splits):
    segs = []
    if kv.prompt_k is not None:
        s_len = kv.prompt_k.orig_shape[1]
        n = max(1, min(int(num_splits), s_len)) if num_splits else 0
        segs.append(_dec.packed_segment(kv.prompt_k, kv.prompt_v, batched=False, splits=n,
                                        split_len=(-(-s_len // n)) if n else 0))
    if kv.cold_k is not None:
        s_len = kv.cold_k.orig_shape[1]
        n = max(1, min(int(num_splits), s_len)) if num_splits else 0
        segs.append(_dec.packed_segment(kv.cold_k, kv.cold_v, batched=False, splits=n,
                                        split_len=(-(-s_len // n)) if n else 0))
    if kv.hot_k is not None and kv.hot_k.shape[1] > 0:
        segs.append(_dec.fp16_segment(kv.hot_k.to(torch.float16), kv.hot_v.to(torch.float16),
                                      batched=False))
    if not segs:
        raise ValueError("all three tiers are empty: nothing to attend")
    return segs


def fused_three_tier_decode(q, kv, num_attention_heads, num_splits: int = 8, block_n: int = 64):
    """Prompt + cold (per-token packed) + FP16 hot attention (``attention_triton.py:487-511``).

    q ``[Hq, hd]`` fp16; kv is a ``reference.ThreeTierKV`` with ``[Hkv, len, hd]`` tiers.
    One launch; each packed tier is cut into ``num_splits`` splits as in the reference.
    """
    segs = _three_tier_segments(kv, num_splits)
    return _dec.fused_decode(_dec.Problem(q, segs, num_attention_heads))[0]


def fused_three_tier_decode_single(q, kv, num_attention_heads, num_splits: int = 32,
                                   block_n: int = 64):
    """Single-launch three-tier decode (``attention_triton.py:414-484``).

    The reference's single launch predicates every tier's loads per token; here
    each workgroup owns one tier's chunk, so the launch carries no cross-tier
    redundancy.  Splits are chosen by the MI355X planner.
    """
    segs = _three_tier_segments(kv, 0)
    return _dec.fused_decode(_dec.Problem(q, segs, num_attention_heads))[0]


# ---------------------------------------------------------------------------
# production KIVI path (attention_triton.py:514-669)
# ---------------------------------------------------------------------------
def _kivi_layer_partial(q, key: PackedTensor, value: PackedTensor, num_attention_heads: int,
                        num_splits: int | None = None, block_n: int | None = None,
                        num_warps: int | None = None):
    """(m, l, acc) of one batch-stripped KIVI segment (``attention_triton.py:604-639``)."""
    if key.axis != 1 or value.axis != 2 or len(key.orig_shape) != 3:
        raise ValueError("K must be packed along tokens and V along head_dim, batch removed")
    hkv, seq_len, head_dim = key.orig_shape
    if tuple(value.orig_shape) != tuple(key.orig_shape) or seq_len <= 0:
        raise ValueError("packed K/V shapes differ or the segment is empty")
    if q.shape != (num_attention_heads, head_dim) or q.dtype != torch.float16:
        raise ValueError("query must be [Hq, head_dim] float16")
    if num_attention_heads % hkv or head_dim & (head_dim - 1):
        raise ValueError("Hq must be a multiple of Hkv and head_dim a power of two")
    if q.device != key.packed.device or q.device != value.packed.device:
        raise ValueError("query and packed K/V must be on the same device")
    splits, split_len = _override_plan(seq_len, num_attention_heads, head_dim, q.device,
                                       num_splits, block_n, num_warps)
    seg = _dec.packed_segment(key, value, batched=False, splits=splits, split_len=split_len)
    return _dec.decode_mlacc(_dec.Problem(q, [seg], num_attention_heads))


def _remove_batch(pt: PackedTensor) -> PackedTensor:
    if pt.orig_shape[0] != 1:
        raise ValueError("the PhaseKV decode path takes batch = 1 (use fused_phasekv_decode_batched)")
    return replace(pt, packed=pt.packed[0], scale=pt.scale[0], mins=pt.mins[0],
                   orig_shape=tuple(pt.orig_shape[1:]), axis=pt.axis - 1)


def _kivi_segment(segment, splits: int, split_len: int) -> _dec.Segment:
    """The decode segment of a batch-1 ``PackedKVSegment``, built once per segment object
    (packed segments do not change after they are made) and per launch override."""
    hit = getattr(segment, "_pk_decode_segment", None)
    if (hit is not None and hit[0] == (splits, split_len) and hit[1] is segment.key
            and hit[2] is segment.value):
        return hit[3]
    key, value = _remove_batch(segment.key), _remove_batch(segment.value)
    if key.axis != 1 or value.axis != 2:
        raise ValueError("K must be packed along tokens and V along head_dim")
    seg = _dec.packed_segment(key, value, batched=False, splits=splits, split_len=split_len)
    try:
        segment._pk_decode_segment = ((splits, split_len), segment.key, segment.value, seg)
    except AttributeError:      # a caller's segment type without instance attributes
        pass
    return seg


def _reused_problem(q: torch.Tensor, tiers, num_attention_heads: int) -> _dec.Problem:
    """The batch-1 decode problem of ``tiers``, kept on the tiers object across calls.

    Between cooling events a layer's packed K/V (``PackedTensor`` objects) and its hot
    buffer stay the same objects; a decode step changes only q and the hot window's
    length.  The problem (descriptors, C arrays, device checks) is rebuilt when the
    packed K/V list, the hot buffer or the head count changes; otherwise the call writes
    q's pointer and strides and the hot segment's length into the kept C structure.  The
    launch copies the descriptors into its kernel arguments, so the next call may
    overwrite them.
    """
    segments = [tiers.prompt, *tiers.prompt_extensions, *tiers.cold]
    packed = [t for s in segments for t in (s.key, s.value)]
    hot_len = tiers.hot_len
    hot = (tiers.hot_k, tiers.hot_v) if hot_len else None
    kept = getattr(tiers, "_pk_problem", None)
    if kept is not None:
        k_packed, k_hot, k_hq, problem = kept
        if (k_hq == num_attention_heads and len(k_packed) == len(packed)
                and all(a is b for a, b in zip(k_packed, packed))
                and (k_hot is None) == (hot is None)
                and (hot is None or (k_hot[0] is hot[0] and k_hot[1] is hot[1]))
                and q.dtype == torch.float16 and q.dim() == 2 and q.is_cuda
                and q.get_device() == problem.device.index
                and q.shape[0] == problem.hq and q.shape[1] == problem.hd):
            if q.stride(-1) != 1:
                q = q.contiguous()
            q3 = q.unsqueeze(0)
            problem.q = q3
            problem.c.q = q3.data_ptr()
            problem.c.q_bstride, problem.c.q_hstride = q3.stride(0), q3.stride(1)
            if hot is not None:
                # the hot window is the last segment of the launch's own list
                problem._arr[len(problem.segments) - 1].length = hot_len
                problem.segments[-1].length = hot_len
            return problem
    # a cooling event appends cold segments: the device table of the kept problem is
    # extended in place (one small write launch) instead of written again
    problem = phasekv_problem(q, tiers, num_attention_heads,
                              reuse_table=kept[3].table if kept is not None else None)
    if hot is not None:
        d = problem.segments[-1].desc
        if d.k_data != hot[0].data_ptr() or d.v_data != hot[1].data_ptr():
            return problem      # the hot window was copied, not read in place: no reuse
    try:
        tiers._pk_problem = (packed, hot, num_attention_heads, problem)
    except AttributeError:      # a caller's tiers type without instance attributes
        pass
    return problem


def _with_table(q: torch.Tensor, segs, candidates, num_attention_heads: int,
                reuse_table: _dec.SegmentTable | None = None) -> _dec.Problem:
    """The problem of ``segs``: more segments than one launch's list holds put the eligible
    candidates (the cold segments) into a device segment table, so the partials stay one
    launch whatever the number of cold segments.  A ``reuse_table`` whose entries are a
    prefix of the new table is extended instead of written again."""
    inline, tsegs = _dec.split_for_table(segs, candidates)
    table = None
    if tsegs:
        if (reuse_table is not None and reuse_table.count <= len(tsegs)
                and reuse_table.device == q.device
                and all(a is b for a, b in zip(reuse_table.segments, tsegs))):
            table = reuse_table
        else:
            table = _dec.SegmentTable(q.device, tsegs[0].head_dim, capacity=2 * len(tsegs))
        table.extend(tsegs[table.count:])
    return _dec.Problem(q, inline, num_attention_heads, table=table)


def phasekv_problem(q: torch.Tensor, tiers, num_attention_heads: int, batched: bool = False,
                    prompt_lens: torch.Tensor | None = None, num_splits: int | None = None,
                    block_n: int | None = None, num_warps: int | None = None,
                    reuse_table: _dec.SegmentTable | None = None) -> _dec.Problem:
    """The decode problem (every packed segment + the hot window) of one layer's tiers."""
    segs, cold = [], []
    n_first = 1 + len(tiers.prompt_extensions)
    for i, segment in enumerate([tiers.prompt, *tiers.prompt_extensions, *tiers.cold]):
        cold.append(i >= n_first)
        if batched:
            lens = prompt_lens.to(torch.int32) if (i == 0 and prompt_lens is not None) else None
            segs.append(_dec.packed_segment(segment.key, segment.value, batched=True,
                                            seq_lens=lens))
            continue
        shape = tuple(segment.key.orig_shape)
        if len(shape) != 4:
            raise ValueError("packed K/V must be [1, Hkv, S, hd]")
        splits, split_len = _override_plan(shape[2], num_attention_heads, shape[3], q.device,
                                           num_splits, block_n, num_warps)
        segs.append(_kivi_segment(segment, splits, split_len))
    if tiers.hot_len:
        hot_k, hot_v = tiers.hot_views()
        segs.append(_dec.fp16_segment(hot_k if batched else hot_k[0],
                                      hot_v if batched else hot_v[0], batched=batched))
        cold.append(False)
    return _with_table(q, segs, cold, num_attention_heads, reuse_table)


def fused_phasekv_decode(q: torch.Tensor, tiers, num_attention_heads: int,
                         num_splits: int | None = None, block_n: int | None = None,
                         num_warps: int | None = None) -> torch.Tensor:
    """batch=1 PhaseKV decode attention over every packed segment and the hot window.

    ``tiers`` is ``PhaseKVCache.layer_tiers(i)`` (or any object with ``prompt``,
    ``prompt_extensions``, ``cold``, ``hot_len`` and ``hot_views()``).  q ``[Hq, hd]``
    fp16 -> ``[Hq, hd]`` fp16 (``attention_triton.py:643-669``).
    """
    if num_splits is None and block_n is None and num_warps is None:
        problem = _reused_problem(q, tiers, num_attention_heads)
    else:
        problem = phasekv_problem(q, tiers, num_attention_heads, num_splits=num_splits,
                                  block_n=block_n, num_warps=num_warps)
    return _dec.fused_decode(problem)[0]


def fused_phasekv_decode_batched(q: torch.Tensor, tiers, num_attention_heads: int,
                                 prompt_lens: torch.Tensor | None = None) -> torch.Tensor:
    """Batched PhaseKV decode: q ``[B, Hq, hd]`` over tiers with batch B -> ``[B, Hq, hd]``.

    ``prompt_lens`` (int32 ``[B]`` on the device) gives ragged valid prompt
    lengths; rows are quantized on their own (each row's K groups start at its
    token 0) and padded to the tier's length.  Beyond the reference, which
    takes batch = 1 only.
    """
    return _dec.fused_decode(phasekv_problem(q, tiers, num_attention_heads, batched=True,
                                             prompt_lens=prompt_lens))


# Chunk tokens x context tokens x Hkv x hd from which the input-chunk attention runs
# the packed tiers once with the chunk's queries as heads rather than once per query
# token.  Under graph capture only GPU time counts: the two methods' measured
# crossover on MI355X lies between 1.5e8 and 2.2e8.  An eager call also pays the heads
# form's host work, about 35 us more than the batch form's (a second decode problem,
# the query transpose, two more launches), while a host-bound caller's GPU time hides
# behind its other host work: in an eager 4-layer Qwen2.5-7B-shaped model the heads
# form lost at 1.1e9 (64 tokens over 33K) and won at 2.2e9 (128 tokens over 33K).
CHUNK_HEADS_MIN_WORK = 160_000_000
CHUNK_HEADS_MIN_WORK_EAGER = 1_600_000_000


def fused_phasekv_prompt_chunk_attention(q: torch.Tensor, tiers, num_attention_heads: int,
                                         method: str = "auto") -> torch.Tensor:
    """Causal attention of a whole input chunk over the packed cache, in one pass.

    q ``[T, Hq, hd]`` fp16 holds the chunk's T queries in token order; the chunk's
    K/V are the last T rows of the hot window (``PhaseKVCache.append_prompt_token``).
    Query t attends to every packed segment, the hot rows before the chunk, and the
    chunk's rows 0..t: what the reference's adapter computes with one decode call per
    chunk token (``qwen2_attention.py:100-106``, ``phasekv_cache.py:344-371``).
    Returns ``[T, Hq, hd]`` fp16.

    ``method="heads"``: two partial launches and one merge.  The T queries ride as
    ``T * Hq`` heads (head ``(kv, g, t)``) over the packed segments and the pre-chunk
    hot rows, so each KV chunk is read once per 16 query rows; the chunk's own rows are
    a batch of T over one broadcast segment with ``t + 1`` valid rows for query t; the
    two launches' split partials are merged in one pass.
    ``method="batch"``: one decode launch with the T queries as a batch of T over
    broadcast segments (every tier read once per query token, mostly from the caches)
    and the whole window with ``start + t + 1`` valid rows for query t: fewer launches,
    more reads.  ``"auto"`` takes ``"heads"`` once T * context tokens * Hkv * hd reaches
    ``CHUNK_HEADS_MIN_WORK`` under graph capture, or ``CHUNK_HEADS_MIN_WORK_EAGER`` in an
    eager call, else ``"batch"`` (GPU time on MI355X: at 4.5K context tokens, Hkv 4,
    hd 128 the two tie at T = 64 and heads is 1.5x faster at T = 256; at 33K tokens
    heads wins from T = 16, 1.9x at T = 256; at 544 tokens, Hkv 2, hd 64 batch wins at
    every T up to 256).
    """
    if method not in ("auto", "heads", "batch"):
        raise ValueError("method must be auto, heads or batch")
    if q.dim() != 3 or q.shape[1] != num_attention_heads:
        raise ValueError("q must be [T, Hq, hd] with Hq = num_attention_heads")
    T, hq, hd = q.shape
    hot_len = tiers.hot_len
    if T <= 0 or T > hot_len:
        raise ValueError(f"the chunk's {T} tokens must be the last rows of the hot window "
                         f"(hot_len={hot_len})")
    hot_k, hot_v = tiers.hot_views()
    if hot_k.shape[0] != 1:
        raise ValueError("the PhaseKV prompt chunk path takes batch = 1")
    start = hot_len - T
    if method == "auto":
        context = hot_len + sum(seg.key.orig_shape[-2] for seg in
                                [tiers.prompt, *tiers.prompt_extensions, *tiers.cold])
        work = T * context * hot_k.shape[1] * hd
        bound = (CHUNK_HEADS_MIN_WORK if torch.cuda.is_current_stream_capturing()
                 else CHUNK_HEADS_MIN_WORK_EAGER)
        method = "heads" if work >= bound else "batch"
    if method == "batch":
        packed = [tiers.prompt, *tiers.prompt_extensions, *tiers.cold]
        segs = [_dec.packed_segment(_remove_batch(seg.key), _remove_batch(seg.value),
                                    batched=False, broadcast=T)
                for seg in packed]
        cold = [i > len(tiers.prompt_extensions) for i in range(len(packed))]
        lens = torch.arange(start + 1, start + T + 1, dtype=torch.int32, device=q.device)
        segs.append(_dec.fp16_segment(hot_k[0], hot_v[0], batched=False, seq_lens=lens,
                                      broadcast=T))
        cold.append(False)
        return _dec.fused_decode(_with_table(q.contiguous(), segs, cold, hq))
    # (a) packed tiers and the pre-chunk hot rows, the T queries as heads (kv, g, t)
    packed = [tiers.prompt, *tiers.prompt_extensions, *tiers.cold]
    segs = [_dec.packed_segment(_remove_batch(seg.key), _remove_batch(seg.value), batched=False)
            for seg in packed]
    cold = [i > len(tiers.prompt_extensions) for i in range(len(packed))]
    if start:
        segs.append(_dec.fp16_segment(hot_k[0, :, :start], hot_v[0, :, :start], batched=False))
        cold.append(False)
    q_heads = q.permute(1, 0, 2).reshape(1, hq * T, hd)
    heads = _with_table(q_heads, segs, cold, hq * T)
    # (b) the chunk's own rows, causal: query t sees rows start .. start + t
    lens = torch.arange(1, T + 1, dtype=torch.int32, device=q.device)
    chunk = _dec.fp16_segment(hot_k[0, :, start:], hot_v[0, :, start:], batched=False,
                              seq_lens=lens, broadcast=T)
    causal = _dec.Problem(q, [chunk], hq)
    # one merge of both launches' partials: output row (t, h) is row h * T + t of (a)
    # and row t * hq + h of (b)
    return _dec.merged_partials_decode([(heads, 1, T), (causal, hq, 1)], T, hq)


def dense_fp16_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      num_attention_heads: int) -> torch.Tensor:
    """GQA-aware FP16 decode attention over uncompressed K/V (the dense comparator).

    q ``[Hq, hd]`` or ``[B, Hq, hd]``; k, v ``[Hkv, S, hd]`` or ``[B, Hkv, S, hd]`` fp16.
    """
    batched = q.dim() == 3
    seg = _dec.fp16_segment(k, v, batched=batched)
    out = _dec.fused_decode(_dec.Problem(q, [seg], num_attention_heads))
    return out if batched else out[0]
