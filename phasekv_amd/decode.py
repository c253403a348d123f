"""Host side of the decode path: tensors -> C-ABI segment descriptors -> HIP launches.

The drop-in ``kernels.attention_triton`` module and the bench build their calls
from these helpers.  Segment kinds:

* KIVI  — a ``PackedKVSegment`` of the cache: K packed per channel along tokens
  (``quantize_pack(K, bits, axis=-2)``), V packed per token along head_dim
  (``axis=-1``), ``src/phasekv/phasekv_cache.py:101-107``.
* TOKEN — legacy layout, K and V both packed per token
  (``scripts/bench_decode_kernel.py:82-83`` of the reference).
* FP16  — uncompressed fp16 K/V, e.g. the hot window views
  (``src/phasekv/phasekv_cache.py:75-79``), which are strided over the buffer
  capacity and are read in place.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from . import _lib


def _inner_contiguous(t: torch.Tensor) -> torch.Tensor:
    """Return ``t`` if its two innermost dims are dense, else a contiguous copy."""
    if t.dim() >= 2 and t.stride(-1) == 1 and (t.shape[-2] <= 1 or t.stride(-2) == t.shape[-1]):
        return t
    if t.dim() == 1 and t.stride(-1) == 1:
        return t
    return t.contiguous()


def _group_major(t: torch.Tensor) -> bool:
    """``t`` [..., D, n] is the transposed view of dense [..., n, D] storage."""
    if t.dim() < 2:
        return False
    d, g = t.shape[-2], t.shape[-1]
    return d > 1 and t.stride(-2) == 1 and (g <= 1 or t.stride(-1) == d)


def _bh_strides(t: torch.Tensor, batched: bool) -> Tuple[int, int]:
    """(batch stride, head stride) in elements of a [B, H, ...] or [H, ...] tensor."""
    if batched:
        return t.stride(0), t.stride(1)
    return 0, t.stride(0)


class Segment:
    """One C-ABI segment plus the tensors it points to (kept alive by this object)."""

    def __init__(self, desc: _lib.PkSegment, keep: Sequence[torch.Tensor], length: int,
                 num_kv_heads: int, head_dim: int, batch: int, device: torch.device):
        self.desc = desc
        self.keep = list(keep)
        self.length = length
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.batch = batch
        self.device = device


def packed_segment(key, value, *, batched: bool, splits: int = 0, split_len: int = 0,
                   seq_lens: Optional[torch.Tensor] = None,
                   broadcast: Optional[int] = None) -> Segment:
    """Segment from a K/V pair of ``PackedTensor`` (KIVI or legacy per-token layout).

    ``batched``: orig_shape is [B, Hkv, S, hd] (else [Hkv, S, hd]).  ``broadcast``: an
    unbatched segment serves every one of this many batch rows (batch stride 0).
    """
    nd = 4 if batched else 3
    if len(key.orig_shape) != nd or tuple(value.orig_shape) != tuple(key.orig_shape):
        raise ValueError("packed K/V must share one [B, Hkv, S, hd] (or [Hkv, S, hd]) shape")
    tok_axis, dim_axis = nd - 2, nd - 1
    if value.axis != dim_axis:
        raise ValueError("V must be packed along head_dim (per token)")
    if key.axis == tok_axis:
        kind = _lib.PK_SEG_KIVI
    elif key.axis == dim_axis:
        kind = _lib.PK_SEG_TOKEN
    else:
        raise ValueError("K must be packed along tokens (KIVI) or head_dim (per token)")
    shape = tuple(key.orig_shape)
    batch = shape[0] if batched else (broadcast or 1)
    hkv, s_len, hd = shape[-3], shape[-2], shape[-1]
    if s_len <= 0:
        raise ValueError("packed K/V segment is empty")
    dev = _lib.require_device(key.packed, key.scale, key.mins, value.packed, value.scale,
                              value.mins)
    if kind == _lib.PK_SEG_KIVI and _group_major(key.packed):
        kp, data_layout = key.packed, _lib.PK_CODES_TOKEN_MAJOR
    else:
        kp, data_layout = _inner_contiguous(key.packed), _lib.PK_CODES_CHANNEL_MAJOR
    if kind == _lib.PK_SEG_KIVI and _group_major(key.scale) and _group_major(key.mins) \
            and key.scale.stride() == key.mins.stride():
        ks, km, meta_layout = key.scale, key.mins, _lib.PK_META_GROUP_MAJOR
    else:
        ks, km = (_inner_contiguous(t) for t in (key.scale, key.mins))
        meta_layout = _lib.PK_META_CHANNEL_MAJOR
    vp, vs, vm = (_inner_contiguous(t) for t in (value.packed, value.scale, value.mins))
    if ks.stride() != km.stride() or vs.stride() != vm.stride():
        ks, km, vs, vm = ks.contiguous(), km.contiguous(), vs.contiguous(), vm.contiguous()
        meta_layout = _lib.PK_META_CHANNEL_MAJOR
    d = _lib.PkSegment()
    d.kind = kind
    d.length = s_len
    d.k_bits, d.v_bits = key.bits, value.bits
    d.k_group, d.v_group = key.group_size, value.group_size
    d.splits, d.split_len = int(splits), int(split_len)
    d.k_meta_layout, d.k_data_layout = meta_layout, data_layout
    d.seq_lens = 0 if seq_lens is None else seq_lens.data_ptr()
    d.k_data, d.k_scale, d.k_mins = kp.data_ptr(), ks.data_ptr(), km.data_ptr()
    d.v_data, d.v_scale, d.v_mins = vp.data_ptr(), vs.data_ptr(), vm.data_ptr()
    d.k_data_bstride, d.k_data_hstride = _bh_strides(kp, batched)
    d.k_meta_bstride, d.k_meta_hstride = _bh_strides(ks, batched)
    d.v_data_bstride, d.v_data_hstride = _bh_strides(vp, batched)
    d.v_meta_bstride, d.v_meta_hstride = _bh_strides(vs, batched)
    d.tok_stride = 0
    keep = [kp, ks, km, vp, vs, vm] + ([seq_lens] if seq_lens is not None else [])
    return Segment(d, keep, s_len, hkv, hd, batch, dev)


def fp16_segment(k: torch.Tensor, v: torch.Tensor, *, batched: bool, splits: int = 0,
                 split_len: int = 0, seq_lens: Optional[torch.Tensor] = None,
                 broadcast: Optional[int] = None) -> Segment:
    """Segment over uncompressed fp16 K/V [B, Hkv, S, hd] (or [Hkv, S, hd]), read in place.

    ``broadcast``: an unbatched segment serves every one of this many batch rows.
    """
    nd = 4 if batched else 3
    if k.dim() != nd or k.shape != v.shape:
        raise ValueError("fp16 K/V must share one [B, Hkv, S, hd] (or [Hkv, S, hd]) shape")
    if k.dtype != torch.float16 or v.dtype != torch.float16:
        raise ValueError("hot K/V must be float16")
    dev = _lib.require_device(k, v)
    if k.stride(-1) != 1 or v.stride(-1) != 1 or k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    batch = k.shape[0] if batched else (broadcast or 1)
    hkv, s_len, hd = k.shape[-3], k.shape[-2], k.shape[-1]
    if s_len <= 0:
        raise ValueError("fp16 segment is empty")
    d = _lib.PkSegment()
    d.kind = _lib.PK_SEG_FP16
    d.length = s_len
    d.splits, d.split_len = int(splits), int(split_len)
    d.seq_lens = 0 if seq_lens is None else seq_lens.data_ptr()
    d.k_data, d.v_data = k.data_ptr(), v.data_ptr()
    d.k_data_bstride, d.k_data_hstride = _bh_strides(k, batched)
    d.v_data_bstride, d.v_data_hstride = _bh_strides(v, batched)
    d.tok_stride = k.stride(-2)
    keep = [k, v] + ([seq_lens] if seq_lens is not None else [])
    return Segment(d, keep, s_len, hkv, hd, batch, dev)


# Segments longer than this stay in the launch's own segment list: a table segment is
# read whole by one wave, which suits the short cold segments of lazy cooling.
TABLE_MAX_TOKENS = 128


def table_eligible(seg: Segment) -> bool:
    """Whether ``pk_segment_table_write`` takes this segment (see include/phasekv_hip.h):
    a KIVI segment of 2/4-bit codes in the storage ``quantize_pack`` writes, with aligned
    rows, at head_dim 64 / 128 and at most ``TABLE_MAX_TOKENS`` tokens."""
    d = seg.desc
    if d.kind != _lib.PK_SEG_KIVI or seg.head_dim not in (64, 128):
        return False
    if d.k_bits not in (2, 4) or d.v_bits not in (2, 4) or d.splits or d.split_len:
        return False
    if d.length > TABLE_MAX_TOKENS:
        return False
    if (d.k_data_layout != _lib.PK_CODES_TOKEN_MAJOR
            or d.k_meta_layout != _lib.PK_META_GROUP_MAJOR):
        return False
    if not (d.k_group == 32 or (d.length <= 32 and d.k_group >= d.length)) or d.v_group != 32:
        return False
    vma = seg.head_dim // 32
    return (d.k_data % 16 == 0 and d.k_data_bstride % 16 == 0 and d.k_data_hstride % 16 == 0
            and d.k_scale % 8 == 0 and d.k_mins % 8 == 0 and d.k_meta_bstride % 4 == 0
            and d.k_meta_hstride % 4 == 0 and d.v_data % 16 == 0 and d.v_data_bstride % 16 == 0
            and d.v_data_hstride % 16 == 0 and d.v_scale % (2 * vma) == 0
            and d.v_mins % (2 * vma) == 0 and d.v_meta_bstride % vma == 0
            and d.v_meta_hstride % vma == 0)


class SegmentTable:
    """Segment descriptors in device memory (``pk_segment_table_write``), appended to as
    the cache grows, so that a decode over any number of them is one partials launch.

    The entries are written on the current stream by a small kernel; decode launches
    ordered after it read them.  ``segments`` keeps the described tensors alive."""

    def __init__(self, device: torch.device, head_dim: int, capacity: int = 64):
        self.device = device
        self.head_dim = head_dim
        self.entry_bytes = int(_lib.load().pk_segment_table_entry_bytes())
        self.buf = torch.empty(max(1, capacity) * self.entry_bytes, dtype=torch.uint8,
                               device=device)
        self.segments: List[Segment] = []
        self.bits = 0

    @property
    def count(self) -> int:
        return len(self.segments)

    def _write(self, first: int, segs: Sequence[Segment]) -> None:
        if not segs:
            return
        arr = (_lib.PkSegment * len(segs))(*[sg.desc for sg in segs])
        _lib.check(_lib.load().pk_segment_table_write(
            self.buf.data_ptr(), first, len(segs), arr, self.head_dim,
            _lib.stream_ptr(self.device)), "segment_table_write")

    def extend(self, segs: Sequence[Segment]) -> None:
        """Append entries for ``segs`` (each must be ``table_eligible``)."""
        for sg in segs:
            if not table_eligible(sg) or sg.head_dim != self.head_dim:
                raise ValueError("segment not eligible for a device segment table")
        need = (self.count + len(segs)) * self.entry_bytes
        if need > self.buf.numel():
            # a larger table: every entry is written again into it
            self.buf = torch.empty(max(need, 2 * self.buf.numel()), dtype=torch.uint8,
                                   device=self.device)
            self._write(0, self.segments)
        self._write(self.count, segs)
        self.segments.extend(segs)
        for sg in segs:
            self.bits = max(self.bits, sg.desc.k_bits, sg.desc.v_bits)


def split_for_table(segments: List[Segment], candidates: Sequence[bool]):
    """(inline, table) segments: when the list is longer than one launch's segment list,
    the eligible candidates (cold segments) go to a device table, the rest stay inline."""
    if len(segments) <= _lib.PK_MAX_SEGMENTS_PER_LAUNCH:
        return list(segments), []
    inline, table = [], []
    for sg, cand in zip(segments, candidates):
        (table if cand and table_eligible(sg) else inline).append(sg)
    if len(table) < 2:
        return list(segments), []
    return inline, table


class Problem:
    """A decode problem (q, its segment list and an optional device segment table) as the
    C structure, with its keep-alive list."""

    def __init__(self, q: torch.Tensor, segments: List[Segment], num_attention_heads: int,
                 generic_kernel: bool = False, table: Optional[SegmentTable] = None,
                 require_mfma: bool = False):
        if not segments and (table is None or table.count == 0):
            raise ValueError("no KV to attend: every tier is empty")
        if q.dim() == 2:
            q = q.unsqueeze(0)
        if q.dim() != 3:
            raise ValueError("query must be [Hq, hd] or [B, Hq, hd]")
        if q.dtype != torch.float16:
            raise ValueError("query must be float16")
        batch, hq, hd = q.shape
        if hq != num_attention_heads:
            raise ValueError(f"query has {hq} heads, expected {num_attention_heads}")
        dev = _lib.require_device(q, *[t for s in segments for t in s.keep])
        all_segs = list(segments) + (list(table.segments) if table is not None else [])
        hkv = all_segs[0].num_kv_heads
        for s in all_segs:
            if s.num_kv_heads != hkv or s.head_dim != hd:
                raise ValueError("segments must share kv heads and head_dim with the query")
            if s.batch != batch:
                raise ValueError("segments and query must share the batch size")
        if hq % hkv:
            raise ValueError(f"Hq {hq} must be a multiple of Hkv {hkv}")
        if q.stride(-1) != 1:
            q = q.contiguous()
        if table is not None and table.device != dev:
            raise ValueError("the segment table lives on another device")
        self.q = q
        self.segments = segments
        self.table = table
        self.device = dev
        self.batch, self.hq, self.hkv, self.hd = batch, hq, hkv, hd
        arr = (_lib.PkSegment * max(1, len(segments)))(*[s.desc for s in segments])
        self._arr = arr
        p = _lib.PkDecodeProblem()
        p.batch, p.num_q_heads, p.num_kv_heads, p.head_dim = batch, hq, hkv, hd
        p.q = q.data_ptr()
        p.q_bstride, p.q_hstride = q.stride(0), q.stride(1)
        p.segments = ctypes.cast(arr, ctypes.POINTER(_lib.PkSegment))
        p.num_segments = len(segments)
        if generic_kernel and require_mfma:
            raise ValueError("generic_kernel and require_mfma exclude each other")
        p.flags = (_lib.PK_FLAG_GENERIC_KERNEL if generic_kernel else 0) | \
            (_lib.PK_FLAG_REQUIRE_MFMA if require_mfma else 0)
        if table is not None and table.count:
            p.table = table.buf.data_ptr()
            p.table_count = table.count
            p.table_bits = table.bits
        self.c = p

    def workspace_size(self) -> Tuple[int, int]:
        lib = _lib.load()
        nbytes = ctypes.c_size_t(0)
        splits = ctypes.c_int32(0)
        _lib.check(lib.pk_decode_workspace_size(ctypes.byref(self.c), ctypes.byref(nbytes),
                                                ctypes.byref(splits)), "decode_workspace_size")
        return nbytes.value, splits.value


# Reusable workspaces per (device, stream): calls on one stream are ordered, so
# they can share one buffer.
_WORKSPACES: Dict[Tuple[int, int], torch.Tensor] = {}


def cached_workspace(device: torch.device, nbytes: int,
                     stream: Optional[int] = None) -> torch.Tensor:
    if stream is None:
        stream = _lib.stream_ptr(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            # a buffer allocated under capture belongs to the graph's pool: keep it for
            # this call only, so a later, larger call cannot free memory a graph reads
            return torch.empty(nbytes, dtype=torch.uint8, device=device)
        size = max(nbytes + nbytes // 2, 4 << 20)
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def fused_decode(problem: Problem) -> torch.Tensor:
    """Normalized attention output [B, Hq, hd] fp16: one partial launch (per 8 segments) + combine."""
    nbytes, _ = problem.workspace_size()
    stream = _lib.stream_ptr(problem.device)
    ws = cached_workspace(problem.device, nbytes, stream)
    out = torch.empty(problem.batch, problem.hq, problem.hd, dtype=torch.float16,
                      device=problem.device)
    _lib.check(_lib.load().pk_fused_decode(ctypes.byref(problem.c), ws.data_ptr(), ws.numel(),
                                           out.data_ptr(), stream), "fused_decode")
    return out


def launch_partials(problem: Problem) -> None:
    """Only the split-partials launch, into the cached workspace (for timing the kernel)."""
    nbytes, _ = problem.workspace_size()
    ws = cached_workspace(problem.device, nbytes)
    _lib.check(_lib.load().pk_decode_partials(ctypes.byref(problem.c), ws.data_ptr(), ws.numel(),
                                              _lib.stream_ptr(problem.device)), "decode_partials")


def decode_partials(problem: Problem):
    """Raw split partials: (pm [B*Hq, C], pl [B*Hq, C], pacc [B*Hq, C, hd]) in a fresh buffer."""
    nbytes, splits = problem.workspace_size()
    ws = torch.empty(nbytes, dtype=torch.uint8, device=problem.device)
    lib = _lib.load()
    _lib.check(lib.pk_decode_partials(ctypes.byref(problem.c), ws.data_ptr(), ws.numel(),
                                      _lib.stream_ptr(problem.device)), "decode_partials")
    rows = problem.batch * problem.hq
    off_m = 0
    align = lambda x: (x + 255) & ~255
    off_l = align(off_m + rows * splits * 4)
    off_acc = align(off_l + rows * splits * 4)
    pm = ws[off_m:off_m + rows * splits * 4].view(torch.float32).view(rows, splits)
    pl = ws[off_l:off_l + rows * splits * 4].view(torch.float32).view(rows, splits)
    pacc = ws[off_acc:off_acc + rows * splits * problem.hd * 4].view(torch.float32)
    return pm, pl, pacc.view(rows, splits, problem.hd)


def decode_mlacc(problem: Problem):
    """Merged but unnormalized (m [B*Hq], l [B*Hq], acc [B*Hq, hd]) fp32."""
    nbytes, _ = problem.workspace_size()
    ws = cached_workspace(problem.device, nbytes)
    rows = problem.batch * problem.hq
    m = torch.empty(rows, dtype=torch.float32, device=problem.device)
    l = torch.empty(rows, dtype=torch.float32, device=problem.device)
    acc = torch.empty(rows, problem.hd, dtype=torch.float32, device=problem.device)
    lib = _lib.load()
    stream = _lib.stream_ptr(problem.device)
    _lib.check(lib.pk_decode_partials(ctypes.byref(problem.c), ws.data_ptr(), ws.numel(), stream),
               "decode_partials")
    _lib.check(lib.pk_decode_combine(ctypes.byref(problem.c), ws.data_ptr(), None, m.data_ptr(),
                                     l.data_ptr(), acc.data_ptr(), stream), "decode_combine")
    return m, l, acc


def merged_partials_decode(parts, outer: int, inner: int) -> torch.Tensor:
    """Split partials of several decode problems, merged per output row (o, i) in one pass.

    ``parts`` holds ``(problem, outer_stride, inner_stride)``: output row (o, i) reads
    row ``o * outer_stride + i * inner_stride`` of each problem's ``B * Hq`` partial
    rows.  The partials share the per-stream workspace (one launch per problem, then
    ``pk_merge_partial_sets``); returns fp16 ``[outer, inner, hd]``.
    """
    if not 1 <= len(parts) <= _lib.PK_MAX_PARTIAL_SETS:
        raise ValueError(f"between 1 and {_lib.PK_MAX_PARTIAL_SETS} problems")
    dev, hd = parts[0][0].device, parts[0][0].hd
    align = lambda x: (x + 255) & ~255
    sizes, offs, total = [], [], 0
    for problem, _, _ in parts:
        if problem.device != dev or problem.hd != hd:
            raise ValueError("the problems must share the device and head_dim")
        nbytes, splits = problem.workspace_size()
        sizes.append((nbytes, splits))
        offs.append(total)
        total = align(total + nbytes)
    stream = _lib.stream_ptr(dev)
    ws = cached_workspace(dev, total, stream)     # held until every launch is enqueued
    base = ws.data_ptr()
    lib = _lib.load()
    sets = (_lib.PkPartialSet * len(parts))()
    for k, ((problem, so, si), (nbytes, splits), off) in enumerate(zip(parts, sizes, offs)):
        _lib.check(lib.pk_decode_partials(ctypes.byref(problem.c), base + off, nbytes, stream),
                   "decode_partials")
        rows = problem.batch * problem.hq
        off_l = align(rows * splits * 4)              # the layout decode_partials reads back
        off_acc = align(off_l + rows * splits * 4)
        sets[k] = _lib.PkPartialSet(base + off, base + off + off_l, base + off + off_acc, rows,
                                    splits, 0, so, si)
    out = torch.empty(outer, inner, hd, dtype=torch.float16, device=dev)
    _lib.check(lib.pk_merge_partial_sets(sets, len(parts), outer, inner, hd, out.data_ptr(),
                                         None, None, None, stream), "merge_partial_sets")
    return out


def merge_partial_sets(sets, outer: int, inner: int, normalize: bool = True):
    """Log-sum-exp merge of every partial of several sets per output row (o, i).

    ``sets`` holds ``((m, l, acc), outer_stride, inner_stride)`` with m, l ``[rows, n]``
    and acc ``[rows, n, hd]`` fp32 contiguous (as :func:`decode_partials` returns
    them); output row (o, i) reads row ``o * outer_stride + i * inner_stride`` of each
    set.  Returns fp16 ``[outer, inner, hd]``, or unnormalized (m, l, acc) of
    ``[outer * inner]`` rows when ``normalize`` is False.
    """
    if not 1 <= len(sets) <= _lib.PK_MAX_PARTIAL_SETS:
        raise ValueError(f"between 1 and {_lib.PK_MAX_PARTIAL_SETS} partial sets")
    arr = (_lib.PkPartialSet * len(sets))()
    keep, hd = [], None
    for k, ((m, l, acc), so, si) in enumerate(sets):
        _lib.require_device(m, l, acc)
        if m.dtype != torch.float32 or l.dtype != torch.float32 or acc.dtype != torch.float32:
            raise ValueError("partials must be float32")
        if m.dim() != 2 or l.shape != m.shape or acc.dim() != 3 or acc.shape[:2] != m.shape:
            raise ValueError("partials must be m, l [rows, n] and acc [rows, n, hd]")
        if not (m.is_contiguous() and l.is_contiguous() and acc.is_contiguous()):
            raise ValueError("partials must be contiguous")
        if hd is not None and acc.shape[2] != hd:
            raise ValueError("every set must have the same head_dim")
        hd = acc.shape[2]
        keep += [m, l, acc]
        arr[k] = _lib.PkPartialSet(m.data_ptr(), l.data_ptr(), acc.data_ptr(), m.shape[0],
                                   m.shape[1], 0, so, si)
    dev = _lib.require_device(*keep)
    lib = _lib.load()
    stream = _lib.stream_ptr(dev)
    if normalize:
        out = torch.empty(outer, inner, hd, dtype=torch.float16, device=dev)
        _lib.check(lib.pk_merge_partial_sets(arr, len(sets), outer, inner, hd, out.data_ptr(),
                                             None, None, None, stream), "merge_partial_sets")
        return out
    om = torch.empty(outer * inner, dtype=torch.float32, device=dev)
    ol = torch.empty(outer * inner, dtype=torch.float32, device=dev)
    oacc = torch.empty(outer * inner, hd, dtype=torch.float32, device=dev)
    _lib.check(lib.pk_merge_partial_sets(arr, len(sets), outer, inner, hd, None, om.data_ptr(),
                                         ol.data_ptr(), oacc.data_ptr(), stream),
               "merge_partial_sets")
    return om, ol, oacc


def merge_partials(m: torch.Tensor, l: torch.Tensor, acc: torch.Tensor, normalize: bool):
    """Log-sum-exp merge over dim 1 of m, l [rows, n] and acc [rows, n, hd] (fp32)."""
    dev = _lib.require_device(m, l, acc)
    m = m.float().contiguous()
    l = l.float().contiguous()
    acc = acc.float().contiguous()
    rows, n = m.shape
    hd = acc.shape[-1]
    lib = _lib.load()
    stream = _lib.stream_ptr(dev)
    if normalize:
        out = torch.empty(rows, hd, dtype=torch.float16, device=dev)
        _lib.check(lib.pk_merge_partials(m.data_ptr(), l.data_ptr(), acc.data_ptr(), rows, n, hd,
                                         out.data_ptr(), None, None, None, stream),
                   "merge_partials")
        return out
    om = torch.empty(rows, dtype=torch.float32, device=dev)
    ol = torch.empty(rows, dtype=torch.float32, device=dev)
    oacc = torch.empty(rows, hd, dtype=torch.float32, device=dev)
    _lib.check(lib.pk_merge_partials(m.data_ptr(), l.data_ptr(), acc.data_ptr(), rows, n, hd,
                                     None, om.data_ptr(), ol.data_ptr(), oacc.data_ptr(), stream),
               "merge_partials")
    return om, ol, oacc
