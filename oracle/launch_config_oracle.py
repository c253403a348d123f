"""Integer restatement of the reference's split planner.

Test infrastructure only (see ``oracle/__init__.py``).  Follows
``src/phasekv/kernels/launch_config.py:22-64`` step by step.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Plan:
    num_splits: int
    split_len: int
    block_n: int
    num_warps: int


def _cdiv(n: int, d: int) -> int:
    return -(-n // d)


def _pow2_ceil(n: int) -> int:
    p = 1
    while p < n:
        p *= 2
    return p


def _pow2_floor(n: int) -> int:
    p = 1
    while p * 2 <= n:
        p *= 2
    return p


def plan_kivi_decode(seq_len, num_heads, head_dim, sm_count,
                     num_splits=None, block_n=None, num_warps=None) -> Plan:
    if min(seq_len, num_heads, head_dim, sm_count) <= 0:
        raise ValueError("sequence, heads, head_dim and SM count must be positive")
    if head_dim & (head_dim - 1):
        raise ValueError("head_dim must be a power of two")
    if num_splits is not None and num_splits <= 0:
        raise ValueError("num_splits must be positive")
    if block_n is not None and (block_n <= 0 or block_n & (block_n - 1)):
        raise ValueError("block_n must be a positive power of two")
    if num_warps is not None and num_warps not in (1, 2, 4, 8, 16, 32):
        raise ValueError("num_warps must be one of 1, 2, 4, 8, 16, 32")
    if block_n is None:
        block_n = _pow2_floor(max(1, min(32, 1024 // head_dim, seq_len)))
    if num_warps is None:
        num_warps = min(32, max(4, _pow2_ceil(_cdiv(block_n * head_dim, 256))))
    if num_splits is None:
        tiles = _cdiv(seq_len, block_n)
        base = _cdiv(4 * sm_count, num_heads)
        limit = min(128, _pow2_ceil(_cdiv(32 * sm_count, num_heads)))
        want = min(tiles, limit, _pow2_ceil(max(base, _cdiv(tiles, 16))))
        split_len = _cdiv(tiles, want) * block_n
    else:
        split_len = _cdiv(seq_len, min(seq_len, num_splits))
    return Plan(_cdiv(seq_len, split_len), split_len, block_n, num_warps)
