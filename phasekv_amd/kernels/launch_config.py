"""Split planning of the packed decode kernel (drop-in for the reference's launch_config.py).

``plan_kivi_decode`` keeps the reference's interface and integer rules
(``src/phasekv/kernels/launch_config.py:22-64``) so callers that pass explicit
``num_splits`` / ``block_n`` / ``num_warps`` overrides get the same split
boundaries.  The HIP path uses it only when an override is given; without
overrides the library's own MI355X planner sizes the splits (chunks of whole
64-token tiles, about four workgroups per CU over all segments of a call).
"""
from dataclasses import dataclass
from functools import lru_cache


@dataclass(frozen=True)
class DecodeLaunchConfig:
    num_splits: int
    split_len: int
    block_n: int
    num_warps: int


def _ceildiv(n: int, d: int) -> int:
    return (n + d - 1) // d


def _next_power_of_two(n: int) -> int:
    return 1 << (n - 1).bit_length()


@lru_cache(maxsize=2048)
def plan_kivi_decode(seq_len: int, num_heads: int, head_dim: int, sm_count: int,
                     num_splits: int | None = None, block_n: int | None = None,
                     num_warps: int | None = None) -> DecodeLaunchConfig:
    """Splits of one packed segment from its length, head shape and device size.

    Tiles hold at most 1024 elements (``block_n * head_dim``, capped at 32
    tokens); the split count starts near four tiles per CU, grows so a split
    holds about 16 tiles, and is capped at 32 per CU and 128 overall.  Split
    boundaries are tile aligned and trailing empty splits are dropped.  Each
    explicit option overrides its own rule only.
    """
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
        largest = max(1, min(32, 1024 // head_dim, seq_len))
        block_n = 1 << (largest.bit_length() - 1)
    if num_warps is None:
        num_warps = min(32, max(4, _next_power_of_two(_ceildiv(block_n * head_dim, 256))))

    if num_splits is None:
        tiles = _ceildiv(seq_len, block_n)
        floor_splits = _ceildiv(4 * sm_count, num_heads)
        cap = min(128, _next_power_of_two(_ceildiv(32 * sm_count, num_heads)))
        chosen = min(tiles, cap, _next_power_of_two(max(floor_splits, _ceildiv(tiles, 16))))
        split_len = _ceildiv(tiles, chosen) * block_n
    else:
        split_len = _ceildiv(seq_len, min(seq_len, num_splits))
    return DecodeLaunchConfig(_ceildiv(seq_len, split_len), split_len, block_n, num_warps)
