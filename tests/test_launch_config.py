"""Known-answer tests of plan_kivi_decode, for the oracle and the product module.

Values from the reference's tests/test_phasekv_launch_config.py:10-47 and the
published plan table docs/idea/PhaseKV-技术原理与系统设计.md:495-502 (46 SMs,
12 query heads, head_dim 128).
"""
import pytest

from oracle.launch_config_oracle import plan_kivi_decode as oracle_plan
from phasekv_amd.kernels.launch_config import plan_kivi_decode as product_plan

PLANS = [oracle_plan, product_plan]

# (length, num_splits, split_len, block_n) from the published table
TABLE = [(128, 16, 8, 8), (512, 16, 32, 8), (2048, 16, 128, 8), (8192, 64, 128, 8),
         (16384, 128, 128, 8), (28672, 128, 224, 8)]


@pytest.mark.parametrize("plan", PLANS)
def test_published_plan_table(plan):
    for length, splits, split_len, block_n in TABLE:
        c = plan(length, 12, 128, 46)
        assert (c.num_splits, c.split_len, c.block_n) == (splits, split_len, block_n)


@pytest.mark.parametrize("plan", PLANS)
def test_boundaries_cover_segment_without_empty_splits(plan):
    for length in (1, 7, 31, 127, 128, 129, 511, 512, 8193, 28672):
        for heads, dim, sms in ((12, 128, 46), (4, 8, 1), (32, 256, 132), (28, 128, 256)):
            c = plan(length, heads, dim, sms)
            assert 1 <= c.num_splits <= 128
            assert (c.num_splits - 1) * c.split_len < length <= c.num_splits * c.split_len
            assert c.split_len % c.block_n == 0
            assert c.block_n * dim <= 1024


@pytest.mark.parametrize("plan", PLANS)
def test_length_and_hardware_change_parallelism(plan):
    assert plan(128, 12, 128, 46).num_splits < plan(8192, 12, 128, 46).num_splits
    assert plan(8192, 12, 128, 46).num_splits < plan(28672, 12, 128, 46).num_splits
    assert plan(512, 12, 128, 16).num_splits < plan(512, 12, 128, 80).num_splits
    assert plan(512, 12, 256, 46).block_n < plan(512, 12, 64, 46).block_n


@pytest.mark.parametrize("plan", PLANS)
def test_overrides_and_uneven_splits(plan):
    c = plan(8192, 12, 128, 46, 8, 64, 4)
    assert (c.num_splits, c.split_len, c.block_n, c.num_warps) == (8, 1024, 64, 4)
    c = plan(10, 12, 128, 46, num_splits=8)
    assert (c.num_splits, c.split_len) == (5, 2)
    assert plan(512, 12, 128, 46, block_n=16).block_n == 16
    assert plan(512, 12, 128, 46, num_warps=8).num_warps == 8
    assert plan(1, 12, 128, 46, num_splits=100).num_splits == 1


@pytest.mark.parametrize("plan", PLANS)
def test_invalid_parameters(plan):
    for kwargs in ({"num_splits": 0}, {"block_n": 0}, {"block_n": 3}, {"num_warps": 3}):
        with pytest.raises(ValueError):
            plan(128, 12, 128, 46, **kwargs)
    with pytest.raises(ValueError):
        plan(0, 12, 128, 46)
    with pytest.raises(ValueError):
        plan(128, 12, 96, 46)


def test_product_equals_oracle_on_a_sweep():
    for length in (1, 5, 33, 100, 1000, 4096, 4480, 32768, 50000):
        for heads in (1, 7, 14, 28, 32):
            for dim in (8, 64, 128, 256):
                for sms in (1, 46, 256, 304):
                    a, b = oracle_plan(length, heads, dim, sms), product_plan(length, heads, dim, sms)
                    assert (a.num_splits, a.split_len, a.block_n, a.num_warps) == \
                           (b.num_splits, b.split_len, b.block_n, b.num_warps)
