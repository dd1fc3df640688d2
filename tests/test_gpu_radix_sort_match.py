"""The onesweep's ballot-match ranking (stable by construction), forced with
lcpp_test_set_sort_rank_path(2): the sort parity cases of
test_gpu_radix_sort.py (keys, pairs, descending, special floats, look-back
batch boundaries, skewed and constant digits, skipped passes, and the
full-size C3a / C3b / C4 configurations) run again on it.  Which path the
sorts take by default is the first-use lane-order probe's choice
(lcpp_radix_sort_rank_path)."""
import pytest

from conftest import log
from test_gpu_radix_sort import (  # noqa: F401  (collected here with the match path forced)
    test_constant_keys_all_lanes_hot,
    test_full_size_pairs_u64_descending,
    test_full_size_pairs_u64_full_range_8_passes,
    test_full_size_pairs_u64_index,
    test_full_size_u32,
    test_full_size_u32_descending,
    test_kat_float_keys_golden,
    test_kat_pairs_descending_golden,
    test_kat_pairs_golden,
    test_kat_reversed_keys,
    test_keys_descending_vs_oracle,
    test_keys_vs_oracle,
    test_lookback_batch_boundaries,
    test_low_entropy_keys,
    test_pairs_descending_stable_vs_oracle,
    test_pairs_stable_vs_oracle,
    test_skewed_digits_stable,
    test_special_float_keys_vs_oracle,
    test_trivial_passes_skipped,
)

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def match_path(gpu):
    import lc_parallel_primitive_amd as lcpp

    L = lcpp.lib()
    assert L.lcpp_test_set_sort_rank_path(2) == 0
    yield
    assert L.lcpp_test_set_sort_rank_path(0) == 0


def test_rank_path_query_and_override(gpu):
    import ctypes

    import lc_parallel_primitive_amd as lcpp

    L = lcpp.lib()
    path = ctypes.c_int(0)
    for mode in (1, 2):
        assert L.lcpp_test_set_sort_rank_path(mode) == 0
        assert L.lcpp_radix_sort_rank_path(ctypes.byref(path)) == 0 and path.value == mode
    assert L.lcpp_test_set_sort_rank_path(0) == 0
    assert L.lcpp_radix_sort_rank_path(ctypes.byref(path)) == 0 and path.value in (1, 2)
    log(f"default onesweep rank path on this device: {'LDS atomics' if path.value == 1 else 'ballot match'}")
