"""The device-side input generators equal the oracle's host restatement."""
import numpy as np
import pytest

from oracle import oracle as o

pytestmark = pytest.mark.gpu


def test_generators_match_host(gpu):
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen as dg

    n = 100_003
    assert (g.to_host(dg.reduce_i32(n)) == o.gen("reduce_i32", n, dg.SEED_REDUCE)).all()
    assert (g.to_host(dg.u8_u32(n)) == o.gen("u8_u32", n, dg.SEED_SCAN_U32)).all()
    assert (g.to_host(dg.keys_u32(n)) == o.gen("keys_u32", n, dg.SEED_SORT_U32)).all()
    assert (g.to_host(dg.keys_u32_and3(n)) == o.gen("keys_u32_and3", n, *dg.SEED_SORT_AND3)).all()
    assert (g.to_host(dg.keys_u64_low16(n)) == o.gen("keys_u64_low16", n, dg.SEED_PAIRS_U64)).all()
    assert (g.to_host(dg.keys_u64(n)) == o.words(dg.SEED_PAIRS_U64_FULL, n)).all()
    assert (g.to_host(dg.iota_u32(n)) == np.arange(n, dtype=np.uint32)).all()
    # Box-Muller in double through the device libm: equal after rounding to float32
    # except for rare last-ulp differences of log/cos
    dev = g.to_host(dg.normal_f32(n))
    host = o.gen("normal_f32", n, dg.SEED_SCAN_F32)
    ulps = np.abs(dev.view(np.int32).astype(np.int64) - host.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and (ulps == 0).mean() > 0.999


@pytest.mark.parametrize("n", [4, 2044, 2048, 2052, 1 << 20, (1 << 20) + 4])
def test_copy_probe_copies_exactly(gpu, n):
    """The calibration copy reads and writes exactly n words (guard untouched)."""
    import torch

    import gpu_util as g
    from lc_parallel_primitive_amd import datagen as dg

    src = torch.arange(n + 64, dtype=torch.int32, device="cuda").view(torch.uint32)
    dst = torch.zeros(n + 64, dtype=torch.int32, device="cuda").view(torch.uint32)
    dg.copy_probe(src[:n], dst[:n])
    h = g.to_host(dst.view(torch.int32))
    assert (h[:n] == np.arange(n)).all() and (h[n:] == 0).all()


def test_run_keys_match_host(gpu):
    import gpu_util as g
    from lc_parallel_primitive_amd import datagen as dg

    n = 300_007
    w = o.gen("keys_u32", n, dg.SEED_BY_KEY)
    assert (g.to_host(dg.run_keys_i32(n, 7)) == np.cumsum((w & 127) == 0, dtype=np.int32)).all()


@pytest.mark.parametrize("shape", range(9))
def test_copy_shapes_write_where_stated(gpu, shape):
    """The copy-shape probes (ceilings quoted for the scan and onesweep kernels)
    move every word: shapes 0-3 copy in place, 4-8 write in[i] to the position
    the host restatement gives; the guard past n stays untouched."""
    import torch

    import gpu_util as g
    from lc_parallel_primitive_amd import datagen as dg

    n = 20480 * 100 if shape in (1, 2) else 1 << 21  # 128 onesweep tiles: one full XCD group of 16-runs
    src = torch.arange(n + 64, dtype=torch.int32, device="cuda").view(torch.uint32)
    dst = torch.full((n + 64,), -1, dtype=torch.int32, device="cuda").view(torch.uint32)
    dg.copy_shape(src[:n], dst[:n], shape)
    h = g.to_host(dst.view(torch.int32))
    assert (h[n:] == -1).all()
    if shape <= 3:
        assert (h[:n] == np.arange(n)).all()
    else:
        expect = np.empty(n, dtype=np.int32)
        expect[dg.copy_shape_positions(n, shape)] = np.arange(n, dtype=np.int32)
        assert (h[:n] == expect).all()
