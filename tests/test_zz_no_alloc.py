"""The allocation-free W4A8 entry point (rai_w4a8_matmul_noalloc_dev) against
rai_w4a8_matmul_dev, through the C ABI: bit-identical outputs on two calls in
a row on the same device buffers, the second with fewer tokens and a smaller
matrix (the shared scratch keeps the first call's contents), the matrix-core
verify path, the matrix-core GEMM past 64 tokens, the one-token path, and
the size limit."""
import ctypes

import numpy as np
import pytest

from rai_amd.workload import gemv_operands

pytestmark = pytest.mark.gpu


def _run(rai, fn, nib, params, x, rows, cols, m, gs):
    L = rai.lib()
    dn, dp, dx = rai.DeviceArray.from_host(nib), rai.DeviceArray.from_host(params), rai.DeviceArray.from_host(x)
    do = rai.DeviceArray(4 * m * rows)
    rc = getattr(L, fn)(do.ptr, dn.ptr, dp.ptr, dx.ptr, rows, cols, m, gs, None)
    assert rc == 0, L.rai_last_error().decode()
    assert L.rai_device_synchronize() == 0
    return do.to_host(np.float32, m * rows).view(np.uint32)


@pytest.mark.parametrize("calls", [
    [(4096, 4096, 9, 32), (1024, 2048, 5, 32)],     # matrix-core verify path, then smaller
    [(2000, 4096, 16, 32), (300, 512, 1, 32)],      # then the one-token path
    [(512, 14336, 3, 32), (96, 1024, 2, 64)],       # long rows, then group 64
    [(1000, 8192, 128, 128), (64, 256, 17, 32)],    # many tokens, then the tiled path
    [(4096, 4096, 200, 32), (1024, 2048, 70, 32)],  # the matrix-core GEMM (> 64 tokens), twice
])
def test_noalloc_matches_allocating_entry_point(rai, calls):
    for i, (rows, cols, m, gs) in enumerate(calls):
        nib, params, x = gemv_operands(rows, cols, m, gs, seed=rows + m + i)
        want = _run(rai, "rai_w4a8_matmul_dev", nib, params, x, rows, cols, m, gs)
        got = _run(rai, "rai_w4a8_matmul_noalloc_dev", nib, params, x, rows, cols, m, gs)
        assert np.array_equal(got, want), (i, rows, cols, m, gs)


def test_noalloc_rejects_sizes_past_the_scratch(rai):
    L = rai.lib()
    rows, cols, gs = 64, 4096, 32
    nib, params, x = gemv_operands(rows, cols, 1, gs, seed=1)
    dn, dp = rai.DeviceArray.from_host(nib), rai.DeviceArray.from_host(params)
    m = (1 << 20) // cols + 1
    dx = rai.DeviceArray(4 * m * cols)
    do = rai.DeviceArray(4 * m * rows)
    rc = L.rai_w4a8_matmul_noalloc_dev(do.ptr, dn.ptr, dp.ptr, dx.ptr, rows, cols, m, gs, None)
    assert rc == -2  # RAI_E_SHAPE
    assert "scratch" in L.rai_last_error().decode()
