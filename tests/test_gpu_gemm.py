"""GPU parity of the matrix-core W4A8 GEMM (more than 64 tokens, group 32)
against the CPU oracle (the reference's matmul_chunk_i8 path).

Bar: bit-exact f32 outputs (17..64 tokens run the verify kernels, checked
here at the hand-off).  Shapes cover partial 32-row and 128-row
blocks, token counts that leave a partial 32-token tile, K at the 512-column
granularity of the kernel up to 14336, extreme activation scales and
subnormal f16 weight parameters.
"""
import numpy as np
import pytest

from rai_amd.workload import GEMV_SHAPES, gemv_operands

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("rows,cols", [(128, 512), (300, 1024), (17, 2048), (1000, 4096), (77, 14336)])
@pytest.mark.parametrize("m", [17, 33, 64, 65, 100, 256])
def test_mm_bit_exact(rai, ora, rows, cols, m):
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows * 3 + cols + m)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    assert np.array_equal(_bits(got), _bits(want)), (rows, cols, m)


def test_mm_extreme_scales_and_subnormal_params(rai, ora):
    """Activation groups scaled to ~1e30 and ~1e-30 (scales far from 1),
    zero groups, and weight scales/zeros that are f16 subnormals."""
    rows, cols, m = 160, 1024, 90
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=11)
    x = x.reshape(m, cols // 32, 32)
    x[3, 5] *= 1e30
    x[7, 2] *= 1e-30
    x[9, 9] = 0.0
    x[20] *= -3.0e4
    x = x.reshape(m, cols)
    p = params.view(np.float16).reshape(rows, cols // 32, 2).copy()
    p[5, :, 0] = np.float16(3e-6)
    p[6, :, 1] = np.float16(-5e-7)
    p[7, 3, 0] = np.float16(0.0)
    params = p.view(np.uint8).reshape(-1)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("rows,cols", [(256, 1024), (1000, 4096)])
def test_mm_huge_scale_quads_per_token_tile(rai, ora, rows, cols):
    """Activation scales of 2^88 and more flag their quad of groups: a token
    tile holding one runs with the 1024 + n codes and rescales its other
    quads' scales; the other tiles keep the subnormal codes.  Huge groups in
    the first and in the last, partial, token tile (75 tokens), none in the
    middle one."""
    m = 75
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows + 75)
    x = x.reshape(m, cols // 32, 32).copy()
    x[5, 3] *= np.float32(1e30)
    x[70, cols // 32 - 1] *= np.float32(3e29)
    x[40, 7] *= np.float32(1e-30)
    x = x.reshape(m, cols)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    assert np.isfinite(want).all()
    assert np.array_equal(_bits(got), _bits(want)), (rows, cols)


@pytest.mark.parametrize("rows,cols", GEMV_SHAPES)
def test_cfg3_m512_sweep_shapes_bit_exact(rai, ora, rows, cols):
    """W4A8 sweep at M = 512 (prefill-sized) on the four sweep shapes."""
    nib, params, x = gemv_operands(rows, cols, 512, 32, seed=rows + cols + 512)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, 512, 32)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, 512, 32)
    assert np.array_equal(_bits(got), _bits(want)), (rows, cols)


def test_mm_matches_one_token_rows(rai, ora):
    """matmul == matvec per token (gemm.rs:1774-1919 is a scheduling change,
    not a numerical one): row t of an 80-token GEMM equals the one-token GEMV
    of token t."""
    rows, cols, m = 256, 2048, 80
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=5)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    for t in (0, 17, 31, 32, 64, 79):
        one = rai.w4a8_matvec(nib, params, x[t], rows, cols, 32)
        assert np.array_equal(_bits(got[t]), _bits(one)), t
