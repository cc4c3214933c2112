"""GPU parity of the kernel-level C ABI against the CPU oracle.

Bar: bit-exact.  Integer lane sums and f32 outputs must equal the oracle's
(which reproduces the reference's AVX2 path) bit for bit.
"""
import numpy as np
import pytest

from rai_amd.workload import gemv_operands

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _f16b(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def test_known_answers(rai):
    """gemm.rs:2088-2148 through the HIP library."""
    p = np.concatenate([_f16b(1.0), _f16b(0.0)] * 2)
    out = rai.w4a8_matvec(np.full(4, 0x11, np.uint8), p, np.ones(4), 2, 4, 4)
    assert np.all(np.abs(out - 4.0) < 0.05)
    p = np.concatenate([_f16b(0.5), _f16b(-1.0)])
    out = rai.w4a8_matvec(np.array([0x55], np.uint8), p, [2.0, 3.0], 1, 2, 2)
    assert abs(out[0] - 7.5) < 0.05


# (rows, cols, gs): the fast tiled path (gs 32/64/128, full groups) and the
# general path (tiny groups, partial last group, unquantized tails).
SHAPES = [(64, 256, 32), (48, 256, 64), (40, 512, 128), (33, 160, 32), (16, 96, 32),
          (24, 100, 36), (8, 8, 4), (8, 70, 64), (17, 320, 96)]


@pytest.mark.parametrize("rows,cols,gs", SHAPES)
@pytest.mark.parametrize("m", [1, 2, 5, 9, 17])
def test_w4a8_matmul_bit_exact(rai, ora, rows, cols, gs, m):
    nib, params, x = gemv_operands(rows, cols, m, gs, seed=rows * 7 + cols + m)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, gs)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, gs)
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("rows,cols,gs", [(100, 4096, 64), (77, 8192, 128), (300, 14336, 32),
                                          (37, 2048, 64), (65, 32768, 128), (9, 65536, 32)])
@pytest.mark.parametrize("m", [1, 3, 9])
def test_w4a8_matmul_wide_k_bit_exact(rai, ora, rows, cols, gs, m):
    """Long rows at every fast-path group size, row counts that leave a
    partial row block, and K beyond what one block holds in registers."""
    nib, params, x = gemv_operands(rows, cols, m, gs, seed=rows + cols + m)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, gs)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, gs)
    assert np.array_equal(_bits(got), _bits(want)), (rows, cols, gs, m)


@pytest.mark.parametrize("rows,cols", [(100, 512), (256, 4096), (1000, 2048), (17, 14336)])
@pytest.mark.parametrize("m", [2, 3, 4, 8, 12, 16])
def test_w4a8_matrix_core_path_bit_exact(rai, ora, rows, cols, m):
    """Group 32, K a multiple of 256, 2..16 tokens: the matrix-core kernel
    (exact integer products in f16 MFMA, reference-order f32 epilogue),
    including row counts that leave partial 16-row tiles and token counts
    that leave partial 4-token groups."""
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows + 3 * cols + m)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    assert np.array_equal(_bits(got), _bits(want)), (rows, cols, m)


@pytest.mark.parametrize("rows,cols", [(8209, 2304), (16389, 4096)])
@pytest.mark.parametrize("m", [2, 5, 9, 13, 16])
def test_w4a8_register_streamed_path_bit_exact(rai, ora, rows, cols, m):
    """Row counts that select the register-streamed matrix-core kernel (two
    ring depths), a partial last 64-row block, a K whose 18 four-group steps
    leave a partial staging chunk, and every token-group width."""
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows + cols + 5 * m)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    assert np.array_equal(_bits(got), _bits(want)), (rows, cols, m)


@pytest.mark.parametrize("rows", [1000, 8209, 16389])
def test_w4a8_matrix_core_huge_activation_scales(rai, ora, rows):
    """Activation groups scaled past 2^88 (absmax ~1e29..1e30): the chunks
    holding them switch to the 1024 + n code form, which stays exact, and the
    other chunks keep the subnormal form."""
    cols, m = 2304, 9
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows)
    x = x.copy()
    x[3, 64:96] *= np.float32(1e30)
    x[8, 2016:2048] *= np.float32(3e29)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    assert np.isfinite(want).all()
    assert np.array_equal(_bits(got), _bits(want)), rows


@pytest.mark.parametrize("rows,cols", [(1000, 2048), (6150, 4096), (14336, 4096), (16389, 4096),
                                       (6144, 2560), (4096, 14336), (777, 8704)])
@pytest.mark.parametrize("m", [2, 5, 9, 13, 16])
def test_w4a8_register_pipelined_path_bit_exact(rai, ora, rows, cols, m):
    """K / 128 a multiple of 4, K <= 14336 (the register-pipelined
    matrix-core kernel): one token group per block below 6144 rows, up to
    three per wave, eight-wave blocks from 16384 rows, partial row blocks,
    a K whose steps fill one ring pass (2560), and K past 4096 (one token
    group per block, activations of up to 14336 columns in LDS)."""
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows + 11 * cols + m)
    want = ora.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
    assert np.array_equal(_bits(got), _bits(want)), (rows, cols, m)


@pytest.mark.parametrize("rows,cols,m", [(1000, 4096, 9), (6150, 4096, 9), (16389, 4096, 9),
                                         (14336, 4096, 16), (700, 14336, 9)])
def test_w4a8_register_pipelined_huge_scales_and_subnormal_params(rai, ora, rows, cols, m):
    """The register-pipelined kernel with activation groups past 2^88 (its
    1024 + n code form) and f16 weight scales / zero points that are
    subnormal or zero (read straight from the parameter halves), at K = 4096
    and at the longest K (one token group per block)."""
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows + m)
    p = params.copy().view(np.float16).reshape(rows, cols // 32, 2)
    p[::7, ::3, 0] = np.float16(3e-6)
    p[::5, 1::4, 1] = np.float16(-2e-6)
    p[3::11, 2::5, :] = np.float16(0.0)
    params = p.view(np.uint8).reshape(-1)
    for scaled in (False, True):
        xs = x.copy()
        if scaled:
            xs[3, 64:96] *= np.float32(1e30)
            xs[m - 1, 2016:2048] *= np.float32(3e29)
        want = ora.w4a8_matmul(nib, params, xs, rows, cols, m, 32)
        got = rai.w4a8_matmul(nib, params, xs, rows, cols, m, 32)
        assert np.isfinite(want).all()
        assert np.array_equal(_bits(got), _bits(want)), (rows, m, scaled)


@pytest.mark.parametrize("rows,cols,m", [(1024, 4096, 9), (6144, 4096, 9), (16384, 4096, 9), (4096, 14336, 9),
                                         (2048, 2560, 5), (16384, 4096, 16)])
def test_w4a8_tiled_parameters_bit_exact(rai, ora, rows, cols, m):
    """The register-pipelined kernel reading the parameters' 16-row tile copy
    (the batched forward's path; the GEMV timer builds the copy as a loaded
    model does), with and without activation groups past 2^88 (its 1024 + n
    code form) and with f16 weight scales / zero points that are subnormal or
    zero."""
    nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows + 3 * m)
    p = params.copy().view(np.float16).reshape(rows, cols // 32, 2)
    p[::7, ::3, 0] = np.float16(3e-6)
    p[::5, 1::4, 1] = np.float16(-2e-6)
    p[3::11, 2::5, :] = np.float16(0.0)
    params = p.view(np.uint8).reshape(-1)
    timer = rai.GemvTimer(nib, params, rows, cols, 32)
    for scaled in (False, True):
        xs = x.copy()
        if scaled:
            xs[m - 1, 64:96] *= np.float32(1e30)
        want = np.asarray(ora.w4a8_matmul(nib, params, xs, rows, cols, m, 32)).reshape(m, rows)
        _, got = timer.run(xs, m)
        assert np.isfinite(want).all()
        assert np.array_equal(_bits(got), _bits(want)), (rows, cols, m, scaled)


@pytest.mark.parametrize("rows,cols,gs", SHAPES[:6])
def test_lane_sums_bit_exact(rai, ora, rows, cols, gs):
    nib, _, x = gemv_operands(rows, cols, 3, gs, seed=cols)
    assert np.array_equal(rai.w4a8_lane_sums(nib, x, rows, cols, 3, gs),
                          ora.lane_sums(nib, x, rows, cols, 3, gs))


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (14336, 4096), (4096, 14336), (32000, 4096)])
def test_gemv_sweep_shapes_bit_exact(rai, ora, rows, cols):
    """The W4A8 sweep shapes at full size, g32, M in {1, 9}: f32 outputs and,
    for a row slice, the int32 accumulators."""
    for m in (1, 9):
        nib, params, x = gemv_operands(rows, cols, m, 32, seed=rows + m)
        want = ora.w4a8_matmul(nib, params, x, rows, cols, m, 32)
        got = rai.w4a8_matmul(nib, params, x, rows, cols, m, 32)
        assert np.array_equal(_bits(got), _bits(want)), (rows, cols, m)
    nib, _, x = gemv_operands(256, cols, 2, 32, seed=cols)
    assert np.array_equal(rai.w4a8_lane_sums(nib, x, 256, cols, 2, 32),
                          ora.lane_sums(nib, x, 256, cols, 2, 32))


def test_tied_lm_head_bit_exact(rai, ora):
    rng = np.random.default_rng(3)
    for vocab, n, gs in ((96, 64, 64), (500, 256, 64), (77, 100, 36)):
        codes = rng.integers(0, 256, vocab * n, dtype=np.uint8)
        g = -(-n // gs)
        params = np.stack([np.abs(rng.normal(0, 0.01, vocab * g)) + 1e-3,
                           rng.normal(0, 0.1, vocab * g)], axis=1).astype(np.float16)
        params = params.view(np.uint8).reshape(-1)
        h = rng.normal(size=n).astype(np.float32)
        want = ora.tied_lm_head(h, codes, params, vocab, gs)
        got = rai.tied_lm_head(h, codes, params, vocab, gs)
        assert np.array_equal(_bits(got), _bits(want))


def test_embed_lookup_bit_exact(rai, ora):
    rng = np.random.default_rng(4)
    vocab, n, gs = 50, 128, 64
    codes = rng.integers(0, 256, vocab * n, dtype=np.uint8)
    params = np.stack([np.abs(rng.normal(0, 0.01, vocab * 2)) + 1e-3,
                       rng.normal(0, 0.1, vocab * 2)], axis=1).astype(np.float16).view(np.uint8).reshape(-1)
    for t in (0, 17, 49):
        assert np.array_equal(_bits(rai.embed_lookup(t, codes, params, vocab, n, gs)),
                              _bits(ora.embed_lookup(t, codes, params, vocab, n, gs)))
    with pytest.raises(rai.RaiError) as e:
        rai.embed_lookup(vocab, codes, params, vocab, n, gs)
    assert e.value.status == "RAI_E_RANGE"


def test_ngram_kernel_known_answers(rai):
    """lookup.rs:486-571 known answers through the GPU search kernel."""
    from test_cpu_oracle import NGRAM_CASES
    for tokens, mn, mx, k, want in NGRAM_CASES:
        m = rai.find_ngram_draft(tokens, mn, mx, k)
        assert (None if m is None else (m.ngram, m.start, m.len)) == want, tokens


def test_ngram_kernel_matches_oracle(rai, ora):
    rng = np.random.default_rng(5)
    for i in range(60):
        n = int(rng.integers(2, 3000 if i % 10 == 0 else 60))
        t = rng.integers(0, 3 if i % 2 else 50, size=n).tolist()
        mn = int(rng.integers(1, 4))
        mx = int(rng.integers(mn, 6))
        k = int(rng.integers(1, 9))
        m = rai.find_ngram_draft(t, mn, mx, k)
        assert (None if m is None else (m.ngram, m.start, m.len)) == ora.find_ngram_draft(t, mn, mx, k)


def test_shape_errors(rai):
    """validate_weight_buffers (gemm.rs:1169-1213) panics become RAI_E_SHAPE."""
    with pytest.raises(rai.RaiError) as e:
        rai.w4a8_matmul(np.zeros(2, np.uint8), np.zeros(4, np.uint8), np.ones(3), 1, 3, 1, 3)
    assert e.value.status == "RAI_E_SHAPE"


@pytest.mark.gpu
def test_attention_timer_runs_the_production_launches(rai):
    """rai_attention_time_dev times the decode and verify attention launches
    (scores, softmax, PV) and refuses shapes the attention does not take."""
    for m in (1, 9):
        sc, sm, pv = rai.attention_time(8, 2, 64, 1024, 700, m, copies=2, iters=3)
        assert all(np.isfinite(x) and x > 0 for x in (sc, sm, pv))
    with pytest.raises(rai.RaiError) as e:
        rai.attention_time(8, 3, 64, 1024, 700, 1, iters=1)
    assert e.value.status == "RAI_E_SHAPE"
    with pytest.raises(rai.RaiError) as e:
        rai.attention_time(8, 2, 64, 1024, 1020, 9, iters=1)
    assert e.value.status == "RAI_E_RANGE"
