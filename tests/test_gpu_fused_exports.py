"""The kernel-level fused projections, rai_w4a8_fused_qkv_dev and
rai_w4a8_fused_gate_up_dev (gemm.rs:1386-1703), against the oracle's
separate w4a8_matvec of each projection (the reference computes the same
per-row sums from one shared quantization): bit-exact f32 outputs at the
configs' projection shapes, and the reference's shape checks."""
import numpy as np
import pytest

from rai_amd.workload import gemv_operands

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _proj(rows, cols, gs, seed):
    nib, params, _ = gemv_operands(rows, cols, 1, gs, seed=seed)
    return (nib, params, rows, cols, gs)


QKV = [  # (q rows, kv rows, cols, group)
    (4096, 1024, 4096, 32),   # 7B: 32 heads / 8 kv heads of 128
    (2048, 256, 2048, 32),    # 1.1B: 32 heads / 4 kv heads of 64
    (2048, 2048, 2048, 32),   # MoE 1B-7B: 16 heads / 16 kv heads of 128
    (4096, 1024, 4096, 128),  # 7B at group 128
    (96, 24, 200, 8),         # small, ragged groups (200 = 25 groups of 8)
]


@pytest.mark.parametrize("qr,kvr,cols,gs", QKV)
def test_fused_qkv_equals_separate_matvecs(rai, ora, qr, kvr, cols, gs):
    q, k, v = _proj(qr, cols, gs, 1), _proj(kvr, cols, gs, 2), _proj(kvr, cols, gs, 3)
    x = np.random.default_rng(cols + qr).normal(0.0, 1.0, cols).astype(np.float32)
    got = rai.w4a8_fused_qkv(q, k, v, x)
    for g, p in zip(got, (q, k, v)):
        want = ora.w4a8_matvec(p[0], p[1], x, p[2], p[3], p[4])
        assert np.array_equal(_bits(g), _bits(want)), p[2:]


@pytest.mark.parametrize("rows,cols,gs", [(14336, 4096, 32), (5632, 2048, 32), (1024, 2048, 32),
                                          (14336, 4096, 128), (40, 64, 16)])
def test_fused_gate_up_equals_separate_matvecs(rai, ora, rows, cols, gs):
    g, u = _proj(rows, cols, gs, 4), _proj(rows, cols, gs, 5)
    x = np.random.default_rng(rows + cols).normal(0.0, 1.0, cols).astype(np.float32)
    got = rai.w4a8_fused_gate_up(g, u, x)
    for o, p in zip(got, (g, u)):
        want = ora.w4a8_matvec(p[0], p[1], x, p[2], p[3], p[4])
        assert np.array_equal(_bits(o), _bits(want))


def test_fused_projection_checks(rai):
    """Disagreeing cols or group sizes fail as the reference's asserts
    ("Q/K column mismatch", "gate/up group mismatch"), as do odd cols."""
    x = np.zeros(512, np.float32)
    a, b = _proj(64, 512, 32, 1), _proj(32, 256, 32, 2)
    with pytest.raises(rai.RaiError) as e:
        rai.w4a8_fused_qkv(a, b, a, x)
    assert e.value.status == "RAI_E_SHAPE" and "Q/K column mismatch" in str(e.value)
    c = _proj(64, 512, 64, 3)
    with pytest.raises(rai.RaiError) as e:
        rai.w4a8_fused_gate_up(a, c, x)
    assert e.value.status == "RAI_E_SHAPE" and "gate/up group mismatch" in str(e.value)
    d = (a[0], a[1], 64, 511, 32)
    with pytest.raises(rai.RaiError) as e:
        rai.w4a8_fused_gate_up(d, d, x)
    assert e.value.status == "RAI_E_SHAPE"
