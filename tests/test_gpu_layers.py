"""GPU parity of the layer kernels (layers.rs public functions) against the
oracle, bit for bit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("n", [64, 100, 2048, 4096, 5632])
def test_rms_norm_bit_exact(rai, ora, n):
    rng = np.random.default_rng(n)
    rows = 64  # many rows: a 1-ulp sqrt or divide slip shows up in some of them
    x = (rng.normal(size=(rows, n)) * rng.uniform(0.1, 30, size=(rows, 1))).astype(np.float32)
    w = rng.normal(1.0, 0.1, size=n).astype(np.float32)
    got = rai.rms_norm(x, w, 1e-5)
    for r in range(rows):
        assert np.array_equal(_bits(got[r]), _bits(ora.rms_norm(x[r], w, 1e-5))), r


@pytest.mark.parametrize("n", [16, 19, 128, 5632])
def test_silu_mul_bit_exact(rai, ora, n):
    rng = np.random.default_rng(n)
    g = (rng.normal(size=(2, n)) * 4).astype(np.float32)
    u = rng.normal(size=(2, n)).astype(np.float32)
    got = rai.silu_mul(g, u)
    for r in range(2):
        assert np.array_equal(_bits(got[r]), _bits(ora.silu_mul(g[r], u[r]))), r


@pytest.mark.parametrize("hd,nh", [(16, 4), (64, 32), (128, 8), (40, 3)])
def test_rope_bit_exact(rai, ora, hd, nh):
    rng = np.random.default_rng(hd)
    c, s = ora.rope_tables(hd, 300, 10000.0)
    h = rng.normal(size=nh * hd).astype(np.float32)
    for pos in (0, 1, 17, 299):
        assert np.array_equal(_bits(rai.rope_apply(h, nh, hd, c[pos], s[pos])),
                              _bits(ora.rope_apply(h, nh, hd, c[pos], s[pos]))), pos


@pytest.mark.parametrize("hd", [16, 64, 128])
@pytest.mark.parametrize("pos", [0, 6, 7, 8, 15, 100, 1000])
def test_attention_head_bit_exact(rai, ora, hd, pos):
    rng = np.random.default_rng(hd * 1000 + pos)
    q = rng.normal(size=hd).astype(np.float32)
    k = rng.normal(size=(pos + 1, hd)).astype(np.float32)
    v = rng.normal(size=(pos + 1, hd)).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    got = rai.attention_head(q, k, v, pos, hd, float(scale))
    want = ora.attention_head(q, k, v, pos, hd, float(scale))
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("pos", [2047, 2048, 4100, 8191, 9000, 16383, 16384, 20002, 32767, 40001])
def test_attention_head_long_context_bit_exact(rai, ora, hd, pos):
    """Contexts that select each register depth of the softmax (up to 2048,
    4096, 8192 and 16384 positions) and the chunked softmax past them (one
    to twelve 3584-position chunks), with tails of 0..7 positions past the
    last 8-block and chains long enough for the prefetched LDS reads."""
    rng = np.random.default_rng(hd * 7 + pos)
    q = rng.normal(size=hd).astype(np.float32)
    k = rng.normal(size=(pos + 1, hd)).astype(np.float32)
    v = rng.normal(size=(pos + 1, hd)).astype(np.float32)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    got = rai.attention_head(q, k, v, pos, hd, float(scale))
    want = ora.attention_head(q, k, v, pos, hd, float(scale))
    assert np.array_equal(_bits(got), _bits(want)), pos


def test_rope_tables_match_oracle(rai, ora):
    """The library builds RoPE tables on the host with the C library's
    powf/cosf/sinf exactly as RoPETable::with_scaling does: the rotated K rows
    the forward pass stores at positions 0..5 (every head, both layers) equal
    the oracle's bit for bit."""
    from conftest import read_golden
    data = read_golden("tiny-untied.raimodel")
    gm = rai.RaiModel.from_bytes(data)
    om = ora.Model(data, 128)
    kv, okv = gm.create_kv_cache(8), om.create_kv(8)
    toks = (5, 9, 17, 2, 60, 33)
    for p, t in enumerate(toks):
        gm.forward_from_hidden(gm.embed_token(t), p, kv)
    om.forward_batch(np.stack([om.embed_token(t) for t in toks]), np.arange(6), okv)
    hd = gm.config.head_dim
    for layer in range(gm.config.num_layers):
        for head in range(gm.config.num_kv_heads):
            for p in range(6):
                assert np.array_equal(_bits(kv.get_k(layer, head, p, hd)), _bits(okv.get_k(layer, head, p, hd)))
                assert np.array_equal(_bits(kv.get_v(layer, head, p, hd)), _bits(okv.get_v(layer, head, p, hd)))
