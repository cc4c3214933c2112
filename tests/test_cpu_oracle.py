"""CPU tests: pin the oracle against the reference's own golden data and the
mathematics, and check the host-side pieces of the product that need no GPU.

Each check cites the reference test or fixture it mirrors.
"""
import json
import os
import struct

import numpy as np
import pytest

from conftest import golden, read_golden


# ------------------------------------------------------------------ format --

def _linear_row_prefix(data: bytes, off: int, rows: int, cols: int, gs: int, row: int, n: int):
    """Independent numpy dequantizer of one linear row (format.rs:361-367)."""
    r, c = struct.unpack_from("<II", data, off)
    assert (r, c) == (rows, cols)
    groups = -(-cols // gs)
    params = np.frombuffer(data, np.float16, rows * groups * 2, off + 8).reshape(rows, groups, 2)
    nib = np.frombuffer(data, np.uint8, rows * cols // 2, off + 8 + rows * groups * 4)
    out = []
    for col in range(n):
        b = nib[(row * cols + col) // 2]
        code = (b & 15) if col % 2 == 0 else (b >> 4)
        s, z = params[row, col // gs]
        out.append(np.float32(code) * np.float32(s) + np.float32(z))
    return np.array(out, np.float32)


def _sections(data: bytes):
    n = struct.unpack_from("<I", data, 52)[0]
    return [struct.unpack_from("<QQ", data, 64 + 16 * i) for i in range(n)]


@pytest.mark.parametrize("name", ["tiny-tied", "tiny-untied"])
def test_fixture_conformance(ora, name):
    """format_conformance.rs:122-179: header, sections, tied detection and the
    exporter-recorded dequantized values (tolerance f32::EPSILON * max(|e|,1))."""
    data = read_golden(name + ".raimodel")
    side = json.load(open(golden(name + ".expected.json")))
    assert len(data) == side["file_size"]
    m = ora.Model(data, 128)
    cfg = side["config"]
    for k in ("hidden_size", "num_layers", "num_heads", "num_kv_heads", "head_dim",
              "intermediate_size", "vocab_size", "max_context", "group_size",
              "embed_group_size"):
        assert getattr(m.cfg, k) == cfg[k], k
    assert m.cfg.tied == int(side["tied"])
    secs = _sections(data)
    assert len(secs) == side["num_sections"]
    eps = np.finfo(np.float32).eps

    def close(a, e):
        e = np.array(e, np.float32)
        assert np.all(np.abs(a - e) <= eps * np.maximum(np.abs(e), 1.0))

    close(m.embed_token(0), side["expected"]["embedding_row0"])
    H, gs = cfg["hidden_size"], cfg["group_size"]
    close(_linear_row_prefix(data, secs[1][0], cfg["num_heads"] * cfg["head_dim"], H, gs, 0, 8),
          side["expected"]["layer0_q_proj_row0_first8"])
    if not side["tied"]:
        close(_linear_row_prefix(data, secs[-1][0], cfg["vocab_size"], H, gs, 0, 8),
              side["expected"]["lm_head_row0_first8"])


def test_writer_reproduces_convert_fixture(rai):
    """gen_convert_fixture.py:74-109 + convert_matches_python.rs:566: the
    synthetic writer in its LCG/asymmetric-RTN mode is byte-identical to the
    reference exporter's tiny-convert.raimodel (pins min/max RTN, f16 rounding,
    8-bit embedding quantization and the section layout)."""
    img = rai.synth_model(64, 2, 4, 2, 16, 128, 96, 512, group_size=64, embed_group_size=64,
                          tied=True, mode=2)
    assert img.tobytes() == read_golden("tiny-convert.raimodel")


def test_symmetric_rtn_closed_form(rai):
    """Symmetric int4 RTN (code = q+8, zero = -8*scale): every weight dequantizes
    to within half a quantization step of scale*round(w/scale)."""
    img = rai.synth_model(64, 1, 4, 2, 16, 128, 96, 64, group_size=32, seed=3).tobytes()
    secs = _sections(img)
    off = secs[1][0]
    rows, cols = struct.unpack_from("<II", img, off)
    params = np.frombuffer(img, np.float16, rows * 2 * 2, off + 8).reshape(rows, 2, 2)
    s, z = params[..., 0].astype(np.float64), params[..., 1].astype(np.float64)
    assert np.array_equal(z, -8.0 * s)
    assert np.all(s > 0)
    nib = np.frombuffer(img, np.uint8, rows * cols // 2, off + 8 + rows * 2 * 4)
    codes = np.stack([nib & 15, nib >> 4], axis=1).reshape(rows, cols)
    assert codes.min() >= 0 and codes.max() <= 15


# ---------------------------------------------------------------- W4A8 math --

def _f16b(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def test_matvec_known_answers(ora):
    """gemm.rs:2088-2148: identity-like -> 4.0, scale/zero -> 7.5."""
    p = np.concatenate([_f16b(1.0), _f16b(0.0)] * 2)
    out = ora.w4a8_matvec(np.full(4, 0x11, np.uint8), p, np.ones(4), 2, 4, 4)
    assert np.all(np.abs(out - 4.0) < 0.05)
    p = np.concatenate([_f16b(0.5), _f16b(-1.0)])
    out = ora.w4a8_matvec(np.array([0x55], np.uint8), p, [2.0, 3.0], 1, 2, 2)
    assert abs(out[0] - 7.5) < 0.05


def _exact_quant_input(cols, gs, limit=127):
    """gemm.rs:2371-2383: every group attains absmax 1, values t/limit."""
    out = np.empty(cols, np.float32)
    for i in range(cols):
        j = i % gs
        t = limit if j == 0 else (j * 37) % (2 * limit + 1) - limit
        out[i] = np.float32(t) / np.float32(limit)
    return out


@pytest.mark.parametrize("cols,gs", [(256, 64), (256, 32), (512, 128), (96, 32), (160, 96)])
def test_lane_sums_exact_closed_form(ora, cols, gs):
    """With exact_quant_input the int8 activations are exactly t, so every
    integer lane sum equals sum(code * t) over that lane's columns."""
    rng = np.random.default_rng(cols + gs)
    rows = 8
    nib = rng.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    x = _exact_quant_input(cols, gs)
    t = np.rint(x.astype(np.float64) * 127).astype(np.int64)
    got = ora.lane_sums(nib, x, rows, cols, 1, gs)[0]
    codes = np.stack([nib & 15, nib >> 4], axis=1).reshape(rows, cols).astype(np.int64)
    groups = -(-cols // gs)
    for g in range(groups):
        c0, ags = g * gs, min(gs, cols - g * gs)
        c64 = ags // 64
        for lane in range(8):
            cs = [c0 + 64 * c + 8 * lane + j for c in range(c64) for j in range(8)]
            want = (codes[:, cs] * t[cs]).sum(axis=1) if cs else np.zeros(rows)
            assert np.array_equal(got[:, g, lane], want)
        for lane in range(4):
            if 64 * c64 + 32 <= ags:
                cs = [c0 + 64 * c64 + 8 * lane + j for j in range(8)]
                want = (codes[:, cs] * t[cs]).sum(axis=1)
            else:
                want = np.zeros(rows)
            assert np.array_equal(got[:, g, 8 + lane], want)


def test_matvec_f64_dequant_reference(ora):
    """gemm.rs:2423-2446: parallel-path shape against an f64 dequantized
    reference (exact_quant_input), tolerance 5e-3 relative."""
    rows, cols, gs = 4288, 256, 64
    i = np.arange(rows * cols // 2)
    nib = (((i * 7 + 3) % 16) | (((i * 11 + 5) % 16) << 4)).astype(np.uint8)
    s, z = np.float16(0.5), np.float16(-4.0)
    params = np.tile(np.concatenate([_f16b(0.5), _f16b(-4.0)]), rows * (cols // gs))
    x = _exact_quant_input(cols, gs)
    out = ora.w4a8_matvec(nib, params, x, rows, cols, gs)
    codes = np.stack([nib & 15, nib >> 4], axis=1).reshape(rows, cols).astype(np.float64)
    want = ((codes * float(s) + float(z)) * x.astype(np.float64)).sum(axis=1)
    assert np.all(np.abs(out - want) <= 5e-3 * np.maximum(np.abs(want), 1.0))


def test_matmul_equals_matvec_bitwise(ora):
    """gemm.rs:547-549 / 2151-2212: the batched kernel is the per-token kernel."""
    from rai_amd.workload import gemv_operands
    for gs in (32, 64, 128, 4):
        nib, params, x = gemv_operands(48, 256, 7, gs, seed=gs)
        mm = ora.w4a8_matmul(nib, params, x, 48, 256, 7, gs)
        for t in range(7):
            mv = ora.w4a8_matvec(nib, params, x[t], 48, 256, gs)
            assert np.array_equal(mm[t].view(np.uint32), mv.view(np.uint32))


def test_quantize_matches_definition(ora):
    """gemm.rs:280-374: scale = absmax/127, q = clamp(rne(x*inv)), tail pairs
    round half away from zero; sums in the 8-lane order."""
    rng = np.random.default_rng(7)
    x = rng.normal(size=100).astype(np.float32)
    x[5] = 0.0
    qe, qo, sc = ora.quantize_split(x, 36)
    q = np.empty(100, np.int64)
    q[0::2], q[1::2] = qe, qo
    for g in range(3):
        seg = x[g * 36:min(100, g * 36 + 36)]
        amax = np.float32(np.abs(seg).max())
        scale = np.float32(amax / np.float32(127.0))
        assert sc[g] == scale
        inv = np.float32(np.float32(1.0) / scale)
        v = (seg * inv).astype(np.float32)
        body = (len(seg) // 8) * 8
        want = np.concatenate([np.rint(v[:body]),
                               np.sign(v[body:]) * np.floor(np.abs(v[body:]) + 0.5)])
        assert np.array_equal(q[g * 36:g * 36 + len(seg)], np.clip(want, -128, 127))


# ------------------------------------------------------------ layer math --

def test_rms_norm_closed_form(ora):
    """layers.rs test_rms_norm: [1,2,3,4] normalized by sqrt(mean(x^2)+eps)."""
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    out = ora.rms_norm(x, np.ones(4), 1e-5)
    want = x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
    assert np.allclose(out, want, rtol=1e-6)
    rng = np.random.default_rng(1)
    x = rng.normal(size=2048).astype(np.float32)
    w = rng.normal(size=2048).astype(np.float32)
    out = ora.rms_norm(x, w, 1e-5)
    want = x * w / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
    assert np.allclose(out, want, rtol=2e-6, atol=1e-6)


def test_rope_identity_at_position_zero(ora):
    """layers.rs:1933-1983: position 0 leaves q/k unchanged; a later position
    is a rotation (norm preserving)."""
    c, s = ora.rope_tables(64, 16, 10000.0)
    rng = np.random.default_rng(2)
    h = rng.normal(size=4 * 64).astype(np.float32)
    assert np.array_equal(ora.rope_apply(h, 4, 64, c[0], s[0]), h)
    r = ora.rope_apply(h, 4, 64, c[9], s[9]).reshape(4, 64)
    hh = h.reshape(4, 64)
    n0 = hh[:, :32] ** 2 + hh[:, 32:] ** 2
    n1 = r[:, :32] ** 2 + r[:, 32:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5)


def test_schraudolph_constants(ora, rai):
    """layers.rs:855-858: exp_b is the f32-rounded 1065353216-486411 and the
    host restatement of the bit trick agrees with the oracle's AVX2 lanes."""
    assert np.float32(1065353216.0) - np.float32(486411.0) == np.float32(1064866816.0)
    assert ora.schraudolph(0.0) == pytest.approx(1.0, rel=0.03)
    for v in np.linspace(-20, 20, 101, dtype=np.float32):
        e = ora.schraudolph(float(v))
        assert e == pytest.approx(float(np.exp(np.float64(v))), rel=0.07)


def test_silu_mul_against_exact(ora):
    """layers.rs:816-883: Schraudolph SiLU within the documented < 2% of the
    exact value on the 8-wide body; the scalar tail is exact expf."""
    rng = np.random.default_rng(4)
    g = rng.normal(size=19).astype(np.float32) * 3
    u = rng.normal(size=19).astype(np.float32)
    out = ora.silu_mul(g, u)
    exact = g / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(out[:16], exact[:16], rtol=0.03, atol=1e-3)
    tail = (g[16:] / (np.float32(1.0) + np.exp(-g[16:]))).astype(np.float32) * u[16:]
    assert np.array_equal(out[16:], tail.astype(np.float32))


def test_attention_head_matches_softmax(ora):
    """layers.rs:1266-1380: output is softmax(qk*scale) @ v up to the
    Schraudolph approximation, and uniform keys give the mean of v."""
    rng = np.random.default_rng(5)
    hd, pos = 16, 15  # 16 positions: all take the 8-wide Schraudolph body
    q = rng.normal(size=hd).astype(np.float32)
    k = np.zeros((pos + 1, hd), np.float32)
    v = rng.normal(size=(pos + 1, hd)).astype(np.float32)
    out = ora.attention_head(q, k, v, pos, hd, 0.25)
    assert np.allclose(out, v.mean(axis=0), rtol=1e-5, atol=1e-6)
    pos = 11  # 8-wide body plus a 4-position exact-exp tail
    v = v[:pos + 1]
    k = rng.normal(size=(pos + 1, hd)).astype(np.float32)
    out = ora.attention_head(q, k, v, pos, hd, 0.25)
    sc = (k @ q) * 0.25
    p = np.exp(sc - sc.max())
    p /= p.sum()
    assert np.allclose(out, p @ v, rtol=0.1, atol=0.05)


# -------------------------------------------------------- sampler / lookup --

def test_argmax_known_answers(ora):
    """sampler.rs:216-304: greedy picks the max; NaN is never selected; ties go
    to the last index (max_by over total_cmp); -0 < +0."""
    assert ora.argmax([1.0, 5.0, 2.0, 3.0]) == 1
    assert ora.argmax([np.nan, 1.0, 2.0]) == 2
    assert ora.argmax([3.0, 1.0, 3.0, 2.0]) == 2
    assert ora.argmax([0.0, -0.0]) == 0
    assert ora.argmax([-0.0, 0.0]) == 1
    assert ora.argmax([np.nan, np.nan]) == 1
    assert ora.argmax([np.inf, 1.0, np.inf]) == 2


NGRAM_CASES = [
    # lookup.rs:486-571 known answers: (tokens, min, max, K, expected (ngram, start, len) or None)
    ([1, 2, 9, 9, 1, 2, 7, 8, 1, 2], 1, 2, 2, (2, 6, 2)),
    ([5, 6, 7, 1, 2, 3, 6, 7, 4, 5, 6, 7], 1, 3, 2, (3, 3, 2)),
    ([5, 6, 7, 1, 2, 3, 6, 7, 4, 5, 6, 7], 2, 2, 2, (2, 8, 2)),
    ([4, 1, 2, 3, 4], 2, 3, 4, None),
    ([4, 1, 2, 3, 4], 1, 3, 4, (1, 1, 4)),
    ([1, 2, 3, 4, 5], 1, 3, 4, None),
    ([], 1, 3, 4, None),
    ([7], 1, 3, 4, None),
    ([1, 2, 1, 2], 1, 2, 0, None),
    ([1, 2, 3, 4, 3], 1, 1, 8, (1, 3, 2)),
    ([1, 2, 3], 3, 3, 4, None),
    ([1, 2, 3, 4, 5, 6, 1, 2], 1, 2, 3, (2, 2, 3)),
    ([1, 2, 3, 4, 5, 6, 1, 2], 1, 99, 2, (2, 2, 2)),
]


@pytest.mark.parametrize("tokens,mn,mx,k,want", NGRAM_CASES)
def test_find_ngram_known_answers(ora, tokens, mn, mx, k, want):
    assert ora.find_ngram_draft(tokens, mn, mx, k) == want


def _brute_ngram(t, mn, mx, k):
    n = len(t)
    if k == 0 or n < 2:
        return None
    for g in range(min(mx, n - 1), max(mn, 1) - 1, -1):
        for s in range(n - g - 1, -1, -1):
            if t[s:s + g] == t[n - g:]:
                return (g, s + g, min(k, n - s - g))
    return None


def test_find_ngram_brute_force(ora):
    rng = np.random.default_rng(11)
    for _ in range(300):
        n = int(rng.integers(0, 40))
        t = rng.integers(0, 4, size=n).tolist()
        mn = int(rng.integers(1, 4))
        mx = int(rng.integers(mn, 6))
        k = int(rng.integers(0, 9))
        assert ora.find_ngram_draft(t, mn, mx, k) == _brute_ngram(t, mn, mx, k)


# --------------------------------------------------------- model invariants --

def _token_sequence(vocab, n):
    """model_invariants.rs:22-31 LCG token sequence."""
    state = 0x9E3779B97F4A7C15
    out = []
    for _ in range(n):
        state = (state * 6364136223846793005 + 1442695040888963407) & ((1 << 64) - 1)
        out.append((state >> 33) % vocab)
    return out


@pytest.mark.parametrize("name", ["tiny-tied.raimodel", "tiny-untied.raimodel",
                                  "tiny-convert.raimodel"])
def test_oracle_batched_equals_sequential(ora, name):
    """model_invariants.rs:92-134 (argmax equal, |dlogit| <= 2e-3); the
    reference states the two are bit-identical (BENCHMARKS.md:129-131), which
    is what the oracle checks."""
    m = ora.Model(read_golden(name), 128)
    H, V = m.cfg.hidden_size, m.cfg.vocab_size
    toks = _token_sequence(V, 12)
    kv = m.create_kv(64)
    seq = []
    for p, t in enumerate(toks):
        h = m.forward_from_hidden(m.embed_token(t), p, kv)
        seq.append(m.hidden_to_logits(h))
    kv2 = m.create_kv(64)
    hs = np.stack([m.embed_token(t) for t in toks])
    hb = m.forward_batch(hs, np.arange(12), kv2)
    lb = m.hidden_to_logits_batch(hb, 12)
    for i in range(12):
        assert np.array_equal(lb[i].view(np.uint32), seq[i].view(np.uint32))


def test_oracle_kv_watermark(ora):
    """kv_cache.rs:447-469 / model_invariants.rs:159-183: a gap store and a
    stale read are errors; truncate + refill is consistent."""
    m = ora.Model(read_golden("tiny-untied.raimodel"), 128)
    kv = m.create_kv(32)
    with pytest.raises(ora.OracleError):
        m.forward_from_hidden(m.embed_token(1), 3, kv)
    h0 = m.forward_from_hidden(m.embed_token(1), 0, kv)
    m.forward_from_hidden(m.embed_token(2), 1, kv)
    kv.truncate(1)
    assert kv.filled(0) == 1
    m.forward_from_hidden(m.embed_token(2), 1, kv)
    kv3 = m.create_kv(32)
    assert np.array_equal(m.forward_from_hidden(m.embed_token(1), 0, kv3), h0)


def test_oracle_greedy_lookup_equals_greedy_decode(ora, rai):
    """Greedy prompt-lookup yields exactly the plain greedy token stream
    (the T->0 limit of lookup.rs:359-403 with the batched == sequential
    invariant)."""
    from rai_amd.workload import copy_heavy_prompt
    img = rai.synth_model(128, 2, 4, 2, 32, 256, 300, 512, group_size=32, seed=9)
    m = ora.Model(img, 0)
    prompt = copy_heavy_prompt(60, 300, seed=1).astype(np.int32)
    steps = 40
    want = m.greedy_generate(prompt, steps, 256).tolist()
    dec = ora.LookupDecoder(m, 256)
    pos = dec.prefill(prompt)
    ctx = prompt.tolist()
    got = []
    drafted = 0
    while len(got) < steps:
        toks, met = dec.step(pos, ctx, 8, 1, 3)
        drafted += met.drafted
        got += toks
        ctx += toks
        pos += met.produced
        assert dec.kv_filled() == pos
    assert got[:steps] == want
    assert drafted > 0
    # decode_one from the prefilled state gives the same stream.
    dec1 = ora.LookupDecoder(m, 256)
    pos = dec1.prefill(prompt)
    last, plain = int(prompt[-1]), []
    for _ in range(steps):
        last = dec1.decode_one(pos, last)
        plain.append(last)
        pos += 1
    assert plain == want


# ------------------------------------------------------- product, host side --

def test_library_exports_every_declared_symbol(rai):
    """The C ABI library loads and exports every function include/rai_hip.h declares."""
    import re
    hdr = open(os.path.join(os.path.dirname(golden("")), "..", "..", "include", "rai_hip.h")).read()
    names = set(re.findall(r"^\s*(?:int|void|const char \*)\s*\*?\s*(rai_\w+)\s*\(", hdr, re.M))
    assert len(names) > 30
    lib = rai.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def _corrupt(data: bytes, off: int, val: bytes) -> bytes:
    b = bytearray(data)
    b[off:off + len(val)] = val
    return bytes(b)


@pytest.mark.parametrize("mutation,status", [
    (lambda d: b"XAIM" + d[4:], "RAI_E_FORMAT"),
    (lambda d: _corrupt(d, 4, struct.pack("<I", 3)), "RAI_E_FORMAT"),
    (lambda d: d[:40], "RAI_E_FORMAT"),
    (lambda d: d + b"\0", "RAI_E_FORMAT"),
    (lambda d: d[:-1], "RAI_E_FORMAT"),
    (lambda d: _corrupt(d, 48, b"\x03"), "RAI_E_FORMAT"),
    (lambda d: _corrupt(d, 49, b"\x03"), "RAI_E_FORMAT"),
    (lambda d: _corrupt(d, 24, struct.pack("<I", 12)), "RAI_E_FORMAT"),
    (lambda d: _corrupt(d, 52, struct.pack("<I", 9)), "RAI_E_FORMAT"),
    (lambda d: _corrupt(d, 44, struct.pack("<f", float("nan"))), "RAI_E_FORMAT"),
])
def test_hostile_files_are_rejected_before_upload(rai, mutation, status):
    """format.rs:1556-2173: malformed files are errors, never a wrong model.
    Validation happens on the host before any device call."""
    data = mutation(read_golden("tiny-untied.raimodel"))
    with pytest.raises(rai.RaiError) as e:
        rai.RaiModel.from_bytes(data)
    assert e.value.status == status


def test_invalid_scale_is_rejected(rai):
    """validate_group_params (format.rs:1492-1504): a zero or non-finite scale."""
    data = read_golden("tiny-untied.raimodel")
    secs = _sections(data)
    bad = _corrupt(data, secs[1][0] + 8, np.float16(0.0).tobytes())
    with pytest.raises(rai.RaiError) as e:
        rai.RaiModel.from_bytes(bad)
    assert e.value.status == "RAI_E_FORMAT"


def test_max_groups_gate(rai):
    """MAX_GROUPS (gemm.rs:1167): a group-32 model with K = 5632 needs 176
    groups and is refused at the reference limit; a raised limit admits it."""
    img = rai.synth_model(64, 1, 4, 2, 16, 5632, 96, 64, group_size=32, seed=1)
    with pytest.raises(rai.RaiError) as e:
        rai.RaiModel.from_bytes(img, max_groups=0)
    assert e.value.status == "RAI_E_FORMAT"
    assert "176" in str(e.value)
