"""CPU pins for the oracle functions no reference fixture covers: RoPE tables
and rotation, the tied 8-bit head, MoE routing, the layer composition of
forward_batch, and the expf restatement the kernels use for exact tails.

Each check is chosen so that a plausible mistake fails it: a wrong RoPE
exponent or sign, adjacent instead of half-split pairs, a GQA head map of
qh % nkv, swapped norms, a missing residual, a wrong attention scale, ties
resolved to the highest expert index, or renormalised expert weights.
"""
import os
import struct
import subprocess

import numpy as np
import pytest

from conftest import ROOT, read_golden
from textbook_model import TextbookModel


# ------------------------------------------------------------------- RoPE --

@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("theta", [1e4, 1e6])
def test_rope_tables_against_float64(ora, hd, theta):
    """RoPETable::with_scaling (layers.rs:561-633): cos/sin(p * theta^(-2i/hd)).
    The f32 table's angle carries the rounding of inv_freq and of p * inv_freq
    (a few ulps of the angle); a wrong exponent or a flipped sign is O(1)."""
    c, s = ora.rope_tables(hd, 4096, theta)
    half = hd // 2
    inv = theta ** (-2.0 * np.arange(half) / hd)
    for p in (1, 7, 4095):
        ang = p * inv
        tol = 1e-6 + 4e-7 * ang  # f32 rounding of inv_freq and of the product
        assert np.all(np.abs(c[p] - np.cos(ang)) <= tol), p
        assert np.all(np.abs(s[p] - np.sin(ang)) <= tol), p
    assert np.array_equal(c[0], np.ones(half, np.float32))
    assert np.array_equal(s[0], np.zeros(half, np.float32))


@pytest.mark.parametrize("hd,nh", [(16, 3), (64, 2), (128, 4)])
def test_rope_apply_half_split_rotation(ora, hd, nh):
    """RoPETable::apply (layers.rs:689-726) at position 1 is the rotation of the
    pairs (i, i + hd/2): x0' = x0 c - x1 s, x1' = x1 c + x0 s."""
    c, s = ora.rope_tables(hd, 4, 10000.0)
    rng = np.random.default_rng(hd)
    h = rng.normal(size=nh * hd).astype(np.float32)
    got = ora.rope_apply(h, nh, hd, c[1], s[1]).reshape(nh, hd).astype(np.float64)
    x = h.reshape(nh, hd).astype(np.float64)
    half = hd // 2
    cc, ss = c[1].astype(np.float64), s[1].astype(np.float64)
    want = np.concatenate([x[:, :half] * cc - x[:, half:] * ss, x[:, half:] * cc + x[:, :half] * ss], axis=1)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    # the mistaken sign / pairing differ by far more than that
    wrong_sign = np.concatenate([x[:, :half] * cc + x[:, half:] * ss, x[:, half:] * cc - x[:, :half] * ss], axis=1)
    assert np.abs(got - wrong_sign).max() > 0.1


# -------------------------------------------------------------- tied head --

def test_tied_lm_head_exact_input(ora):
    """Mirror of gemm.rs:2703-2741: vocab 1200, hidden 256, group 64, codes
    (i*31+7) % 256, every group scale 0.03125 and zero -4.0 (f16), a hidden
    vector whose +-63 quantization is exact; the f64 dequantized product
    within 5e-3 * max(|e|, 1)."""
    vocab, hidden, gs = 1200, 256, 64
    codes = ((np.arange(vocab * hidden) * 31 + 7) % 256).astype(np.uint8)
    groups = hidden // gs
    par = np.empty((vocab * groups, 2), np.float16)
    par[:, 0], par[:, 1] = 0.03125, -4.0
    j = np.arange(hidden) % gs
    t = np.where(j == 0, 63, (j * 37) % 127 - 63)
    h = (t / 63.0).astype(np.float32)
    got = ora.tied_lm_head(h, codes, par.view(np.uint8).reshape(-1), vocab, gs).astype(np.float64)
    w = codes.reshape(vocab, hidden).astype(np.float64) * 0.03125 - 4.0
    want = w @ h.astype(np.float64)
    assert np.all(np.abs(got - want) <= 5e-3 * np.maximum(np.abs(want), 1.0))
    # the quantization really is exact here: the int path equals the f64 sum
    # up to the f32 epilogue
    assert np.allclose(got, want, rtol=1e-5, atol=1e-3)


# ---------------------------------------------------------------- routing --

def _route_f64(router, x, k, norm):
    logits = router.astype(np.float64) @ x.astype(np.float64)
    p = np.exp(logits - logits.max())
    p /= p.sum()
    order = sorted(range(len(p)), key=lambda e: (-p[e], e))[:k]
    w = p[order]
    if norm:
        w = w / w.sum()
    return order, w


@pytest.mark.parametrize("norm", [False, True])
def test_route_experts_brute_force_and_ties(ora, norm):
    """route_experts (layers.rs:1808-1870): softmax over all experts, then
    the top k; exact ties (identical router rows) go to the lowest index."""
    rng = np.random.default_rng(7)
    E, H, k = 16, 64, 5
    for trial in range(20):
        router = rng.normal(size=(E, H)).astype(np.float32) * 0.3
        x = rng.normal(size=H).astype(np.float32)
        if trial % 2 == 0:
            # exact ties among the strongest experts
            best = int(np.argmax(router @ x))
            for e in rng.choice([e for e in range(E) if e != best], size=3, replace=False):
                router[e] = router[best]
        sel, wts = ora.route_experts(router, x, E, k, norm)
        order, w = _route_f64(router, x, k, norm)
        assert sel.tolist() == order, (trial, sel, order)
        assert np.allclose(wts, w, rtol=1e-5, atol=1e-7)
        tied = [e for e in sel if np.array_equal(router[e], router[sel[0]])]
        assert tied == sorted(tied)


# ------------------------------------------------------------ composition --

def _truncate_layers(img: bytes, n: int) -> bytes:
    """The same model with only its first n layers (sections rewritten)."""
    d = bytes(img)
    hsz = 64 if struct.unpack_from("<I", d, 4)[0] == 1 else 128
    L = struct.unpack_from("<I", d, 12)[0]
    nsec = struct.unpack_from("<I", d, 52)[0]
    secs = [struct.unpack_from("<QQ", d, hsz + 16 * i) for i in range(nsec)]
    keep = [secs[0]] + secs[1:1 + n] + secs[1 + L:]
    hdr = bytearray(d[:hsz])
    struct.pack_into("<I", hdr, 12, n)
    struct.pack_into("<I", hdr, 52, len(keep))
    off, table, body = hsz + 16 * len(keep), b"", b""
    for o, s in keep:
        table += struct.pack("<QQ", off, s)
        body += d[o:o + s]
        off += s
    return bytes(hdr) + table + body


def _composition_models(rai):
    # One layer each: across layers the occasional int8 boundary crossings
    # (see MEDIAN_TOL) cascade into later quantizations.
    return {
        "tiny-tied": _truncate_layers(read_golden("tiny-tied.raimodel"), 1),
        "tiny-untied": _truncate_layers(read_golden("tiny-untied.raimodel"), 1),
        "tiny-convert": _truncate_layers(read_golden("tiny-convert.raimodel"), 1),
        # four query heads per kv head
        "gqa4": bytes(rai.synth_model(128, 1, 8, 2, 16, 256, 300, 256, group_size=32, seed=3,
                                      weight_std=0.05)),
        # OLMoE-style routing: 8 experts, top 3, softmax over all
        "moe": bytes(rai.synth_model(128, 1, 4, 4, 32, 64, 200, 256, group_size=32, num_experts=8,
                                     experts_per_token=3, seed=4, weight_std=0.1)),
    }


# The textbook model differs from the f32 oracle by f32 rounding, which now and
# then moves an int8 activation across a rounding boundary (a local jump of
# ~ws*as); the median relative difference over all hidden values is therefore
# small (measured <= 1.7e-4), while every planted composition mistake moves
# most values (measured >= 8.5e-3).  The fixtures' second layer is dropped
# (the file's sections rewritten) for the same reason.
MEDIAN_TOL = 1e-3

MISTAKES = {
    "tiny-tied": ["gqa", "rope_sign", "rope_pairs", "no_attn_residual", "norm_swap", "scale"],
    "tiny-untied": ["gqa", "rope_sign", "rope_pairs", "no_attn_residual", "norm_swap", "scale"],
    "tiny-convert": ["gqa", "rope_sign", "rope_pairs", "no_attn_residual", "norm_swap", "scale"],
    "gqa4": ["gqa", "rope_sign", "rope_pairs", "no_attn_residual", "scale"],
    "moe": ["rope_sign", "no_attn_residual", "scale", "moe_renorm"],
}


def _oracle_hidden_logits(ora, img, toks):
    om = ora.Model(img, 0)
    hs = np.stack([om.embed_token(t) for t in toks])
    oh = om.forward_batch(hs, np.arange(len(toks)), om.create_kv(64))
    return oh.astype(np.float64), om.hidden_to_logits_batch(oh, len(toks)).astype(np.float64)


def _median_rel(a, b):
    return float(np.median(np.abs(a - b)) / np.abs(b).max())


@pytest.mark.parametrize("name", list(MISTAKES))
def test_forward_composition_against_float64_textbook(ora, rai, name):
    """forward_batch + hidden_to_logits_batch (model.rs:692-1033) against an
    independent float64 statement of the model (tests/textbook_model.py):
    hidden states and logits of 40 tokens at positions 0..39, and the argmax
    of the logits.  Then each planted composition mistake in the textbook
    model must move the comparison far past the tolerance."""
    img = _composition_models(rai)[name]
    V = struct.unpack_from("<I", img, 32)[0]
    toks = np.random.default_rng(1).integers(0, V, 40).tolist()
    oh, ol = _oracle_hidden_logits(ora, img, toks)
    tb = TextbookModel(img)
    th = tb.hidden(toks)
    tl = tb.logits(th)
    assert _median_rel(th, oh) <= MEDIAN_TOL
    assert _median_rel(tl, ol) <= 5 * MEDIAN_TOL
    top = np.sort(tl, axis=1)
    clear = top[:, -1] - top[:, -2] > 1e-2 * np.abs(tl).max()  # no near-tie
    assert np.array_equal(ol.argmax(1)[clear], tl.argmax(1)[clear])
    for mk in MISTAKES[name]:
        bad = TextbookModel(img, mk).hidden(toks)
        assert _median_rel(bad, oh) > 5 * MEDIAN_TOL, mk


# ------------------------------------------------------------------- expf --

def test_expf_restatement_matches_host_libm(tmp_path):
    """rai_amd/csrc/exact_math.h's expf_glibc (the exact tails of the softmax,
    SiLU and the router on the GPU) equals the host C library's expf on a
    strided sample of every float bit pattern in [-110, 89]."""
    exe = tmp_path / "exact_math_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I",
                    os.path.join(ROOT, "rai_amd", "csrc"), os.path.join(ROOT, "tests", "exact_math_check.cpp"),
                    "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe), "-110", "89", "97"], check=True, capture_output=True, text=True).stdout
    checked, bad, first = out.split()
    assert int(checked) > 20_000_000
    assert int(bad) == 0, f"first mismatch at {first}"


# The PCG32 reference implementation's demo (pcg32_srandom_r(42, 54), then
# pcg32_random_r): its published first outputs.
_PCG_DEMO_42_54 = [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_seed_from_u64_against_the_pcg32_reference_vector(ora):
    """SeedableRng::seed_from_u64 (rand_core 0.6.4) fills the ChaCha key with
    PCG32 outputs: state = state * 6364136223846793005 + 11634580027462260723,
    then the XSH RR output of the new state.  The PCG reference demo runs the
    same multiplier and output function with increment 109 (sequence 54).
    For each state S_k the demo outputs from, the seed (S_k - increment) /
    multiplier (mod 2^64) makes the oracle's first step land on S_k, so its
    first key word must be the demo's k-th output: a wrong output function,
    multiplier, increment or step order fails it."""
    m64, mul, inc_rand = 1 << 64, 6364136223846793005, 11634580027462260723
    inv = pow(mul, -1, m64)
    inc = (54 << 1) | 1  # pcg32_srandom_r(initstate = 42, initseq = 54)
    s = (0 * mul + inc) % m64
    s = (s + 42) % m64
    s = (s * mul + inc) % m64
    for k, want in enumerate(_PCG_DEMO_42_54):
        seed = ((s - inc_rand) * inv) % m64
        assert int(ora.Rng(seed=seed).key()[0]) == want, k
        s = (s * mul + inc) % m64


class _Pcg32:
    """rand_pcg 0.3's Lcg64Xsh32 (Pcg32): state and stream words, XSH RR
    output of the state before each step."""

    MUL = 6364136223846793005

    def __init__(self, state, stream):
        self.inc = ((stream << 1) | 1) % (1 << 64)
        self.state = (state + self.inc) % (1 << 64)
        self._step()

    def _step(self):
        self.state = (self.state * self.MUL + self.inc) % (1 << 64)

    def next_u32(self):
        s = self.state
        self._step()
        xs = (((s >> 18) ^ s) >> 27) & 0xFFFFFFFF
        rot = s >> 59
        return ((xs >> rot) | (xs << ((32 - rot) & 31))) & 0xFFFFFFFF

    def next_u64(self):
        lo = self.next_u32()
        return lo | (self.next_u32() << 32)


def test_standard_float_conversions_against_rand_value_stability(ora):
    """rand 0.8's Standard f32 / f64 against that crate's own value-stability
    vectors (distributions/float.rs), drawn from its test generator
    Pcg32(0x6f44f5646c2a7334, 11634580027462260723).  The generator is
    restated here and checked first against the PCG32 reference demo (seed
    42, sequence 54: pcg32_srandom_r runs the same steps as this
    constructor), so a wrong conversion in the oracle (bits kept, scale,
    rounding) is what a mismatch points to."""
    demo = _Pcg32(42, 54)
    assert [demo.next_u32() for _ in range(6)] == _PCG_DEMO_42_54
    rng = _Pcg32(0x6F44F5646C2A7334, 11634580027462260723)
    f32 = [np.float32(ora.Rng.standard_f32(rng.next_u32())) for _ in range(3)]
    assert f32 == [np.float32(0.0035963655), np.float32(0.7346052), np.float32(0.09778172)]
    rng = _Pcg32(0x6F44F5646C2A7334, 11634580027462260723)
    f64 = [ora.Rng.standard_f64(rng.next_u64()) for _ in range(3)]
    assert f64 == [0.7346051961657583, 0.20298547462974248, 0.8166436635290655]
    # gen_f32 / gen_f64 apply the same conversion to the ChaCha stream.
    a, b = ora.Rng(seed=5), ora.Rng(seed=5)
    assert a.gen_f32() == np.float32(ora.Rng.standard_f32(b.next_u32()))
    assert a.gen_f64() == ora.Rng.standard_f64(b.next_u64())
