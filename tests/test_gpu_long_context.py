"""Contexts past 16,384 positions, up to the model's max_context.

The reference accepts any position below the header's max_context
(format.rs:158, MAX_CONTEXT 1,000,000), grows its KV cache by doubling
(kv_cache.rs:105-126) and runs attention over every cached position with no
length cap (layers.rs:1266-1380, 1675-1747).  These tests hand both sides the
same cached K/V rows (rai_kv_import / the oracle's KVCache import, the bulk
form of KVCache::store), then run forward passes and prompt-lookup steps at
20,000 and 32,768 positions and compare bit for bit.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CAP = 32800  # above 32,768 so the last step's attention span is the capacity


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# One layer at two head groupings of the configs: four query heads per kv
# head at head_dim 128 (the 7B shape) and eight at head_dim 64 (the 1.1B).
SHAPES = {
    "g4-hd128": dict(hidden_size=512, num_heads=4, num_kv_heads=1, head_dim=128),
    "g8-hd64": dict(hidden_size=512, num_heads=8, num_kv_heads=1, head_dim=64),
}


def _model(rai, shape, seed):
    s = SHAPES[shape]
    return rai.synth_model(s["hidden_size"], 1, s["num_heads"], s["num_kv_heads"], s["head_dim"], 1024, 1000,
                           CAP, group_size=32, seed=seed)


def _kv_rows(cfg, npos, seed):
    """Random cached rows [nkv][npos][hd]: keys of unit scale (scores spread
    over a few units, so the softmax is far from a point mass) and values."""
    rng = np.random.default_rng(seed)
    shape = (cfg.num_kv_heads, npos, cfg.head_dim)
    k = (rng.standard_normal(shape, np.float32) * np.float32(0.25)).astype(np.float32)
    v = rng.standard_normal(shape, np.float32)
    return k, v


@pytest.mark.parametrize("shape", list(SHAPES))
@pytest.mark.parametrize("pos,m", [(20000, 1), (20000, 9), (20000, 80), (32759, 9), (32767, 1)])
def test_forward_past_16384_positions_bit_exact(rai, ora, shape, pos, m):
    """forward_batch at positions pos..pos+m-1 over pos imported cache rows:
    hidden states, the rows the pass stores and the logits equal the
    oracle's (one token: the fused one-token path; nine: the verify path;
    80: the prefill path's 64-token attention groups)."""
    img = _model(rai, shape, seed=pos + m)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    cfg = om.cfg
    k, v = _kv_rows(cfg, pos, seed=pos * 3 + m)
    okv, gkv = om.create_kv(CAP), gm.create_kv_cache(CAP)
    for kv in (okv, gkv):
        kv.import_rows(0, 0, k)
        kv.import_rows(0, 1, v)
    rng = np.random.default_rng(m)
    toks = rng.integers(0, cfg.vocab_size, m)
    hs = np.stack([om.embed_token(int(t)) for t in toks])
    oh = om.forward_batch(hs, np.arange(pos, pos + m), okv)
    gh = gm.forward_batch(hs, np.arange(pos, pos + m), gkv)
    assert np.array_equal(_bits(gh), _bits(oh))
    assert gkv.filled(0) == pos + m
    for p in (pos, pos + m - 1):
        assert np.array_equal(_bits(gkv.export(0, 0, pos + m, cfg.num_kv_heads, cfg.head_dim)[:, p]),
                              _bits(np.stack([okv.get_k(0, h, p, cfg.head_dim) for h in range(cfg.num_kv_heads)])))
    ol = om.hidden_to_logits_batch(oh, m)
    gl = gm.hidden_to_logits_batch(gh, m)
    assert np.array_equal(_bits(gl), _bits(ol))


def _context_without_repeats(n, vocab, seed):
    """n token ids in which no 3-gram occurs twice (so a min_ngram = 3 search
    finds no draft)."""
    rng = np.random.default_rng(seed)
    out, seen = [], set()
    while len(out) < n:
        t = int(rng.integers(0, vocab))
        if len(out) >= 2 and (out[-2], out[-1], t) in seen:
            continue
        if len(out) >= 2:
            seen.add((out[-2], out[-1], t))
        out.append(t)
    return out


def _periodic_context(n, vocab, period, seed):
    """n token ids repeating one random span: every suffix 3-gram recurs, so
    each step drafts the full k tokens."""
    rng = np.random.default_rng(seed)
    span = rng.integers(0, vocab, period).tolist()
    return [span[i % period] for i in range(n)]


@pytest.mark.parametrize("graphs", ["1", "0"])
@pytest.mark.parametrize("pos,kind", [(20000, "verify"), (20000, "decode"), (32762, "verify"),
                                      (32765, "decode")])
def test_lookup_steps_past_16384_positions_match_oracle(rai, ora, monkeypatch, graphs, pos, kind):
    """Prompt-lookup steps (k = 8, n-gram 3) from an imported cache state at
    20,000 and ~32,768 positions, with step graphs on (per attention span:
    first use eager, then captured and replayed; the steps from 32,762 and
    32,765 reach past 32,768 positions, into the span that ends at the
    capacity) and off: tokens and metrics equal the oracle's step by step."""
    monkeypatch.setenv("RAI_STEP_GRAPHS", graphs)
    img = _model(rai, "g4-hd128", seed=11)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    cfg = om.cfg
    gd, od = rai.LookupDecoder(gm, CAP), ora.LookupDecoder(om, CAP)
    k, v = _kv_rows(cfg, pos, seed=pos)
    for which, rows in ((0, k), (1, v)):
        gd.kv_cache.import_rows(0, which, rows)
        od.import_kv(0, which, rows)
    # The caller's context (LookupDecoder::step takes it from the caller):
    # a periodic one, so each step drafts the full k tokens, or one without
    # a repeated 3-gram, so no step drafts.  The tokens a step produces
    # advance the position; the context keeps its own continuation.
    n = pos + 64
    if kind == "verify":
        seq = _periodic_context(n, cfg.vocab_size, 97, seed=pos)
    else:
        seq = _context_without_repeats(n, cfg.vocab_size, seed=pos)
    lcfg = rai.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3)
    steps = 0
    while steps < 7 and pos + 9 < CAP:
        ctx = seq[:pos + 1]
        gt, gmet = gd.step(pos, ctx, lcfg)
        ot, omet = od.step(pos, ctx, 8, 3, 3)
        assert gt == ot, (steps, pos)
        assert (gmet.accepted, gmet.drafted, gmet.produced) == (omet.accepted, omet.drafted, omet.produced)
        assert gmet.drafted == (8 if kind == "verify" else 0)
        pos += gmet.produced
        steps += 1
    assert steps >= 3


def test_kv_import_round_trip_and_errors(rai):
    """rai_kv_import is rai_kv_export's inverse (K rows and d-major V rows),
    sets the watermark, and refuses positions past the cache."""
    img = _model(rai, "g8-hd64", seed=3)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    cfg = gm.config
    kv = gm.create_kv_cache(300)
    k, v = _kv_rows(cfg, 257, seed=9)
    kv.import_rows(0, 0, k)
    kv.import_rows(0, 1, v)
    assert kv.filled(0) == 257
    assert np.array_equal(kv.export(0, 0, 257, cfg.num_kv_heads, cfg.head_dim), k)
    assert np.array_equal(kv.export(0, 1, 257, cfg.num_kv_heads, cfg.head_dim), v)
    with pytest.raises(rai.RaiError) as e:
        kv.import_rows(0, 0, np.zeros((cfg.num_kv_heads, 301, cfg.head_dim), np.float32))
    assert e.value.status == "RAI_E_RANGE"
