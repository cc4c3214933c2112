"""GPU parity of the model-level path against the CPU oracle.

Bar: bit-exact logits and hidden states (the kernels reproduce the
reference's f32 operation order), identical greedy token streams, identical
per-step lookup metrics, and the reference's error behaviour.
"""
import numpy as np
import pytest

from conftest import read_golden
from rai_amd.workload import copy_heavy_prompt, uniform_prompt

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _token_sequence(vocab, n):
    state = 0x9E3779B97F4A7C15
    out = []
    for _ in range(n):
        state = (state * 6364136223846793005 + 1442695040888963407) & ((1 << 64) - 1)
        out.append((state >> 33) % vocab)
    return out


FIXTURES = ["tiny-tied.raimodel", "tiny-untied.raimodel", "tiny-convert.raimodel"]


def _small_synth(rai, **kw):
    args = dict(hidden_size=256, num_layers=3, num_heads=8, num_kv_heads=2, head_dim=32,
                intermediate_size=512, vocab_size=1000, max_context=1024, group_size=32, seed=7)
    args.update(kw)
    return rai.synth_model(args.pop("hidden_size"), args.pop("num_layers"), args.pop("num_heads"),
                           args.pop("num_kv_heads"), args.pop("head_dim"),
                           args.pop("intermediate_size"), args.pop("vocab_size"),
                           args.pop("max_context"), **args)


MODELS = {
    "tiny-tied": lambda rai: read_golden("tiny-tied.raimodel"),
    "tiny-untied": lambda rai: read_golden("tiny-untied.raimodel"),
    "tiny-convert": lambda rai: read_golden("tiny-convert.raimodel"),
    "synth-g32": lambda rai: _small_synth(rai),
    "synth-g128": lambda rai: _small_synth(rai, hidden_size=512, intermediate_size=1024,
                                           group_size=128, num_heads=4, head_dim=128, seed=2),
    "synth-gqa8-hd64": lambda rai: _small_synth(rai, num_heads=8, num_kv_heads=1, head_dim=64,
                                                hidden_size=512, seed=5),
}


@pytest.mark.parametrize("name", list(MODELS))
def test_embed_forward_logits_bit_exact(rai, ora, name):
    """embed_token, forward_batch and hidden_to_logits_batch equal the oracle
    bit for bit (model.rs:371-403, 692-1033)."""
    img = MODELS[name](rai)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    V = om.cfg.vocab_size
    toks = _token_sequence(V, 19)
    for t in toks[:3]:
        assert np.array_equal(_bits(gm.embed_token(t)), _bits(om.embed_token(t)))
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(64), gm.create_kv_cache(64)
    oh = om.forward_batch(hs[:11], np.arange(11), okv)
    gh = gm.forward_batch(hs[:11], np.arange(11), gkv)
    assert np.array_equal(_bits(gh), _bits(oh))
    # a second batch continuing from position 11 (verify-sized)
    oh2 = om.forward_batch(hs[11:], np.arange(11, 19), okv)
    gh2 = gm.forward_batch(hs[11:], np.arange(11, 19), gkv)
    assert np.array_equal(_bits(gh2), _bits(oh2))
    ol = om.hidden_to_logits_batch(np.concatenate([oh, oh2]), 19)
    gl = gm.hidden_to_logits_batch(np.concatenate([gh, gh2]), 19)
    assert np.array_equal(_bits(gl), _bits(ol))
    assert gkv.filled(0) == 19


@pytest.mark.parametrize("kw", [
    {},
    # 128 groups per row (the widest fused row), a 16384+-row lm_head (the
    # tiled kernel) and m1-kernel projections.
    dict(hidden_size=4096, num_layers=1, num_heads=32, num_kv_heads=8, head_dim=128,
         intermediate_size=1024, vocab_size=17000, max_context=64, seed=11),
])
def test_single_token_fused_norm_bit_exact(rai, ora, kw):
    """One-token forward and logits, where each projection behind a norm
    normalises and quantizes its input inside the GEMV launch, equal the
    oracle bit for bit after a few positions of context."""
    img = _small_synth(rai, **kw)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    toks = _token_sequence(om.cfg.vocab_size, 6)
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(64), gm.create_kv_cache(64)
    om.forward_batch(hs[:4], np.arange(4), okv)
    gm.forward_batch(hs[:4], np.arange(4), gkv)
    for p in (4, 5):
        oh = om.forward_batch(hs[p:p + 1], np.arange(p, p + 1), okv)
        gh = gm.forward_batch(hs[p:p + 1], np.arange(p, p + 1), gkv)
        assert np.array_equal(_bits(gh), _bits(oh)), p
        assert np.array_equal(_bits(gm.hidden_to_logits_batch(gh, 1)),
                              _bits(om.hidden_to_logits_batch(oh, 1))), p


@pytest.mark.parametrize("hd", [128, 96, 80])
def test_multi_token_attention_batches_bit_exact(rai, ora, hd):
    """Batches of 300, 13, 40 and 9 tokens continuing from earlier positions
    with four query heads per kv head: the PV kernel's several-token blocks
    (three tokens per block for nine, eight per block beyond twelve, the
    last block partial, several 128-position tiles) against the oracle's
    per-token chains, bit for bit.  head_dim 128 and 96 take the 32-dim
    slices with four tokens per compute lane, 80 the 16-dim slices with
    two."""
    img = _small_synth(rai, hidden_size=1024, num_layers=2, num_heads=8, num_kv_heads=2, head_dim=hd,
                       intermediate_size=1024, vocab_size=500, max_context=512, seed=23)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    toks = _token_sequence(om.cfg.vocab_size, 362)
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(512), gm.create_kv_cache(512)
    p = 0
    for n in (300, 13, 40, 9):
        oh = om.forward_batch(hs[p:p + n], np.arange(p, p + n), okv)
        gh = gm.forward_batch(hs[p:p + n], np.arange(p, p + n), gkv)
        assert np.array_equal(_bits(gh), _bits(oh)), (p, n)
        p += n


def test_hidden_3072_norm_chains_bit_exact(rai, ora):
    """Hidden 3072: the RMSNorm sum of squares runs its 16 chains as three
    register segments of 48 elements per lane (rows of 1024, 2048 and 4096
    take one, two and four), in the one-token GEMV prologue and the
    several-token norm+quantize kernel; forwards of 5, 1 and 9 tokens and
    their logits against the oracle, bit for bit."""
    img = _small_synth(rai, hidden_size=3072, num_layers=1, num_heads=24, num_kv_heads=8, head_dim=128,
                       intermediate_size=1024, vocab_size=500, max_context=64, seed=31)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    toks = _token_sequence(om.cfg.vocab_size, 15)
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(64), gm.create_kv_cache(64)
    p = 0
    for n in (5, 1, 9):
        oh = om.forward_batch(hs[p:p + n], np.arange(p, p + n), okv)
        gh = gm.forward_batch(hs[p:p + n], np.arange(p, p + n), gkv)
        assert np.array_equal(_bits(gh), _bits(oh)), (p, n)
        assert np.array_equal(_bits(gm.hidden_to_logits_batch(gh, n)),
                              _bits(om.hidden_to_logits_batch(oh, n))), (p, n)
        p += n


def test_single_token_short_context_one_launch_bit_exact(rai, ora):
    """One-token steps at every position from 0 to 389 with eight query
    heads per kv head and head_dim 64: up to 384 positions the scores, the
    softmax and PV run as one launch per kv head (fewer than 8 positions, a
    multiple of 8, every tail length 1..7), past it the separate kernels;
    hidden states bit for bit against the oracle."""
    img = _small_synth(rai, hidden_size=1024, num_layers=1, num_heads=16, num_kv_heads=2, head_dim=64,
                       intermediate_size=1024, vocab_size=500, max_context=512, seed=37)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    toks = _token_sequence(om.cfg.vocab_size, 390)
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(512), gm.create_kv_cache(512)
    for p in range(390):
        oh = om.forward_batch(hs[p:p + 1], np.arange(p, p + 1), okv)
        gh = gm.forward_batch(hs[p:p + 1], np.arange(p, p + 1), gkv)
        assert np.array_equal(_bits(gh), _bits(oh)), p


@pytest.mark.parametrize("graphs", ["1", "0"])
def test_short_context_greedy_lookup_equals_oracle(rai, ora, monkeypatch, graphs):
    """Greedy lookup decoding from a 40-token prompt through position 300
    with eight query heads per kv head and head_dim 64 (one-launch attention
    for one-token steps, step graphs captured per 256-position span), token
    for token against the oracle's decoder."""
    monkeypatch.setenv("RAI_STEP_GRAPHS", graphs)
    img = _small_synth(rai, hidden_size=1024, num_layers=2, num_heads=16, num_kv_heads=2, head_dim=64,
                       intermediate_size=1024, vocab_size=600, max_context=1024, seed=53)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    prompt = copy_heavy_prompt(40, 600, seed=9)
    cfg = rai.LookupConfig(max_draft=8, min_ngram=1, max_ngram=3)
    toks, _ = rai.LookupDecoder(gm, 1024).generate(prompt, 260, cfg)
    want = om.greedy_generate(prompt.astype(np.int32), len(toks), 1024).tolist()
    assert toks == want


def test_single_token_attention_long_context_bit_exact(rai, ora):
    """One-token steps after 1100 positions with four query heads per kv
    head and head_dim 128: the softmax's sum chains past their read-ahead,
    row tails of 5, 6, 7, 0 and 1 exact exponentials, and PV over five
    256-position V chunks, against the oracle, bit for bit."""
    img = _small_synth(rai, hidden_size=1024, num_layers=1, num_heads=8, num_kv_heads=2, head_dim=128,
                       intermediate_size=1024, vocab_size=500, max_context=2048, seed=29)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    toks = _token_sequence(om.cfg.vocab_size, 1105)
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(2048), gm.create_kv_cache(2048)
    om.forward_batch(hs[:1100], np.arange(1100), okv)
    gm.forward_batch(hs[:1100], np.arange(1100), gkv)
    for p in range(1100, 1105):
        oh = om.forward_batch(hs[p:p + 1], np.arange(p, p + 1), okv)
        gh = gm.forward_batch(hs[p:p + 1], np.arange(p, p + 1), gkv)
        assert np.array_equal(_bits(gh), _bits(oh)), p


@pytest.mark.parametrize("nh,nkv,hd", [(16, 16, 128), (16, 1, 64)])
def test_pv_head_groupings_bit_exact(rai, ora, nh, nkv, hd):
    """The PV kernel instances for one query head per kv head (head_dim 128,
    the OLMoE grouping) and sixteen (head_dim 64): one-token and nine-token
    batches after 600 positions, bit for bit against the oracle."""
    img = _small_synth(rai, hidden_size=1024, num_layers=1, num_heads=nh, num_kv_heads=nkv, head_dim=hd,
                       intermediate_size=1024, vocab_size=500, max_context=1024, seed=nh + nkv + hd)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    toks = _token_sequence(om.cfg.vocab_size, 610)
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(1024), gm.create_kv_cache(1024)
    for a, b in ((0, 600), (600, 601), (601, 610)):
        oh = om.forward_batch(hs[a:b], np.arange(a, b), okv)
        gh = gm.forward_batch(hs[a:b], np.arange(a, b), gkv)
        assert np.array_equal(_bits(gh), _bits(oh)), (a, b)


@pytest.mark.parametrize("nh,nkv,hd", [(8, 2, 128), (16, 2, 64), (8, 8, 128)])
def test_pv_long_context_through_kv_cache_bit_exact(rai, ora, nh, nkv, hd):
    """The production PV path (d-major V cache, LDS-flag tile hand-off) at
    4352 and 8192 positions, four, eight and one query heads per kv head: a
    one-token and a nine-token batch after each prefill, against the oracle
    bit for bit."""
    img = _small_synth(rai, hidden_size=1024, num_layers=1, num_heads=nh, num_kv_heads=nkv, head_dim=hd,
                       intermediate_size=1024, vocab_size=500, max_context=8256, seed=nh * hd)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    toks = _token_sequence(om.cfg.vocab_size, 8193)
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(8256), gm.create_kv_cache(8256)
    p = 0
    for end in (4342, 8183):
        om.forward_batch(hs[p:end], np.arange(p, end), okv)
        gm.forward_batch(hs[p:end], np.arange(p, end), gkv)
        for n in (1, 9):
            oh = om.forward_batch(hs[end:end + n], np.arange(end, end + n), okv)
            gh = gm.forward_batch(hs[end:end + n], np.arange(end, end + n), gkv)
            assert np.array_equal(_bits(gh), _bits(oh)), (end, n)
            end += n
        p = end
    assert gkv.filled(0) == 8193


def test_attention_wait_give_up_is_reported(rai, ora):
    """A PV tile hand-off wait that gives up (forced from the host with a
    poll limit of 1; every kernel still ends) fails the call with RAI_E_HIP
    and leaves the KV watermark where it was; with the default limit the
    same batch then runs and equals the oracle."""
    img = _small_synth(rai, hidden_size=1024, num_layers=1, num_heads=8, num_kv_heads=2, head_dim=128,
                       intermediate_size=1024, vocab_size=500, max_context=4096, seed=41)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    toks = _token_sequence(om.cfg.vocab_size, 2304)
    hs = np.stack([om.embed_token(t) for t in toks])
    okv, gkv = om.create_kv(4096), gm.create_kv_cache(4096)
    om.forward_batch(hs[:2048], np.arange(2048), okv)
    gm.forward_batch(hs[:2048], np.arange(2048), gkv)
    rai.set_attention_spin(1)
    try:
        with pytest.raises(rai.RaiError) as e:
            gm.forward_batch(hs[2048:], np.arange(2048, 2304), gkv)
        assert e.value.status == "RAI_E_HIP"
    finally:
        rai.set_attention_spin(0)
    assert gkv.filled(0) == 2048
    oh = om.forward_batch(hs[2048:], np.arange(2048, 2304), okv)
    gh = gm.forward_batch(hs[2048:], np.arange(2048, 2304), gkv)
    assert np.array_equal(_bits(gh), _bits(oh))


@pytest.mark.parametrize("max_context", [20000, 65536])
def test_step_graphs_with_large_capacity_match_oracle(rai, ora, max_context):
    """Decoders whose KV capacity exceeds the longest attention context (the
    step graphs size attention for min(capacity, 16384) positions) keep the
    oracle's tokens and metrics step by step, graphs on."""
    img = _small_synth(rai, max_context=max_context, seed=43)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    prompt = copy_heavy_prompt(300, 1000, seed=max_context)
    cfg = rai.LookupConfig(max_draft=8, min_ngram=1, max_ngram=3)
    gd, od = rai.LookupDecoder(gm, max_context), ora.LookupDecoder(om, max_context)
    gpos, opos = gd.prefill(prompt), od.prefill(prompt.astype(np.int32))
    ctx = prompt.tolist()
    for i in range(40):
        gt, gmet = gd.step(gpos, ctx, cfg)
        ot, omet = od.step(opos, ctx, 8, 1, 3)
        assert gt == ot, i
        assert (gmet.accepted, gmet.drafted, gmet.produced) == (omet.accepted, omet.drafted, omet.produced)
        ctx += gt
        gpos += gmet.produced
        opos += omet.produced


def test_step_graphs_with_a_long_context_match_eager(rai, monkeypatch):
    """Replayed steps read the position from the device step record and
    size the attention for the whole 8192-position cache; past 7168
    positions their token stream stays that of eager launches, which are
    sized for the live context."""
    img = _small_synth(rai, max_context=8192, seed=31)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    prompt = copy_heavy_prompt(7300, 1000, seed=4)
    cfg = rai.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3)
    monkeypatch.setenv("RAI_STEP_GRAPHS", "0")
    eager_toks, _ = rai.LookupDecoder(gm, 8192).generate(prompt, 40, cfg)
    monkeypatch.setenv("RAI_STEP_GRAPHS", "1")
    graph_toks, _ = rai.LookupDecoder(gm, 8192).generate(prompt, 40, cfg)
    assert graph_toks == eager_toks


@pytest.mark.parametrize("name", FIXTURES)
def test_batched_equals_sequential_on_gpu(rai, name):
    """model_invariants.rs:92-134 on the GPU path: batched and sequential
    forwards give bit-identical logits."""
    gm = rai.RaiModel.from_bytes(read_golden(name))
    V = gm.config.vocab_size
    toks = _token_sequence(V, 12)
    kv = gm.create_kv_cache(64)
    seq = []
    for p, t in enumerate(toks):
        seq.append(gm.hidden_to_logits(gm.forward_from_hidden(gm.embed_token(t), p, kv)))
    kv2 = gm.create_kv_cache(64)
    hb = gm.forward_batch(np.stack([gm.embed_token(t) for t in toks]), np.arange(12), kv2)
    lb = gm.hidden_to_logits_batch(hb, 12)
    for i in range(12):
        assert np.array_equal(_bits(lb[i]), _bits(seq[i]))


def test_kv_watermark_and_errors(rai):
    """kv_cache.rs:143-204 watermark rules and the lookup.rs/model.rs errors."""
    gm = rai.RaiModel.from_bytes(read_golden("tiny-untied.raimodel"))
    kv = gm.create_kv_cache(16)
    h = gm.embed_token(3)
    with pytest.raises(rai.RaiError) as e:
        gm.forward_from_hidden(h, 2, kv)  # gap: filled is 0
    assert e.value.status == "RAI_E_WATERMARK"
    gm.forward_from_hidden(h, 0, kv)
    gm.forward_from_hidden(h, 1, kv)
    assert kv.filled(0) == 2
    kv.get_k(0, 0, 1, 16)
    with pytest.raises(rai.RaiError) as e:
        kv.get_v(0, 0, 2, 16)
    assert e.value.status == "RAI_E_WATERMARK"
    kv.truncate(1)
    assert kv.filled(1) == 1
    with pytest.raises(rai.RaiError) as e:
        kv.get_k(0, 0, 1, 16)
    assert e.value.status == "RAI_E_WATERMARK"
    with pytest.raises(rai.RaiError) as e:
        gm.embed_token(96)
    assert e.value.status == "RAI_E_RANGE"
    with pytest.raises(rai.RaiError) as e:
        gm.forward_batch(np.stack([h, h]), [1, 3], kv)
    assert e.value.status == "RAI_E_ARG"
    with pytest.raises(rai.RaiError) as e:
        gm.forward_from_hidden(h, 16, kv)
    assert e.value.status in ("RAI_E_RANGE", "RAI_E_WATERMARK")


@pytest.mark.parametrize("name,prompt_len,steps,ngram", [
    ("synth-g32", 200, 48, (3, 3)),
    ("synth-g32", 64, 30, (1, 3)),
    ("tiny-untied", 40, 24, (1, 2)),
    ("tiny-tied", 30, 20, (1, 3)),
    ("synth-gqa8-hd64", 150, 40, (2, 3)),
])
def test_lookup_greedy_token_identity(rai, ora, name, prompt_len, steps, ngram):
    """Greedy prompt-lookup on the GPU: each step's tokens and metrics equal
    the oracle's LookupDecoder step, the KV watermark is the produced
    frontier (lookup.rs:411), and the whole stream equals the oracle's plain
    greedy decode."""
    img = MODELS[name](rai)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    V = om.cfg.vocab_size
    prompt = copy_heavy_prompt(prompt_len, V, seed=prompt_len)
    max_ctx = min(om.cfg.max_context, 512)
    cfg = rai.LookupConfig(max_draft=8, min_ngram=ngram[0], max_ngram=ngram[1], temperature=0.0)
    gd, od = rai.LookupDecoder(gm, max_ctx), ora.LookupDecoder(om, max_ctx)
    gpos, opos = gd.prefill(prompt), od.prefill(prompt.astype(np.int32))
    assert gpos == opos == prompt_len - 1
    ctx = prompt.tolist()
    got = []
    drafted = 0
    while len(got) < steps:
        gt, gmet = gd.step(gpos, ctx, cfg)
        ot, omet = od.step(opos, ctx, 8, ngram[0], ngram[1])
        assert gt == ot
        assert (gmet.accepted, gmet.drafted, gmet.produced) == (omet.accepted, omet.drafted,
                                                                omet.produced)
        assert (gmet.matched_ngram or 0) == omet.matched_ngram
        drafted += gmet.drafted
        got += gt
        ctx += gt
        gpos += gmet.produced
        opos += omet.produced
        assert gd.kv_cache.filled(0) == gpos
    want = om.greedy_generate(prompt.astype(np.int32), steps, max_ctx).tolist()
    assert got[:steps] == want
    assert drafted > 0


def test_lookup_step_next_search_follows_the_caller(rai, ora):
    """Each step also searches the next step's draft over its own extended
    context; a caller that continues differently (rewritten context tail,
    other search parameters, a rolled-back position) must get the search of
    what it passed.  Every step's tokens and metrics equal the oracle's on
    the same inputs."""
    img = MODELS["synth-g32"](rai)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    prompt = copy_heavy_prompt(200, om.cfg.vocab_size, seed=17)
    gd, od = rai.LookupDecoder(gm, 512), ora.LookupDecoder(om, 512)
    gpos, opos = gd.prefill(prompt), od.prefill(prompt.astype(np.int32))
    ctx = prompt.tolist()
    rng = np.random.default_rng(5)
    drafted = 0
    for i in range(40):
        kind = i % 4
        lo, hi = (1, 3) if kind == 2 else (3, 3)
        k = 4 if kind == 2 else 8
        if kind == 1:
            # Rewrite the tail with an earlier 3-gram (a forced draft).
            src = int(rng.integers(0, len(ctx) - 8))
            ctx[-3:] = ctx[src:src + 3]
        if kind == 3 and i > 4:
            # Roll back one token: position and context shrink together.
            ctx = ctx[:-1]
            gpos -= 1
            opos -= 1
            gd.kv_cache.truncate(gpos)
        cfg = rai.LookupConfig(max_draft=k, min_ngram=lo, max_ngram=hi, temperature=0.0)
        gt, gmet = gd.step(gpos, ctx, cfg)
        ot, omet = od.step(opos, ctx, k, lo, hi)
        assert gt == ot, i
        assert (gmet.accepted, gmet.drafted, gmet.produced) == (omet.accepted, omet.drafted, omet.produced), i
        assert (gmet.matched_ngram or 0) == omet.matched_ngram, i
        drafted += gmet.drafted
        ctx += gt
        gpos += gmet.produced
        opos += omet.produced
    assert drafted > 0


def test_lookup_generate_loop_matches_greedy(rai):
    """The native generate loop (cli/run.rs:517-633 without the tokenizer)
    produces the same stream as plain greedy decoding on the GPU."""
    img = _small_synth(rai, seed=11)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    prompt = copy_heavy_prompt(300, 1000, seed=3)
    cfg = rai.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3)
    toks, stats = rai.LookupDecoder(gm, 1024).generate(prompt, 64, cfg)
    want = rai.LookupDecoder(gm, 1024).greedy_generate(prompt, len(toks))
    assert toks == want
    assert stats["generated"] == len(toks) >= 64
    assert stats["steps"] <= stats["generated"]


def test_step_graph_replay_matches_eager(rai, monkeypatch):
    """The decode step replayed as a HIP graph (position read from the
    device step record, capacity-sized attention grids) produces the same
    token stream and metrics as eager launches, over enough steps that every
    verify size used is captured and replayed several times."""
    img = _small_synth(rai, seed=21)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    prompt = copy_heavy_prompt(260, 1000, seed=9)
    cfg = rai.LookupConfig(max_draft=8, min_ngram=1, max_ngram=3)
    monkeypatch.setenv("RAI_STEP_GRAPHS", "0")
    eager_toks, eager_stats = rai.LookupDecoder(gm, 1024).generate(prompt, 120, cfg)
    monkeypatch.setenv("RAI_STEP_GRAPHS", "1")
    graph_toks, graph_stats = rai.LookupDecoder(gm, 1024).generate(prompt, 120, cfg)
    assert graph_toks == eager_toks
    for key in ("steps", "steps_with_draft", "drafted", "accepted", "generated"):
        assert graph_stats[key] == eager_stats[key], key
    assert graph_toks == rai.LookupDecoder(gm, 1024).greedy_generate(prompt, len(graph_toks))


def test_lookup_config_errors(rai):
    """validate_lookup_config (lookup.rs:457-475); temperatures must be finite
    (above 1e-6 the step samples exactly, below it accepts greedily)."""
    gm = rai.RaiModel.from_bytes(read_golden("tiny-untied.raimodel"))
    d = rai.LookupDecoder(gm, 64)
    pos = d.prefill([1, 2, 3, 1, 2])
    for bad, status in ((dict(max_draft=0), "RAI_E_ARG"), (dict(min_ngram=0), "RAI_E_ARG"),
                        (dict(min_ngram=4, max_ngram=3), "RAI_E_ARG"),
                        (dict(temperature=float("inf")), "RAI_E_ARG")):
        with pytest.raises(rai.RaiError) as e:
            d.step(pos, [1, 2, 3, 1, 2], rai.LookupConfig(**bad))
        assert e.value.status == status
    with pytest.raises(rai.RaiError) as e:
        d.step(pos, [1, 2, 3, 1, 200], rai.LookupConfig())
    assert e.value.status == "RAI_E_RANGE"


def test_moe_forward_bit_exact(rai, ora):
    """OLMoE-shaped routing (layers.rs:1808-1870, model.rs:208-261): softmax
    over all experts, top-k, weighted accumulation in selection order."""
    img = rai.synth_model(128, 2, 4, 4, 32, 64, 500, 256, group_size=32, num_experts=8,
                          experts_per_token=3, seed=4)
    om = ora.Model(img, 0)
    gm = rai.RaiModel.from_bytes(img)
    toks = _token_sequence(500, 9)
    hs = np.stack([om.embed_token(t) for t in toks])
    oh = om.forward_batch(hs, np.arange(9), om.create_kv(32))
    gh = gm.forward_batch(hs, np.arange(9), gm.create_kv_cache(32))
    assert np.array_equal(_bits(gh), _bits(oh))
    assert np.array_equal(_bits(gm.hidden_to_logits_batch(gh, 9)),
                          _bits(om.hidden_to_logits_batch(oh, 9)))


def test_tinyllama_shape_lookup_identity(rai):
    """Full TinyLlama shape (22 layers, g32, K=5632 needs 176 groups):
    greedy prompt-lookup equals plain greedy decoding on the GPU, and both
    layer-0 KV rows are written (a size-independent property)."""
    from rai_amd.workload import TINYLLAMA
    s = dict(TINYLLAMA)
    img = rai.synth_model(s["hidden_size"], s["num_layers"], s["num_heads"], s["num_kv_heads"],
                          s["head_dim"], s["intermediate_size"], s["vocab_size"], 1024,
                          group_size=32, seed=1)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    del img
    prompt = copy_heavy_prompt(256, s["vocab_size"], seed=8)
    cfg = rai.LookupConfig(max_draft=8, min_ngram=3, max_ngram=3)
    toks, stats = rai.LookupDecoder(gm, 1024).generate(prompt, 48, cfg)
    want = rai.LookupDecoder(gm, 1024).greedy_generate(prompt, len(toks))
    assert toks == want
