"""GPU parity of draft-model speculative decoding (SpeculativeDecoder,
speculative.rs:61-391) with the oracle: every step's tokens and metrics are
equal, in the greedy variant and with exact sampling from the same seed.
A draft that is the target itself accepts every draft token (the
all-accepted branch: bonus token and the draft's catch-up forward); a
different draft exercises rejection and the residual correction.
"""
import numpy as np
import pytest

from rai_amd.workload import copy_heavy_prompt

pytestmark = pytest.mark.gpu


def _models(rai, ora):
    tgt = rai.synth_model(256, 3, 4, 2, 64, 512, 600, 512, group_size=32, seed=21)
    dft = rai.synth_model(128, 2, 4, 4, 32, 256, 600, 512, group_size=32, seed=22)
    return ((rai.RaiModel.from_bytes(dft), ora.Model(dft, 0)), (rai.RaiModel.from_bytes(tgt), ora.Model(tgt, 0)))


def _drive(rai, ora, gpair_d, gpair_t, k, temperature, seed, steps=24, max_ctx=256):
    (gd_m, od_m), (gt_m, ot_m) = gpair_d, gpair_t
    gd = rai.SpeculativeDecoder(gd_m, gt_m, max_ctx)
    od = ora.SpecDecoder(od_m, ot_m, max_ctx)
    gd.seed(seed)
    rng = ora.Rng(seed=seed)
    prompt = copy_heavy_prompt(40, 600, seed=seed)
    gpos, opos = gd.prefill(prompt), od.prefill(prompt)
    assert gpos == opos == 39
    last = int(prompt[-1])
    acc = drafted = 0
    for i in range(steps):
        gt, gm = gd.step(gpos, last, k, temperature)
        ot, om = od.step(opos, last, k, temperature, rng)
        assert gt == ot, (i, gt, ot)
        assert (gm["accepted"], gm["drafted"], gm["produced"]) == (om.accepted, om.drafted, om.produced), i
        assert gd.target_kv.filled(0) == gpos + gm["produced"]
        acc += gm["accepted"]
        drafted += gm["drafted"]
        gpos += gm["produced"]
        opos += om.produced
        last = gt[-1]
        if gpos + k + 2 >= max_ctx:
            break
    return acc, drafted


@pytest.mark.parametrize("k,temperature", [(4, 0.0), (8, 0.7), (1, 1.5)])
def test_speculative_matches_oracle(rai, ora, k, temperature):
    d, t = _models(rai, ora)
    acc, drafted = _drive(rai, ora, d, t, k, temperature, seed=k)
    assert drafted > 0


@pytest.mark.parametrize("temperature", [0.0, 0.9])
def test_self_draft_accepts_everything(rai, ora, temperature):
    """Draft == target: greedy drafts always match, and p_target / p_draft = 1
    accepts every sampled draft."""
    _, t = _models(rai, ora)
    acc, drafted = _drive(rai, ora, t, t, 6, temperature, seed=3, steps=12)
    assert acc == drafted > 0


def test_speculative_errors(rai):
    a = rai.RaiModel.from_bytes(rai.synth_model(128, 1, 4, 4, 32, 256, 600, 128, seed=1))
    b = rai.RaiModel.from_bytes(rai.synth_model(128, 1, 4, 4, 32, 256, 700, 128, seed=1))
    with pytest.raises(rai.RaiError):
        rai.SpeculativeDecoder(a, b, 64)  # vocabularies differ
    d = rai.SpeculativeDecoder(a, a, 64)
    pos = d.prefill(np.arange(10, dtype=np.uint32))
    with pytest.raises(rai.RaiError):
        d.step(pos, 5, 0, 0.5)  # draft_k = 0
    with pytest.raises(rai.RaiError):
        d.step(pos, 900, 2, 0.5)  # token outside the vocabulary


def test_greedy_speculation_equals_greedy_decoding(rai, ora):
    """The greedy variant of draft-model speculation emits the target's own
    greedy continuation whatever the draft (accepted drafts are the target's
    argmax, the first rejection emits it): its tokens equal the oracle's
    plain greedy decode of the target (decode_one, lookup.rs:428-455)."""
    d, t = _models(rai, ora)
    (gd_m, _), (gt_m, ot_m) = d, t
    prompt = copy_heavy_prompt(40, 600, seed=77)
    dec = rai.SpeculativeDecoder(gd_m, gt_m, 256)
    pos = dec.prefill(prompt)
    last, got = int(prompt[-1]), []
    while len(got) < 48:
        toks, _ = dec.step(pos, last, 5, 0.0)
        got += toks
        pos += len(toks)
        last = toks[-1]
    want = ot_m.greedy_generate(prompt.astype(np.int32), 48, 256).tolist()
    assert got[:48] == want


@pytest.mark.parametrize("temperature", [0.0, 0.9])
def test_draft_cache_is_whole_after_an_all_accepted_step(rai, ora, temperature):
    """After a step in which every draft is accepted, the draft model's
    catch-up row (position pos + k) is in the draft cache when the step
    returns: with the target as its own draft, the draft cache's K and V rows
    0..pos+k equal the oracle's for the same tokens, read right after the
    step through rai_kv_export."""
    _, (gm, om) = _models(rai, ora)
    prompt = copy_heavy_prompt(40, 600, seed=12)
    dec = rai.SpeculativeDecoder(gm, gm, 256)
    dec.seed(4)
    pos = dec.prefill(prompt)
    toks, met = dec.step(pos, int(prompt[-1]), 6, temperature)
    assert met["accepted"] == 6
    n = pos + 7  # rows 0 .. pos + k
    assert dec.draft_kv.filled(0) == n
    seq = prompt.tolist() + toks
    okv = om.create_kv(256)
    h = np.stack([om.embed_token(int(x)) for x in seq[:n]])
    om.forward_batch(h, np.arange(n), okv)
    cfg = om.cfg
    for layer in range(cfg.num_layers):
        for which in (0, 1):
            got = dec.draft_kv.export(layer, which, n, cfg.num_kv_heads, cfg.head_dim)
            get = okv.get_k if which == 0 else okv.get_v
            want = np.stack([np.stack([get(layer, hh, p, cfg.head_dim) for p in range(n)])
                             for hh in range(cfg.num_kv_heads)])
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (layer, which)
