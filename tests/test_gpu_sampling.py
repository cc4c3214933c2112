"""GPU parity of exact-sampling prompt lookup (lookup.rs:359-403,
speculative.rs:414-513, sampler.rs:47-182) with the oracle.

The device generator's draws equal the oracle's StdRng (whose ChaCha block
function and buffering are pinned by the RFC vectors in
test_cpu_sampling.py) bit for bit, and sampled lookup steps driven over the
same contexts with the same seed produce the same tokens and metrics.
"""
import os

import numpy as np
import pytest

from rai_amd.workload import copy_heavy_prompt

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _oracle_draw(r, k):
    if k == 0:
        return r.next_u32()
    if k == 1:
        return r.next_u64()
    if k == 2:
        return int(np.float32(r.gen_f32()).view(np.uint32))
    return int(np.float64(r.gen_f64()).view(np.uint64))


@pytest.mark.parametrize("seed", [0, 42, 2**63 + 5])
def test_device_rng_matches_oracle(rai, ora, seed):
    rng = np.random.default_rng(seed % 1000)
    kinds = rng.integers(0, 4, size=700)
    kinds[60:70] = 1  # u64 reads across the first refill at odd and even indices
    got = rai.std_rng_draws(seed, kinds)
    r = ora.Rng(seed=seed)
    want = [_oracle_draw(r, int(k)) for k in kinds]
    assert got.tolist() == want


def _drive(rai, ora, gm, om, prompt, steps, temperature, seed, ngram, max_ctx=256, force_every=3):
    cfg = rai.LookupConfig(max_draft=8, min_ngram=ngram[0], max_ngram=ngram[1], temperature=temperature)
    gd, od = rai.LookupDecoder(gm, max_ctx), ora.LookupDecoder(om, max_ctx)
    gd.seed(seed)
    orng = ora.Rng(seed=seed)
    gpos, opos = gd.prefill(prompt), od.prefill(prompt.astype(np.int32))
    ctx = prompt.tolist()
    drafted = accepted = 0
    for i in range(steps):
        if force_every and i % force_every == 1 and len(ctx) > 40:
            src = 5 + (11 * i) % (len(ctx) - 30)
            ctx[-3:] = ctx[src:src + 3]
        gt, gmet = gd.step(gpos, ctx, cfg)
        ot, omet = od.step_sampled(opos, ctx, 8, ngram[0], ngram[1], temperature, orng)
        assert gt == ot, (i, gt, ot)
        assert (gmet.accepted, gmet.drafted, gmet.produced) == (omet.accepted, omet.drafted, omet.produced), i
        drafted += gmet.drafted
        accepted += gmet.accepted
        ctx += gt
        gpos += gmet.produced
        opos += omet.produced
        if gpos + 10 >= max_ctx:
            break
    return drafted, accepted


@pytest.mark.parametrize("temperature,seed", [(0.05, 1), (0.8, 2), (3.0, 3)])
def test_sampled_lookup_matches_oracle(rai, ora, temperature, seed):
    """Tiny fixture (vocab small enough that drafts are accepted at low
    temperature and corrected at high temperature); step graphs replay."""
    with open(os.path.join(ROOT, "tests", "golden", "tiny-untied.raimodel"), "rb") as f:
        data = f.read()
    gm = rai.RaiModel.from_bytes(data)
    om = ora.Model(data, 128)
    prompt = copy_heavy_prompt(64, 96, seed=seed)  # the fixture's vocabulary: 96 ids
    drafted, accepted = _drive(rai, ora, gm, om, prompt, 60, temperature, seed, (1, 3))
    assert drafted > 0
    if temperature < 0.1:
        assert accepted > 0


def test_sampled_lookup_mistral_width_matches_oracle(rai, ora):
    """Sampled steps at a 32000-token vocabulary (the sum and search chains
    at full length) on a 2-layer Mistral-width model."""
    from rai_amd.workload import MISTRAL_7B as s
    img = rai.synth_model(s["hidden_size"], 2, s["num_heads"], s["num_kv_heads"], s["head_dim"],
                          s["intermediate_size"], s["vocab_size"], 256, group_size=32, seed=11)
    gm = rai.RaiModel.from_bytes(img, max_groups=1024)
    om = ora.Model(img, 0)
    del img
    prompt = copy_heavy_prompt(48, s["vocab_size"], seed=4)
    drafted, _ = _drive(rai, ora, gm, om, prompt, 12, 1.0, 9, (3, 3))
    assert drafted > 0


def test_temperature_must_be_finite(rai):
    with open(os.path.join(ROOT, "tests", "golden", "tiny-untied.raimodel"), "rb") as f:
        gm = rai.RaiModel.from_bytes(f.read())
    d = rai.LookupDecoder(gm, 64)
    pos = d.prefill(np.arange(10, dtype=np.uint32))
    with pytest.raises(rai.RaiError):
        d.step(pos, list(range(10)), rai.LookupConfig(max_draft=4, temperature=float("nan")))
