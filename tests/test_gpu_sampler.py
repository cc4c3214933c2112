"""The plain sampler of `rai run` (no speculation) on the GPU against the
oracle: apply_repetition_penalty over the context, then sample_token with
the whole SamplerConfig (sampler.rs:47-199; run.rs:720-721).

Bar: the same token for every draw from the same StdRng seed, over
vocabularies of 1,000 to 50,304 and the configurations that reach each
branch: greedy (with the penalty), top-k alone (k = 1, k = 40, k = V - 1),
top-p alone (a nucleus of thousands of candidates, taken 1024 at a time on
the device), both, top-p = 0, NaN / +inf / all -inf rows, tied logits and
repeated context tokens.  Then the decode loop itself, and `rai-run`'s plain
mode with the reference's default options, token for token against the
oracle's decode loop on the same file.
"""
import os
import subprocess

import numpy as np
import pytest

from rai_amd.workload import copy_heavy_prompt

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUN = os.path.join(ROOT, "rai_amd", "lib", "rai-run")

CONFIGS = [  # temperature, top_k, top_p, repetition_penalty
    (0.7, 40, 0.9, 1.1),      # rai run's defaults
    (1.0, 0, 1.0, 1.0),       # plain softmax sampling
    (0.5, 1, 1.0, 1.0),       # top-k 1
    (1.2, 0, 0.9, 1.0),       # top-p alone: thousands of candidates
    (0.8, 5000, 0.5, 1.3),
    (0.0, 40, 0.9, 1.1),      # greedy after the penalty
    (1e-7, 0, 1.0, 1.0),      # greedy by the threshold
    (1.5, -1, 0.999, 0.5),    # top_k = V - 1, a penalty below 1
    (0.9, 0, 1e-6, 1.0),      # the top candidate only
    (2.0, 0, 0.0, 1.0),
]


def _logits(kind, V, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(V) * 2.5).astype(np.float32)
    if kind == "specials":
        x[rng.integers(0, V, 20)] = np.nan
        x[rng.integers(0, V, 3)] = np.inf
        x[rng.integers(0, V, 20)] = -np.inf
    elif kind == "ties":
        x = np.round(x).astype(np.float32)  # about a dozen distinct values, thousands of ties
    elif kind == "dead":
        x[:] = -np.inf
        x[rng.integers(0, V, 5)] = np.nan
    return x


@pytest.mark.parametrize("V", [1000, 32000, 50304])
@pytest.mark.parametrize("cfg", CONFIGS)
def test_sample_tokens_equal_oracle(rai, ora, V, cfg):
    t, k, p, pen = cfg
    k = V - 1 if k < 0 else k
    logits = _logits("normal", V, seed=V + int(100 * t) + k)
    recent = np.random.default_rng(V).integers(0, V, 300)
    recent[::7] = recent[0]  # repeated tokens are penalised once
    seed = 1234 + V
    got = rai.sample_tokens(logits, recent, rai.SamplerConfig(t, k, p, pen), seed, 48)
    rng = ora.Rng(seed=seed)
    want = [ora.sample_plain(logits, recent, t, k, p, pen, rng) for _ in range(48)]
    assert got == want


@pytest.mark.parametrize("kind", ["specials", "ties", "dead"])
@pytest.mark.parametrize("cfg", [(0.7, 40, 0.9, 1.1), (1.0, 0, 0.8, 1.0), (0.0, 0, 1.0, 1.0), (1.0, 3, 1.0, 0.7)])
def test_sample_tokens_special_rows_equal_oracle(rai, ora, kind, cfg):
    t, k, p, pen = cfg
    V = 4096
    logits = _logits(kind, V, seed=len(kind))
    recent = np.arange(0, V, 37)
    got = rai.sample_tokens(logits, recent, rai.SamplerConfig(t, k, p, pen), 77, 32)
    rng = ora.Rng(seed=77)
    want = [ora.sample_plain(logits, recent, t, k, p, pen, rng) for _ in range(32)]
    assert got == want


def _model(rai, ora):
    img = rai.synth_model(256, 2, 4, 2, 64, 512, 700, 512, group_size=32, seed=61)
    return img, rai.RaiModel.from_bytes(img), ora.Model(img, 0)


@pytest.mark.parametrize("cfg", [(0.7, 40, 0.9, 1.1), (1.0, 0, 1.0, 1.0), (0.9, 0, 0.95, 1.2)])
@pytest.mark.parametrize("graphs", ["1", "0"])
def test_sample_decode_equals_oracle(rai, ora, monkeypatch, cfg, graphs):
    """The decode loop (decode_one + penalty + sample_token per token) from a
    prefilled state equals the oracle's, step graphs on and off."""
    monkeypatch.setenv("RAI_STEP_GRAPHS", graphs)
    _, gm, om = _model(rai, ora)
    t, k, p, pen = cfg
    prompt = copy_heavy_prompt(70, 700, seed=3)
    gd, od = rai.LookupDecoder(gm, 512), ora.LookupDecoder(om, 512)
    gd.seed(99)
    pos = gd.prefill(prompt)
    assert od.prefill(prompt.astype(np.int32)) == pos
    got = gd.sample_decode(prompt, pos, 40, rai.SamplerConfig(t, k, p, pen))
    rng = ora.Rng(seed=99)
    ctx = prompt.astype(np.int32).tolist()
    want = []
    for i in range(40):
        tok = od.decode_sample(pos + i, ctx[-1], ctx, t, k, p, pen, rng)
        want.append(tok)
        ctx.append(tok)
    assert got == want


def test_rai_run_plain_defaults_equal_oracle(rai, ora, tmp_path):
    """`rai-run` without speculation and with the reference's defaults
    (temperature 0.7, top-k 40, top-p 0.9, repetition penalty 1.1, seed 42;
    run.rs:40-56) prints the oracle decode loop's tokens."""
    img, _, om = _model(rai, ora)
    path = str(tmp_path / "m.raimodel")
    with open(path, "wb") as f:
        f.write(bytes(img))
    prompt = copy_heavy_prompt(40, 700, seed=8)
    ids = ",".join(str(int(x)) for x in prompt)
    r = subprocess.run([RUN, path, "--prompt-ids", ids, "--max-tokens", "24"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    got = [int(x) for x in r.stdout.strip().split(",") if x]
    od = ora.LookupDecoder(om, 512)
    pos = od.prefill(prompt.astype(np.int32))
    rng = ora.Rng(seed=42)
    ctx = prompt.astype(np.int32).tolist()
    want = []
    for i in range(24):
        tok = od.decode_sample(pos + i, ctx[-1], ctx, 0.7, 40, 0.9, 1.1, rng)
        want.append(tok)
        ctx.append(tok)
    assert got == want
