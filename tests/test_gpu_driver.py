"""The drop-in surface around the decode loop, on the GPU:

- RaiModel::load from a .raimodel path (format.rs:557-637) gives the same
  model as the in-memory image (bit-identical logits), and refuses a
  missing or truncated file;
- KVCache::clear (kv_cache.rs) resets every watermark;
- rai-run, the `rai run` generate loop (run.rs:242-633) over the C ABI,
  prints the same tokens as the library's own loops for prompt lookup
  (greedy and sampled, same seed), draft-model speculation and plain
  greedy decoding, and the same tokens as the CPU oracle's decoders on the
  same file;
- the path-loaded model's logits equal the oracle's on the file's bytes.
"""
import os
import subprocess

import numpy as np
import pytest

from rai_amd.workload import copy_heavy_prompt

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUN = os.path.join(ROOT, "rai_amd", "lib", "rai-run")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def model_file(rai, tmp_path_factory):
    d = tmp_path_factory.mktemp("models")
    path = str(d / "m.raimodel")
    rai.synth_model(256, 2, 4, 2, 64, 512, 600, 512, group_size=32, seed=31, path=path)
    draft = str(d / "draft.raimodel")
    rai.synth_model(128, 1, 4, 4, 32, 256, 600, 512, group_size=32, seed=32, path=draft)
    return path, draft


def test_load_from_path_equals_image(rai, model_file):
    path, _ = model_file
    a = rai.RaiModel.load(path)
    with open(path, "rb") as f:
        b = rai.RaiModel.from_bytes(f.read())
    h = np.stack([a.embed_token(t) for t in (3, 9, 27, 81)])
    la = a.hidden_to_logits_batch(a.forward_batch(h, np.arange(4), a.create_kv_cache(16)), 4)
    lb = b.hidden_to_logits_batch(b.forward_batch(h, np.arange(4), b.create_kv_cache(16)), 4)
    assert np.array_equal(_bits(la), _bits(lb))


def test_load_errors(rai, model_file, tmp_path):
    path, _ = model_file
    with pytest.raises(rai.RaiError):
        rai.RaiModel.load(str(tmp_path / "missing.raimodel"))
    cut = tmp_path / "cut.raimodel"
    with open(path, "rb") as f:
        cut.write_bytes(f.read()[:5000])
    with pytest.raises(rai.RaiError):
        rai.RaiModel.load(str(cut))


def test_kv_clear_resets_watermarks(rai, model_file):
    m = rai.RaiModel.load(model_file[0])
    kv = m.create_kv_cache(32)
    m.forward_batch(np.stack([m.embed_token(t) for t in range(5)]), np.arange(5), kv)
    assert kv.filled(0) == 5 and kv.filled(1) == 5
    kv.clear()
    assert kv.filled(0) == 0 and kv.filled(1) == 0
    m.forward_batch(np.stack([m.embed_token(7)]), np.arange(1), kv)  # position 0 is valid again
    assert kv.filled(1) == 1


# Speculative modes need the neutral sampler options (run.rs:134-215); so do
# comparisons with plain greedy decoding, which the default penalty of 1.1
# would change.
NEUTRAL = ["--top-k", "0", "--top-p", "1", "--repetition-penalty", "1"]


def _run(args):
    r = subprocess.run([RUN] + args, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return [int(x) for x in r.stdout.strip().split(",") if x]


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_rai_run_lookup_equals_library(rai, model_file, temperature):
    path, _ = model_file
    prompt = copy_heavy_prompt(60, 600, seed=8)
    ids = ",".join(str(int(t)) for t in prompt)
    got = _run([path, "--prompt-ids", ids, "--max-tokens", "40", "--lookup-k", "6", "--lookup-ngram", "3",
                "--lookup-min-ngram", "1", "--temperature", str(temperature), "--seed", "5"] + NEUTRAL)
    m = rai.RaiModel.load(path)
    dec = rai.LookupDecoder(m, 512)
    dec.seed(5)
    cfg = rai.LookupConfig(max_draft=6, max_ngram=3, min_ngram=1, temperature=temperature)
    pos = dec.prefill(prompt)
    ctx = prompt.tolist()
    want = []
    while len(want) < 40:
        toks, met = dec.step(pos, ctx, cfg)
        take = toks[:40 - len(want)]
        want += take
        ctx += take
        pos += len(take)
    assert got == want


def test_rai_run_draft_and_plain_equal_library(rai, model_file):
    path, draft = model_file
    prompt = copy_heavy_prompt(30, 600, seed=9)
    ids = ",".join(str(int(t)) for t in prompt)
    got = _run([path, "--prompt-ids", ids, "--max-tokens", "24", "--draft", draft, "--draft-k", "4",
                "--temperature", "0.9", "--seed", "11"] + NEUTRAL)
    t, d = rai.RaiModel.load(path), rai.RaiModel.load(draft)
    dec = rai.SpeculativeDecoder(d, t, 512)
    dec.seed(11)
    pos = dec.prefill(prompt)
    last, want = int(prompt[-1]), []
    while len(want) < 24:
        toks, met = dec.step(pos, last, 4, 0.9)
        take = toks[:24 - len(want)]
        want += take
        pos += len(take)
        last = take[-1]
    assert got == want
    plain = _run([path, "--prompt-ids", ids, "--max-tokens", "16", "--temperature", "0"] + NEUTRAL)
    assert plain == rai.LookupDecoder(t, 512).greedy_generate(prompt, 16)


def test_rai_run_rejects_bad_arguments(model_file):
    path, draft = model_file
    r = subprocess.run([RUN, path, "--prompt-ids", "1,2", "--lookup-k", "2", "--draft", draft],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "mutually exclusive" in r.stderr
    # Speculation with the default top-k / top-p / penalty, and options out
    # of range.
    for bad in (["--lookup-k", "2"], ["--draft", draft, "--top-k", "0", "--top-p", "1"], ["--top-p", "0"],
                ["--repetition-penalty", "5"], ["--temperature", "2.5"]):
        r = subprocess.run([RUN, path, "--prompt-ids", "1,2"] + bad, capture_output=True, text=True, timeout=60)
        assert r.returncode == 2, bad


def _oracle(ora, path):
    with open(path, "rb") as f:
        return ora.Model(f.read(), 0)


def test_load_from_path_matches_oracle(rai, ora, model_file):
    """RaiModel::load (format.rs:557-637) of a file: embedding rows, hidden
    states and logits equal the oracle's reading of the same bytes."""
    path, draft = model_file
    for p in (path, draft):
        g, o = rai.RaiModel.load(p), _oracle(ora, p)
        toks = [3, 9, 27, 81, 243, 599]
        for t in toks[:2]:
            assert np.array_equal(_bits(g.embed_token(t)), _bits(o.embed_token(t)))
        h = np.stack([o.embed_token(t) for t in toks])
        gh = g.forward_batch(h, np.arange(6), g.create_kv_cache(16))
        oh = o.forward_batch(h, np.arange(6), o.create_kv(16))
        assert np.array_equal(_bits(gh), _bits(oh))
        assert np.array_equal(_bits(g.hidden_to_logits_batch(gh, 6)), _bits(o.hidden_to_logits_batch(oh, 6)))


def test_rai_run_plain_greedy_matches_oracle(rai, ora, model_file):
    """`rai run` without speculation at temperature 0 (run.rs:640-735:
    prefill of the first N - 1 tokens, then one decode per token) prints the
    oracle's greedy decode of the same file."""
    path, _ = model_file
    prompt = copy_heavy_prompt(50, 600, seed=21)
    ids = ",".join(str(int(t)) for t in prompt)
    got = _run([path, "--prompt-ids", ids, "--max-tokens", "32", "--temperature", "0"] + NEUTRAL)
    want = _oracle(ora, path).greedy_generate(prompt.astype(np.int32), 32, 512).tolist()
    assert got == want


@pytest.mark.parametrize("temperature", [0.0, 0.8])
def test_rai_run_lookup_matches_oracle(rai, ora, model_file, temperature):
    """`rai run --lookup-k 6` (run.rs:517-633) prints the oracle
    LookupDecoder's tokens: greedy, and sampled with the oracle's StdRng
    seeded as the driver seeds the decoder's (run.rs:345)."""
    path, _ = model_file
    prompt = copy_heavy_prompt(60, 600, seed=8)
    ids = ",".join(str(int(t)) for t in prompt)
    got = _run([path, "--prompt-ids", ids, "--max-tokens", "40", "--lookup-k", "6", "--lookup-ngram", "3",
                "--lookup-min-ngram", "1", "--temperature", str(temperature), "--seed", "5"] + NEUTRAL)
    od = ora.LookupDecoder(_oracle(ora, path), 512)
    rng = ora.Rng(seed=5)
    pos = od.prefill(prompt.astype(np.int32))
    ctx = prompt.tolist()
    want = []
    while len(want) < 40:
        if temperature > 0:
            toks, met = od.step_sampled(pos, ctx, 6, 1, 3, temperature, rng)
        else:
            toks, met = od.step(pos, ctx, 6, 1, 3)
        take = toks[:40 - len(want)]
        want += take
        ctx += take
        pos += len(take)
    assert got == want


@pytest.mark.parametrize("temperature", [0.0, 0.9])
def test_rai_run_draft_matches_oracle(rai, ora, model_file, temperature):
    """`rai run --draft` (run.rs:405-517) prints the oracle
    SpeculativeDecoder's tokens for the same seed."""
    path, draft = model_file
    prompt = copy_heavy_prompt(30, 600, seed=9)
    ids = ",".join(str(int(t)) for t in prompt)
    got = _run([path, "--prompt-ids", ids, "--max-tokens", "24", "--draft", draft, "--draft-k", "4",
                "--temperature", str(temperature), "--seed", "11"] + NEUTRAL)
    od = ora.SpecDecoder(_oracle(ora, draft), _oracle(ora, path), 512)
    rng = ora.Rng(seed=11)
    pos = od.prefill(prompt.astype(np.int32))
    last, want = int(prompt[-1]), []
    while len(want) < 24:
        toks, met = od.step(pos, last, 4, temperature, rng)
        take = toks[:24 - len(want)]
        want += take
        pos += len(take)
        last = take[-1]
    assert got == want
