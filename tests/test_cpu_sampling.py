"""CPU pins of the oracle's exact-sampling restatement (test infrastructure).

- ChaCha block function, counter/stream layout and four-block buffering:
  RFC 7539 A.1 keystream test vectors 1 and 2 (20 rounds, zero key and
  nonce; they are also rand_chacha's ChaCha20 zero-seed true values) and
  the RFC 8439 2.3.2 block-function vector.
- BlockRng reads: next_u64 = two consecutive words, low first, including
  across a refill (rand_core 0.6.4 BlockRng::next_u64).
- softmax_probabilities (speculative.rs:431-477) against a float64 softmax
  and its special cases (NaN, +inf, all -inf).
- sample_token's own tests (sampler.rs:228-306), mirrored.
- The speculative-sampling identity the accept / correct / bonus loop
  exists for (lookup.rs:359-403): the first emitted token is distributed as
  the target's softmax whatever the draft; a correction drawn from the
  target instead of the residual max(0, p - q) fails it.
StdRng::seed_from_u64 and the f32/f64 conversions have no published vector:
parity-unpinned beyond their published algorithm (rand_core 0.6.4, rand 0.8.6).
"""
import numpy as np
import pytest

from oracle import ora

RFC7539_TV1 = [0xade0b876, 0x903df1a0, 0xe56a5d40, 0x28bd8653, 0xb819d2bd, 0x1aed8da0, 0xccef36a8, 0xc70d778b,
               0x7c5941da, 0x8d485751, 0x3fe02477, 0x374ad8b8, 0xf4b8436a, 0x1ca11815, 0x69b687c3, 0x8665eeb2]
RFC7539_TV2 = [0xbee7079f, 0x7a385155, 0x7c97ba98, 0x0d082d73, 0xa0290fcb, 0x6965e348, 0x3e53c612, 0xed7aee32,
               0x7621b729, 0x434ee69c, 0xb03371d5, 0xd539d874, 0x281fed31, 0x45fb0a51, 0x1f0ae1ac, 0x6f4d794b]
RFC8439_232 = [0xe4e7f110, 0x15593bd1, 0x1fdd0f50, 0xc47120a3, 0xc7f4d1c7, 0x0368c033, 0x9aaa2204, 0x4e6cd4c3,
               0x466482d2, 0x09aa9f07, 0x05d7c214, 0xa2028bd9, 0xd19c12b5, 0xb94e16de, 0xe883d0cb, 0x4e3c50a2]


def test_chacha20_zero_key_keystream_through_the_buffer():
    r = ora.Rng(key=np.zeros(8, np.uint32), rounds=20)
    assert [r.next_u32() for _ in range(32)] == RFC7539_TV1 + RFC7539_TV2


def test_chacha20_block_function_rfc8439():
    key = np.arange(32, dtype=np.uint8).view(np.uint32)
    # RFC 8439 nonce 00:00:00:09:00:00:00:4a:00:00:00:00 over the 64-bit
    # counter (words 12-13) and 64-bit stream (words 14-15) layout.
    got = ora.chacha_block(key, 1 | (0x09000000 << 32), 0x4a000000, 20)
    assert got.tolist() == RFC8439_232


@pytest.mark.parametrize("skip", [0, 1, 61, 62, 63, 64, 65, 127])
def test_u64_reads_are_consecutive_words_across_refills(skip):
    a, b = ora.Rng(seed=77), ora.Rng(seed=77)
    for _ in range(skip):
        a.next_u32()
    words = [b.next_u32() for _ in range(skip + 6)]
    got = [a.next_u64() for _ in range(3)]
    want = [words[skip + 2 * i] | (words[skip + 2 * i + 1] << 32) for i in range(3)]
    assert got == want


def test_rounds_parameter_changes_the_stream():
    assert ora.Rng(seed=1, rounds=12).next_u32() != ora.Rng(seed=1, rounds=20).next_u32()


def test_softmax_probabilities_against_float64():
    rng = np.random.default_rng(3)
    for t in (0.3, 0.7, 1.0, 2.5):
        x = (rng.normal(size=513) * 4).astype(np.float32)
        p = ora.softmax_probabilities(x, t)
        z = x.astype(np.float64) / t
        want = np.exp(z - z.max())
        want /= want.sum()
        assert np.allclose(p, want, rtol=2e-5, atol=1e-9), t


def test_softmax_probabilities_special_cases():
    p = ora.softmax_probabilities([np.nan, 0.0, 1.0], 1.0)
    assert p[0] == 0.0 and abs(p.sum() - 1.0) < 1e-6
    p = ora.softmax_probabilities([np.inf, 2.0, np.inf, -np.inf], 0.5)
    assert p.tolist() == [0.5, 0.0, 0.5, 0.0]
    p = ora.softmax_probabilities([-np.inf, np.nan, -np.inf, -np.inf], 1.0)
    assert p.tolist() == [0.25] * 4


def test_sample_token_reference_tests():
    """sampler.rs:228-306: low temperature concentrates on the top logit;
    non-finite logits never select NaN; greedy below 1e-6."""
    rng = ora.Rng(seed=42)
    counts = np.zeros(3, int)
    for _ in range(100):
        counts[ora.sample_token([1.0, 2.0, 3.0], 0.1, rng)] += 1
    assert counts[2] > 90
    rng = ora.Rng(seed=7)
    assert ora.sample_token([np.nan, 1.0, 2.0], 0.0, rng) == 2
    for _ in range(32):
        assert ora.sample_token([np.inf, np.inf, 0.0, np.nan], 0.7, rng) < 2
    assert ora.sample_token([np.nan, -np.inf], 0.7, rng) < 2


@pytest.mark.parametrize("draft", [0, 2, 4])
def test_accept_and_correct_preserve_the_target_distribution(draft):
    """Speculative sampling's identity: with a point-mass draft on `draft`,
    the first emitted token is distributed as softmax(target / T)."""
    logits = np.array([[1.0, 0.2, 2.0, -1.0, 0.5], [0.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    t = 0.8
    p = ora.softmax_probabilities(logits[0], t).astype(np.float64)
    rng = ora.Rng(seed=100 + draft)
    n = 20000
    counts = np.zeros(5)
    for _ in range(n):
        toks, acc = ora.sampled_accept(logits, [draft], t, rng)
        counts[toks[0]] += 1
        assert (acc == 1) == (toks[0] == draft) and len(toks) == 1 + acc
    chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
    assert chi2 < 25.0, (counts / n, p)  # 4 degrees of freedom: p < 1e-4 for a correct rule


def test_bonus_token_follows_the_last_row():
    logits = np.array([[0.0] * 4, [3.0, 0.0, 1.0, 2.0]], np.float32)
    logits[0, 1] = 30.0  # the draft (1) is accepted with probability ~1
    t = 1.3
    p = ora.softmax_probabilities(logits[1], t).astype(np.float64)
    rng = ora.Rng(seed=5)
    n = 12000
    counts = np.zeros(4)
    for _ in range(n):
        toks, acc = ora.sampled_accept(logits, [1], t, rng)
        assert acc == 1 and toks[0] == 1
        counts[toks[1]] += 1
    chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
    assert chi2 < 22.0, (counts / n, p)


@pytest.mark.parametrize("t", [0.6, 1.0])
def test_draft_model_acceptance_preserves_the_target_distribution(t):
    """SpeculativeDecoder's acceptance (speculative.rs:329-350) with
    sample_correction's residual max(0, p - q) (speculative.rs:478-513),
    with a draft distribution q that is not a point mass: the draft token is
    drawn from q, and the first emitted token must follow p =
    softmax(target / T) (chi-squared over 20000 draws), with the draft
    accepted at the rate sum(min(p, q)).  The same checks have the power to
    reject two plausible mistakes: a correction drawn from p instead of the
    residual, and an acceptance test against p_target instead of
    p_target / p_draft."""
    target = np.array([[1.0, 0.2, 2.0, -1.0, 0.5], [0.3, -0.4, 1.1, 0.0, 0.9]], np.float32)
    draft = np.array([[0.1, 1.5, 1.8, 0.4, -0.3]], np.float32)
    p = ora.softmax_probabilities(target[0], t).astype(np.float64)
    q = ora.softmax_probabilities(draft[0], t).astype(np.float64)
    q /= q.sum()
    pick = np.random.default_rng(int(t * 100))
    rng = ora.Rng(seed=int(t * 1000) + 3)
    n = 20000
    counts = np.zeros(5)
    accepted = 0
    for _ in range(n):
        d = int(pick.choice(5, p=q))
        toks, acc = ora.spec_accept(target, draft, [d], t, rng)
        assert (acc == 1) == (toks[0] == d) and len(toks) == 1 + acc
        counts[toks[0]] += 1
        accepted += acc
    limit = 25.0  # 4 degrees of freedom: p < 1e-4 for a correct rule
    chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
    assert chi2 < limit, (counts / n, p)
    beta = np.minimum(p, q).sum()
    sigma = np.sqrt(n * beta * (1 - beta))
    assert abs(accepted - n * beta) < 5 * sigma, (accepted / n, beta)
    # Power: the expected statistic of each mistaken rule is far past the limits.
    wrong_correction = np.minimum(p, q) + (1.0 - beta) * p
    assert n * ((wrong_correction - p) ** 2 / p).sum() > 4 * limit
    assert abs(n * (q * p).sum() - n * beta) > 20 * sigma


# ---- sample_token with the whole SamplerConfig and the repetition penalty --
# (sampler.rs:47-199: the `rai run` token without speculation)

def _softmax64(x):
    z = np.asarray(x, np.float64)
    e = np.exp(z - z.max())
    return e / e.sum()


def test_sampler_reference_tests_mirrored():
    """sampler.rs:216-317: greedy pick, low temperature concentration, the
    penalty on one token (and once per distinct token), top-k = 2 keeping
    only the two largest, non-finite logits, non-finite options falling back
    (T NaN = greedy, top_p NaN = 1, penalty NaN = none)."""
    rng = ora.Rng(seed=42)
    assert ora.sample_plain([1.0, 5.0, 2.0, 3.0], [], 0.0, 40, 0.9, 1.0, rng) == 1
    counts = np.zeros(3, int)
    for _ in range(100):
        counts[ora.sample_plain([1.0, 2.0, 3.0], [], 0.1, 0, 1.0, 1.0, rng)] += 1
    assert counts[2] > 90
    # [1, 2, 3, 4] with token 3 penalised by 2 -> [1, 2, 3, 2]: greedy picks 2.
    assert ora.sample_plain([1.0, 2.0, 3.0, 4.0], [3], 0.0, 0, 1.0, 2.0, rng) == 2
    # once per distinct token: [1, 4] -> [1, 2] (argmax 1), not [1, 0.5].
    assert ora.sample_plain([1.0, 4.0], [1, 1, 1], 0.0, 0, 1.0, 2.0, rng) == 1
    # a negative logit is multiplied: [-1, -3] with token 0 penalised by 4 -> [-4, -3].
    assert ora.sample_plain([-1.0, -3.0], [0], 0.0, 0, 1.0, 4.0, rng) == 1
    counts = np.zeros(5, int)
    for _ in range(200):
        counts[ora.sample_plain([1.0, 5.0, 3.0, 4.0, 2.0], [], 1.0, 2, 1.0, 1.0, rng)] += 1
    assert counts[0] == counts[2] == counts[4] == 0 and counts[1] > 0 and counts[3] > 0
    assert ora.sample_plain([np.nan, 1.0, 2.0], [], 0.0, 40, 0.9, 1.1, rng) == 2
    for _ in range(32):
        assert ora.sample_plain([np.inf, np.inf, 0.0, np.nan], [], 0.7, 40, 0.9, 1.0, rng) < 2
    assert ora.sample_plain([np.nan, -np.inf], [], 0.7, 40, 0.9, 1.0, rng) < 2
    assert ora.sample_plain([1.0, 3.0, 2.0], [], np.nan, (1 << 62), np.nan, np.nan, rng) == 1
    # penalty NaN changes nothing: [1, 4] stays, greedy 1.
    assert ora.sample_plain([1.0, 4.0], [1], 0.0, 0, 1.0, np.nan, rng) == 1


def _nucleus(p, top_p):
    order = sorted(range(len(p)), key=lambda i: (-p[i], i))
    keep, cum = [], 0.0
    for i in order:
        keep.append(i)
        cum += p[i]
        if cum >= top_p:
            break
    q = np.zeros(len(p))
    q[keep] = p[keep]
    return q / q.sum()


@pytest.mark.parametrize("t,top_k,top_p,penalty", [(0.8, 3, 1.0, 1.0), (1.0, 0, 0.6, 1.0), (0.7, 5, 0.9, 1.3),
                                                   (1.3, 0, 0.95, 0.5)])
def test_sampler_distribution_against_float64(t, top_k, top_p, penalty):
    """The draws follow the distribution the config defines, computed here
    in float64 from the definitions (penalty on the distinct recent tokens,
    x / T, the k largest, softmax, the smallest descending prefix reaching
    top_p, renormalised): chi-squared over 20000 draws.  Keeping one
    nucleus token too many, or filtering k + 1 tokens, moves the expected
    statistic far past the limit (checked here)."""
    logits = np.array([1.2, -0.4, 2.0, 0.3, 1.7, -1.5, 0.9, 2.4, 0.0, 1.1], np.float32)
    recent = [7, 2, 7, 5]
    x = logits.astype(np.float64).copy()
    if abs(penalty - 1.0) >= 1e-6:
        for tkn in set(recent):
            x[tkn] = x[tkn] / penalty if x[tkn] > 0 else x[tkn] * penalty
    x = x / t
    if 0 < top_k < len(x):
        thr = np.sort(x)[::-1][top_k - 1]
        x = np.where(x < thr, -np.inf, x)
    p = _softmax64(x)
    q = _nucleus(p, top_p) if top_p < 1 else p
    rng = ora.Rng(seed=int(1000 * t) + top_k)
    n = 20000
    counts = np.zeros(len(logits))
    for _ in range(n):
        counts[ora.sample_plain(logits, recent, t, top_k, top_p, penalty, rng)] += 1
    assert np.all(counts[q == 0] == 0), (counts, q)
    live = q > 0
    chi2 = ((counts[live] - n * q[live]) ** 2 / (n * q[live])).sum()
    dof = int(live.sum()) - 1
    limit = dof + 8 * np.sqrt(2 * dof) + 10
    assert chi2 < limit, (chi2, counts / n, q)
    # Power against plausible mistakes.
    if top_p < 1:
        order = sorted(range(len(p)), key=lambda i: (-p[i], i))
        k_in = int((q > 0).sum())
        if k_in < int((p > 0).sum()):
            wrong = np.zeros(len(p))
            wrong[order[:k_in + 1]] = p[order[:k_in + 1]]
            wrong /= wrong.sum()
            assert n * (((wrong - q) ** 2)[live] / q[live]).sum() + n * wrong[~live].sum() > 4 * limit
    if 0 < top_k < len(x) - 1 and top_p >= 1 and abs(penalty - 1.0) < 1e-6:
        # Filtering at the (k + 1)-th value instead of the k-th: the extra
        # token would show up in the draws about this often.
        z = np.asarray(logits, np.float64) / t
        wrong = _softmax64(np.where(z < np.sort(z)[::-1][top_k], -np.inf, z))
        assert n * wrong[~live].sum() > 50
