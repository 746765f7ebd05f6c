"""The token sampler (dwim inference/sampler.rs): the oracle's restatement
pinned on the CPU, then the device's (dwim_sampler_*) against it.

Pins of the oracle, each chosen so that a plausible slip fails one:
  * the reference's own unit tests (sampler.rs:148-196), restated;
  * the generator: its first state from seed 1 worked out by hand, and its
    draws uniform on [0, 1);
  * the candidates: the order (larger logit first, the lower index among
    equal ones, -0 equal to 0), the clamp of top_k, the softmax against a
    float64 one, and the top_p / min_p cut against its definition;
  * sample: the picks' frequencies against the kept probabilities;
  * verify: a certain draft always kept; a draft outside the kept set never,
    its replacements distributed as the kept tokens; a draft of probability
    p kept at a rate p.
The device sampler must then give the oracle's tokens, acceptances and
generator state, call after call, on the same logits and settings.
"""
import numpy as np
import pytest

import oracle as O


def _logits(vocab, seed, scale=3.0):
    return (np.random.default_rng(seed).standard_normal(vocab) * scale).astype(np.float32)


# ---- the oracle ------------------------------------------------------------


def test_reference_unit_tests():
    # picks_from_the_top_k_in_order (sampler.rs:151-170)
    logits = np.zeros(1000, np.float32)
    logits[7], logits[300], logits[999] = 5.0, 4.0, 3.0
    assert O.Sampler(0.0, 20, 0.95, 0.0, 1).sample(logits) == 7
    s = O.Sampler(1.0, 3, 0.01, 0.0, 1)
    assert all(s.sample(logits) == 7 for _ in range(20))
    s = O.Sampler(100.0, 2, 1.0, 0.0, 1)
    picks = {s.sample(logits) for _ in range(200)}
    assert 7 in picks and 300 in picks and 999 not in picks
    # drops_tokens_far_less_likely_than_the_top (sampler.rs:172-195)
    logits[999] = 0.0
    s = O.Sampler(1.0, 1000, 1.0, 0.1, 1)
    picks = {s.sample(logits) for _ in range(200)}
    assert picks == {7, 300}
    s = O.Sampler(1.0, 1000, 1.0, 1.0, 1)
    assert all(s.sample(logits) == 7 for _ in range(20))


def test_generator_first_state_and_uniformity():
    # from state 1: s ^= s >> 12 leaves 1; s ^= s << 25 gives 2^25 + 1; s >> 27
    # is then 0, so the third step leaves it
    v, s = O.xorshift_next(1)
    assert s == (1 << 25) + 1 and 0.0 <= v < 1.0
    # seed 0 starts from 1 (Rng(seed.max(1)))
    assert O.Sampler(0.0, 1, 1.0, 0.0, 0).rng == 1 and O.Sampler(0.0, 1, 1.0, 0.0, 9).rng == 9
    draws, st = [], 12345
    for _ in range(100_000):
        x, st = O.xorshift_next(st)
        draws.append(x)
    d = np.array(draws)
    assert d.min() >= 0.0 and d.max() < 1.0
    assert abs(d.mean() - 0.5) < 0.005
    # 16 bins, chi-square well inside the 0.999 quantile of 15 degrees (37.7)
    counts = np.bincount((d * 16).astype(int), minlength=16)
    chi2 = ((counts - len(d) / 16) ** 2 / (len(d) / 16)).sum()
    assert chi2 < 37.7
    # the 24-bit values are exact multiples of 2^-24
    assert np.all(d * (1 << 24) == np.floor(d * (1 << 24)))


def test_candidates_order_and_cut():
    x = np.array([1.0, 3.0, -0.0, 3.0, 0.0, 2.0, 3.0, -1.0], np.float32)
    s = O.Sampler(1.0, 5, 1.0, 0.0, 1)
    tok, pr, tot = s.candidates(x)
    # the three 3.0s in index order, then 2.0, then 1.0
    assert list(tok) == [1, 3, 6, 5, 0]
    want = np.exp(np.float64(x[tok]) - 3.0)
    want /= want.sum()
    np.testing.assert_allclose(pr, want, rtol=2e-6)
    assert abs(tot - float(np.float32(pr.sum()))) < 1e-6
    # -0 and 0 tie: the lower index first
    y = np.array([-1.0, 0.0, -0.0, -2.0], np.float32)
    assert list(O.Sampler(1.0, 2, 1.0, 0.0, 1).candidates(y)[0]) == [1, 2]
    z = np.array([-1.0, -0.0, 0.0, -2.0], np.float32)
    assert list(O.Sampler(1.0, 2, 1.0, 0.0, 1).candidates(z)[0]) == [1, 2]
    # top_k beyond the vocabulary, and zero, are clamped
    assert len(O.Sampler(1.0, 100, 1.0, 0.0, 1).candidates(x)[0]) == 8
    assert list(O.Sampler(1.0, 0, 1.0, 0.0, 1).candidates(x)[0]) == [1]
    # temperature zero: the most likely alone, certain
    tok, pr, tot = O.Sampler(0.0, 5, 0.5, 0.5, 1).candidates(x)
    assert list(tok) == [1] and list(pr) == [1.0] and tot == 1.0
    # top_p: the shortest prefix whose total reaches it; min_p: none below
    # min_p times the first
    lg = _logits(5000, 3, 1.0)
    full_t, full_p, _ = O.Sampler(1.0, 50, 1.0, 0.0, 1).candidates(lg)
    for top_p in (0.05, 0.3, 0.9):
        t, p, tot = O.Sampler(1.0, 50, top_p, 0.0, 1).candidates(lg)
        n = len(t)
        assert list(t) == list(full_t[:n])
        assert np.float32(full_p[:n - 1].sum()) < top_p <= tot + 1e-6 or n == 50
    for min_p in (0.2, 0.6):
        t, p, _ = O.Sampler(1.0, 50, 1.0, min_p, 1).candidates(lg)
        n = len(t)
        assert np.all(full_p[:n] >= min_p * full_p[0])
        assert n == 50 or full_p[n] < min_p * full_p[0]


def test_sample_frequencies_follow_the_kept_probabilities():
    lg = np.array([2.0, 1.5, 1.0, 0.5, 0.0, -5.0], np.float32)
    s = O.Sampler(1.0, 5, 1.0, 0.0, 7)
    tok, pr, tot = s.candidates(lg)
    n = 20_000
    picks = np.array([s.sample(lg) for _ in range(n)])
    assert 5 not in picks  # outside the top 5
    counts = np.array([(picks == t).sum() for t in tok])
    expected = pr / tot * n
    chi2 = ((counts - expected) ** 2 / expected).sum()
    assert chi2 < 18.5  # 4 degrees of freedom, 0.999 quantile


def test_verify_keeps_a_draft_as_often_as_sample_would_pick_it():
    lg = np.array([2.0, 1.5, 1.0, 0.5, 0.0], np.float32)
    # at temperature zero the most likely is certain: always kept, no draw
    s = O.Sampler(0.0, 5, 1.0, 0.0, 3)
    st = s.rng
    assert s.verify(lg, 0) == (0, True) and s.rng == st
    # a draft outside the kept tokens is never kept; its replacements are
    # distributed as the kept tokens are
    s = O.Sampler(1.0, 3, 1.0, 0.0, 5)
    tok, pr, tot = s.candidates(lg)
    n = 20_000
    outs = [s.verify(lg, 4) for _ in range(n)]
    assert not any(a for _, a in outs)
    picks = np.array([t for t, _ in outs])
    counts = np.array([(picks == t).sum() for t in tok])
    expected = pr / tot * n
    assert ((counts - expected) ** 2 / expected).sum() < 13.8  # 2 degrees, 0.999
    # a draft of probability p is kept at a rate p
    s = O.Sampler(1.0, 5, 1.0, 0.0, 11)
    tok, pr, tot = s.candidates(lg)
    p = pr[list(tok).index(1)] / tot
    outs = [s.verify(lg, 1) for _ in range(n)]
    rate = np.mean([a for _, a in outs])
    assert abs(rate - p) < 4 * np.sqrt(p * (1 - p) / n)
    # and when it is not kept, the other token is never the draft
    assert all(t != 1 for t, a in outs if not a)


# ---- the device ------------------------------------------------------------


@pytest.fixture(scope="module")
def gpu():
    from dwim_amd import device as D
    g = D.Hip(0)
    yield g
    g.close()


SETTINGS = [
    # temperature, top_k, top_p, min_p, seed
    (0.0, 20, 0.95, 0.05, 1),     # greedy
    (1.0, 20, 0.95, 0.05, 42),    # the reference's defaults (loaded.rs:112-118)
    (0.7, 1, 1.0, 0.0, 3),
    (1.0, 64, 1.0, 0.0, 5),       # the largest top k the rounds take
    (1.0, 65, 0.9, 0.0, 6),       # sorted rows from here on
    (1.5, 300, 1.0, 0.02, 7),
    (100.0, 2, 1.0, 0.0, 8),
]


@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [248_320, 1000, 4097])
@pytest.mark.parametrize("settings", SETTINGS)
def test_device_sampler_matches_the_oracle(gpu, vocab, settings):
    t, k, p, m, seed = settings
    dev = gpu.sampler(t, k, p, m, seed)
    ref = O.Sampler(t, k, p, m, seed)
    rows = 3
    lg = np.concatenate([_logits(vocab, 100 + r) for r in range(rows)])
    buf = gpu.buffer(lg)
    for step in range(12):
        r = step % rows
        row = lg[r * vocab:(r + 1) * vocab]
        want = ref.sample(row)
        got = dev.sample(buf, r, vocab)
        assert got == want, (settings, vocab, step)
    assert dev.rng == ref.rng


@pytest.mark.gpu
@pytest.mark.parametrize("settings", [SETTINGS[0], SETTINGS[1], SETTINGS[4], (1.0, 5, 1.0, 0.0, 9)])
def test_device_verify_matches_the_oracle(gpu, settings):
    t, k, p, m, seed = settings
    vocab = 248_320
    dev = gpu.sampler(t, k, p, m, seed)
    ref = O.Sampler(t, k, p, m, seed)
    lg = _logits(vocab, 7)
    buf = gpu.buffer(lg)
    order = np.argsort(-lg, kind="stable")
    # drafts: the most likely, the second, one in the tail, and again
    accepted = 0
    for d in [order[0], order[1], order[2], 12345, order[0], order[3], order[1], 7]:
        want = ref.verify(lg, int(d))
        got = dev.verify(buf, int(d))
        assert got == want, (settings, int(d))
        accepted += want[1]
    assert dev.rng == ref.rng


@pytest.mark.gpu
def test_device_sampler_breaks_ties_by_index(gpu):
    # few distinct logits (many ties), with -0 and 0 among them: the k kept
    # are the first indices of the largest values, as the reference inserts
    vocab = 248_320
    rng = np.random.default_rng(5)
    lg = np.round(rng.standard_normal(vocab) * 2.0).astype(np.float32)
    lg[rng.integers(0, vocab, 500)] = -0.0
    lg[lg.argmax()] = lg.max()
    buf = gpu.buffer(lg)
    for t, k, seed in [(0.0, 20, 1), (1.0, 40, 2), (1.0, 100, 3), (3.0, 64, 4)]:
        dev = gpu.sampler(t, k, 1.0, 0.0, seed)
        ref = O.Sampler(t, k, 1.0, 0.0, seed)
        for _ in range(6):
            assert dev.sample(buf) == ref.sample(lg)
        assert dev.rng == ref.rng


@pytest.mark.gpu
def test_device_sampler_refuses_settings_that_keep_nothing(gpu):
    from dwim_amd.device import DwimError
    for args in [(-1.0, 20, 0.9, 0.0, 1), (1.0, 20, 0.0, 0.0, 1), (1.0, 20, 0.9, 1.5, 1)]:
        with pytest.raises(DwimError):
            gpu.sampler(*args)
    s = gpu.sampler(1.0, 20, 0.9, 0.0, 1)
    with pytest.raises(DwimError):
        s.sample(gpu.buffer(np.zeros(100, np.float32)), 1, 100)  # no row 1
