"""The host sampler (uaii_sample_token) against the reference's own
sample_token_f32 (libs/uaii-runtime/src/sampling.cpp:22-125, compiled into
oracle/_ref): temperature, top-k, top-p, repetition penalty and a seeded
mt19937_64 must pick the same id from the same row. CPU only."""
import numpy as np
import pytest

import oracle
import uaii_amd

PARAMS = [
    # temperature, top_p, top_k, repetition penalty
    (0.0, 1.0, 0, 1.0),     # greedy
    (0.0, 1.0, 0, 1.3),     # greedy order but not greedy(): penalty path
    (0.7, 1.0, 0, 1.0),     # temperature only
    (1.0, 1.0, 40, 1.0),    # top-k (the nth_element arrangement decides the pick)
    (0.8, 0.9, 0, 1.0),     # nucleus
    (0.9, 0.95, 50, 1.2),   # everything
    (1.5, 0.5, 5, 1.0),
]


def rows(vocab, n, seed):
    """Logits rows (what the session samples from, session.cpp:974-978) of two
    spreads, plus a probability row, which the sampler must treat like any other
    row of scores."""
    rng = np.random.default_rng(seed)
    for i in range(n):
        if i % 3 == 2:
            x = rng.normal(0, 3, vocab).astype(np.float32)
            e = np.exp(x - x.max())
            yield (e / e.sum()).astype(np.float32)
        else:
            yield rng.normal(0, 2 + 4 * (i % 3), vocab).astype(np.float32)


@pytest.mark.parametrize("vocab", [50, 3000, 32000])
@pytest.mark.parametrize("prm", PARAMS, ids=lambda p: f"T{p[0]}_p{p[1]}_k{p[2]}_r{p[3]}")
def test_sampler_matches_reference(vocab, prm):
    if oracle.ref() is None:
        pytest.skip("reference kernels not built (make -C oracle ref needs /root/reference)")
    t, tp, tk, rp = prm
    for i, row in enumerate(rows(vocab, 6, vocab)):
        pen = list(range(0, vocab, 7))[:20]
        for seed in (1, 12345, 2 ** 63 + 5):
            p = uaii_amd.sample_params(t, tp, tk, rp, seed=seed)
            got = uaii_amd.sample_token(row, p, pen)
            want = oracle.ref_sample_token(row, t, tp, tk, rp, seed, pen)
            assert got == want, (i, seed)


def test_sampler_distribution_follows_softmax_of_logits():
    """The sampler softmaxes the row it is given (sampling.cpp:80-92), and the
    session gives it the logits: at temperature T with no truncation the draw
    frequencies over many seeds follow softmax(logits / T). Sampling a row that
    had already been softmaxed would flatten them (here to about 0.39/0.33/0.28
    at T = 1), which this bar rejects."""
    logits = np.array([2.0, 0.0, -1.0], np.float32)
    for T in (1.0, 0.5):
        z = logits.astype(np.float64) / T
        want = np.exp(z - z.max()) / np.exp(z - z.max()).sum()
        counts = np.zeros(3)
        n = 4000
        for seed in range(n):
            counts[uaii_amd.sample_token(logits, uaii_amd.sample_params(T, 1.0, 0, 1.0, seed=seed))] += 1
        freq = counts / n
        # 5 standard deviations of a binomial frequency
        assert np.all(np.abs(freq - want) < 5 * np.sqrt(want * (1 - want) / n) + 1e-3), (T, freq, want)
    flat = np.exp(logits - logits.max()) / np.exp(logits - logits.max()).sum()
    resoft = np.exp(flat) / np.exp(flat).sum()
    assert abs(resoft[0] - 0.84) > 0.3  # the probs-reading mistake is far outside the bar


def test_uniforms_are_the_reference_draws():
    """uaii_sample_uniforms(seed, n) gives the r the reference's sampler draws
    (sampling.cpp:111-112) from mt19937_64(seed): over a flat-ish row walked in
    index order (no top-k / top-p) the reference picks the first id whose
    cumulative probability reaches r, which fixes r to within one id's mass."""
    if oracle.ref() is None:
        pytest.skip("reference kernels not built (make -C oracle ref needs /root/reference)")
    V = 1000
    row = np.random.default_rng(3).normal(0, 0.5, V).astype(np.float32)
    e = np.exp(row.astype(np.float64) - row.max())
    cum = np.cumsum(e / e.sum())
    checked = 0
    for seed in range(150):
        r = float(uaii_amd.sample_uniforms(seed, 1)[0])
        want = oracle.ref_sample_token(row, 1.0, 1.0, 0, 1.0, seed, [])
        if np.abs(cum - r).min() < 1e-6:
            continue  # within float rounding of a boundary
        assert want == int(np.searchsorted(cum, r)), (seed, r)
        checked += 1
    assert checked >= 140
    # a sequence is the generator's successive draws: the first of n equals n = 1
    seq = uaii_amd.sample_uniforms(77, 5)
    assert seq[0] == uaii_amd.sample_uniforms(77, 1)[0] and len(set(seq.tolist())) == 5
    assert np.all((seq >= 0) & (seq < 1))
