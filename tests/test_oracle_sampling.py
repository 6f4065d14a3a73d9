"""Pins the oracle's stochastic acceptance and top-p sampler (CPU only).

Pinned by what the mathematics fixes, not by restating the code:
  * masses: W / Z equals softmax(l / temperature) (scipy) to 1e-6 relative;
  * nucleus: the set is top-heavy, holds at least ceil(top_p Z) mass, and is
    minimal (dropping its smallest tie group falls below the cutoff);
  * speculative sampling: the emitted first token is distributed as the target
    p whatever the draft q (Leviathan et al. 2023, Theorem 1) - chi-square over
    Monte-Carlo draws; q = p accepts every draft; a draft outside the target's
    nucleus is always rejected and never re-emitted.
"""
import numpy as np
import pytest
from scipy.special import softmax
from scipy.stats import chi2


def test_masses_match_softmax(orc):
    rng = np.random.default_rng(5)
    for temp in (1.0, 0.7, 2.0):
        l = rng.normal(0, 3, 4096).astype(np.float32)
        W, th, zs, z = orc.sd_masses(l, temp, 1.0)
        assert th <= W[W > 0].min() and zs == z == int(W.astype(np.uint64).sum())
        ref = softmax(l.astype(np.float64) / temp)
        got = W.astype(np.float64) / z
        big = W >= 1024
        assert np.all(np.abs(got[big] - ref[big]) <= 1e-6 * ref[big] + 2.0 / z)
        assert W.max() == 2 ** 31 and W[np.argmax(l)] == 2 ** 31


def test_nucleus_is_top_heavy_sufficient_and_minimal(orc):
    rng = np.random.default_rng(6)
    for trial in range(40):
        V = int(rng.integers(2, 3000))
        l = rng.normal(0, 3, V).astype(np.float32)
        if trial % 4 == 0:
            l = np.round(l)  # many exact ties
        top_p = float(rng.uniform(0.05, 0.999))
        W, th, zs, z = orc.sd_masses(l, 0.7, top_p)
        C = int(np.ceil(np.float64(top_p) * np.float64(z)))
        inS = (W >= th) & (W > 0)
        assert zs == int(W[inS].astype(np.uint64).sum())
        assert zs >= C
        if (~inS).any():
            assert W[inS].min() >= W[~inS].max()
        smallest = W[inS].min()
        assert zs - int(W[W == smallest].astype(np.uint64).sum()) < C


def test_nucleus_ties_and_flat(orc):
    l = np.zeros(10, np.float32)
    W, th, zs, z = orc.sd_masses(l, 1.0, 0.5)
    assert th == 2 ** 31 and zs == z == 10 * 2 ** 31  # all ties join at once
    l = np.array([5, 5, 0, -50], np.float32)
    W, th, zs, z = orc.sd_masses(l, 1.0, 0.3)
    assert zs == 2 * 2 ** 31 and W[3] == 0
    with pytest.raises(RuntimeError):
        orc.sd_masses(np.full(4, np.nan, np.float32), 1.0, 0.9)


def _target_probs(orc, row, temp, top_p):
    W, th, zs, _ = orc.sd_masses(row, temp, top_p)
    return np.where((W >= th) & (W > 0), W, 0).astype(np.float64) / zs


@pytest.mark.parametrize("with_draft", [True, False])
def test_speculative_output_is_target_distribution(orc, with_draft):
    rng = np.random.default_rng(7 if with_draft else 8)
    V, K, temp, top_p = 8, 2, 0.7, 0.9
    target = rng.normal(0, 1.5, (K + 1, V)).astype(np.float32)
    draft = rng.normal(0, 1.5, (K, V)).astype(np.float32)
    p0 = _target_probs(orc, target[0], temp, top_p)
    n = 40000
    counts = np.zeros(V)
    accepted = 0
    for s in range(n):
        if with_draft:
            drafts = orc.sample_top_p(draft, temp, top_p, seed=99, offset=s)
        else:
            drafts = np.array([int(rng.integers(0, V)), 0], np.int32)  # any fixed-rule (one-hot) draft
        em, m, acc_len, _ = orc.accept_stochastic(target, draft if with_draft else None, drafts, temp, top_p,
                                                  seed=1234, offset=s)
        assert acc_len == m + 1 and len(em) == m + 1 and em[:m] == list(drafts[:m])
        counts[em[0]] += 1
        accepted += m > 0
    support = p0 > 0
    assert counts[~support].sum() == 0
    exp = n * p0[support]
    stat = ((counts[support] - exp) ** 2 / exp).sum()
    assert stat < chi2.ppf(0.999, support.sum() - 1), (stat, counts, exp)
    assert 0 < accepted < n


def test_identical_draft_accepts_everything(orc):
    rng = np.random.default_rng(9)
    V, K = 64, 3
    target = rng.normal(0, 3, (K + 1, V)).astype(np.float32)
    for s in range(50):
        drafts = orc.sample_top_p(target[:K], 0.7, 0.9, seed=5, offset=s)
        em, m, _, _ = orc.accept_stochastic(target, target[:K], drafts, 0.7, 0.9, seed=6, offset=s)
        assert m == K and em[:K] == list(drafts)


def test_draft_outside_nucleus_is_rejected(orc):
    V, K = 16, 3
    target = np.zeros((K + 1, V), np.float32)
    target[:, 3] = 40.0  # nucleus = {3} at top_p 0.9
    drafts = np.array([3, 7, 3], np.int32)
    for s in range(20):
        em, m, _, _ = orc.accept_stochastic(target, None, drafts, 0.7, 0.9, seed=11, offset=s)
        assert m == 1 and em == [3, 3]


def test_sampler_matches_distribution(orc):
    rng = np.random.default_rng(10)
    V = 12
    row = rng.normal(0, 1, (1, V)).astype(np.float32)
    p = _target_probs(orc, row[0], 1.3, 0.95)
    n = 30000
    counts = np.bincount([orc.sample_top_p(row, 1.3, 0.95, seed=3, offset=s)[0] for s in range(n)], minlength=V)
    sup = p > 0
    assert counts[~sup].sum() == 0
    exp = n * p[sup]
    assert ((counts[sup] - exp) ** 2 / exp).sum() < chi2.ppf(0.999, sup.sum() - 1)
