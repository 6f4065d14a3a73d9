"""GPU tests of stochastic speculative decoding (speculative sampling on the
MTP drafter's K=3 drafts), eager and as captured graphs, on the reduced model.

* Every step's drafts are vmi_sample_top_p of that step's MTP logits, and
  every step's record is the oracle's speculative sampling replayed on that
  step's GPU logits, drafts and counters: bit for bit.
* With top-p small enough that every nucleus is the argmax alone, the stream
  equals greedy decoding token for token.
* Over 2,000 seeds from one committed state the first draft follows the MTP
  layer's distribution q and the first emitted token the target's
  temperature / top-p distribution p (chi-squared, bins of 5% mass, 0.999
  quantile), and the first draft is accepted at the rate sum_j min(p_j, q_j).
* The graph decoder emits what the eager loop emits with the same Sampling.
* A verify row without a finite logit ends the step with the failure record
  [0, 0, 0, -1]: the eager loop and the graph decoder raise VmiError.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from test_gpu_decode import SMALL, _fresh, _greedy_truth, _prompt  # noqa: E402


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def model(gpu):
    from vates_amd.workload import synth_spec_model
    return synth_spec_model(91, **SMALL, device=gpu)


def test_stochastic_records_match_oracle(gpu, orc, model):
    from vates_amd.decode import Sampling, speculative_decode
    K, temp, top_p, seed = 3, 0.7, 0.9, 2024
    prompt = _prompt(gpu, seed=12)
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    sp = Sampling(temp, top_p, seed)
    log("case: eager stochastic decode, 30 tokens traced")
    st = speculative_decode(model, drafter, caches, x, h, prompt.numel(), 30, K=K, trace=True, sampling=sp)
    assert len(st.samples) == st.steps >= 8
    hist = np.zeros(K + 1, int)
    for s, smp in enumerate(st.samples):
        base = smp["offset"]
        assert base == 64 * s
        for i in range(K):
            want = int(orc.sample_top_p(smp["draft"][i:i + 1], temp, top_p, seed, base + i)[0])
            assert smp["drafts"][i] == want, (s, i, smp["drafts"], want)
        em, m, acc, rec = orc.accept_stochastic(smp["target"], smp["draft"], np.array(smp["drafts"], np.int32),
                                                temp, top_p, seed, base + Sampling.ACCEPT_OFFSET)
        n = int(rec[0])
        assert list(smp["record"][:4 + n]) == [int(v) for v in rec[:4 + n]], (s, smp["record"], rec)
        hist[m] += 1
    log(f"matched histogram {hist.tolist()}")
    assert st.tokens == [t for smp in st.samples for t in smp["record"][4:4 + smp["record"][0]]][:30]


def test_tiny_top_p_equals_greedy(gpu, model):
    from vates_amd.decode import GraphSpecDecoder, Sampling, speculative_decode
    n_tok, K = 40, 3
    prompt = _prompt(gpu, seed=13)
    truth = _greedy_truth(gpu, model, prompt, n_tok + 2 * (K + 1))
    sp = Sampling(0.7, 1e-6, 5)
    log("case: top-p 1e-6 eager stochastic decode vs greedy")
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    st = speculative_decode(model, drafter, caches, x, h, prompt.numel(), n_tok, K=K, sampling=sp)
    assert st.tokens == truth[:n_tok], (st.tokens, truth[:n_tok])
    log("case: top-p 1e-6 graph stochastic decode vs greedy")
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    dec = GraphSpecDecoder(model, drafter, caches, K=K, sampling=sp)
    dec.start(x, h, prompt.numel())
    st2 = dec.run(n_tok)
    assert st2.tokens == truth[:n_tok]
    log(f"accept_hist {st.accept_hist}")


def test_graph_stochastic_equals_eager(gpu, model):
    from vates_amd.decode import GraphSpecDecoder, Sampling, speculative_decode
    n_tok, K = 40, 3
    prompt = _prompt(gpu, seed=14)
    sp = Sampling(0.7, 0.9, 77)
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    eager = speculative_decode(model, drafter, caches, x, h, prompt.numel(), n_tok, K=K, sampling=sp)
    for trace in (False, True):
        log(f"case: graph stochastic decode trace={trace} vs eager")
        caches, drafter, x, h = _fresh(gpu, model, prompt)
        dec = GraphSpecDecoder(model, drafter, caches, K=K, sampling=sp)
        dec.start(x, h, prompt.numel())
        st = dec.run(n_tok, trace=trace)
        assert st.tokens == eager.tokens and st.accept_hist == eager.accept_hist, (st.tokens, eager.tokens)
        P = prompt.numel()
        assert all(c.length == P + sum(m + 1 for m in st.accept_hist) for c in caches if c is not None)
    log(f"accept_hist {eager.accept_hist}")


def _chi2_bins(tokens, p, bin_mass=0.05):
    """Chi-squared statistic of token counts against distribution p over
    bins of about `bin_mass` target mass (tokens by descending p), the
    degrees of freedom, and the count outside p's support."""
    c = np.bincount(np.asarray(tokens), minlength=p.size).astype(np.float64)
    order = np.argsort(-p)
    bins, cp, cc = [], 0.0, 0.0
    for t in order[p[order] > 0]:
        cp += p[t]
        cc += c[t]
        if cp >= bin_mass:
            bins.append((cp, cc))
            cp, cc = 0.0, 0.0
    if cp > 0:
        bins[-1] = (bins[-1][0] + cp, bins[-1][1] + cc)
    exp = np.array([b[0] for b in bins]) * len(tokens)
    obs = np.array([b[1] for b in bins])
    return float(((obs - exp) ** 2 / exp).sum()), len(bins) - 1, float(c[p == 0].sum())


def test_first_token_follows_target_distribution(gpu, orc, model):
    """2,000 seeds from one committed state: the first draft follows the
    MTP layer's q, the first emitted token the target's p (chi-squared at the
    0.999 quantile, bins of 5% mass), nothing outside either nucleus, and the
    first draft's acceptance rate is sum_j min(p_j, q_j) within 4 standard
    errors."""
    from scipy.stats import chi2
    from vates_amd.decode import Sampling, speculative_decode
    K, temp, top_p, n = 3, 0.7, 0.9, 2000
    prompt = _prompt(gpu, seed=15)
    first, d1, acc = [], [], []
    p0 = q0 = t0 = None
    log(f"case: first emitted token over {n} seeds")
    for s in range(n):
        caches, drafter, x, h = _fresh(gpu, model, prompt)
        st = speculative_decode(model, drafter, caches, x, h, prompt.numel(), 1, K=K, trace=True,
                                sampling=Sampling(temp, top_p, 5000 + s))
        smp = st.samples[0]
        if s == 0:
            t0 = smp["target"][0].copy()
            W, th, zs, _ = orc.sd_masses(t0, temp, top_p)
            p0 = np.where((W >= th) & (W > 0), W, 0).astype(np.float64) / zs
            W, th, zs, _ = orc.sd_masses(smp["draft"][0], temp, top_p)
            q0 = np.where((W >= th) & (W > 0), W, 0).astype(np.float64) / zs
        elif s % 97 == 0:  # row 0 of the verify batch does not depend on the drafts after it
            assert np.array_equal(smp["target"][0], t0)
        first.append(st.tokens[0])
        d1.append(smp["drafts"][0])
        acc.append(smp["record"][1] > 0)
    for name, toks, dist in (("first draft vs q", d1, q0), ("first token vs p", first, p0)):
        stat, dof, outside = _chi2_bins(toks, dist)
        log(f"{name}: chi2 {stat:.2f} on {dof} dof (0.999 quantile {chi2.ppf(0.999, dof):.2f}), outside {outside}")
        assert outside == 0 and stat < chi2.ppf(0.999, dof), (name, stat, dof)
    rate, theory = float(np.mean(acc)), float(np.minimum(p0, q0).sum())
    log(f"first-draft acceptance {rate:.4f}, theory {theory:.4f}")
    assert abs(rate - theory) <= 4 * np.sqrt(theory * (1 - theory) / n)


def test_failed_acceptance_raises(gpu, model):
    import torch
    from vates_amd._lib import VmiError
    from vates_amd.decode import GraphSpecDecoder, Sampling, SpecModel, speculative_decode
    K = 3
    bad = SpecModel(model.embed, model.layers, model.final_norm, torch.full_like(model.head, float("nan")),
                    model.mtp, model.eps)
    prompt = _prompt(gpu, seed=16)
    sp = Sampling(0.7, 0.9, 1)
    log("case: NaN verify logits, eager stochastic step")
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    with pytest.raises(VmiError, match="finite"):
        speculative_decode(bad, drafter, caches, x, h, prompt.numel(), 4, K=K, sampling=sp)
    log("case: NaN verify logits, graph stochastic step")
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    dec = GraphSpecDecoder(bad, drafter, caches, K=K, sampling=sp)
    dec.start(x, h, prompt.numel())
    with pytest.raises(VmiError, match="finite"):
        dec.run(4)
    torch.cuda.synchronize()
