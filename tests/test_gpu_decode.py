"""GPU tests of the MTP draft step and the speculative decode loop.

* One MTP step (embedding norm, hidden norm, fc, attention block, MoE block,
  final norm, head argmax) against the CPU oracle's composition of the pinned
  pieces: hidden state relative L2 <= 2e-2 and cosine >= 0.999 (bf16
  activations through five blocks), draft token equal wherever the oracle's
  top-two logit margin exceeds 1e-2 of the logit scale.
* Speculative decoding with K=3 emits exactly the tokens of non-speculative
  greedy decoding (the reference's lossless invariant,
  tests/test_mtp_generate.py:421-489), in both verify layouts ([x, d1..dK],
  and the reference's [x, d1..d_{K-1}], generate.py:604), eagerly and as
  captured graphs, with scripted drafts that make every acceptance length
  0..K occur, and with the MTP layer's own drafts; the graph decoder drafts
  exactly what the eager drafter drafts from the same committed state.
* Adaptive depth (draft_adaptive, drafter.py:42-62): the depth of every step
  equals the tau rule replayed in float64 on the MTP logits of that step
  (away from the threshold), the stream equals greedy decoding, and the
  graph decoder reproduces the eager one step for step.
* draft_paths takes its first tokens from the top-P of the MTP logits.
* Tree verification: one forward over the P x K tokens of the paths equals
  each path's chain forward bit for bit; committing the winner leaves every
  cache as a chain forward of its accepted prefix would; tree decoding emits
  the greedy stream.
* The minimal tree (draft_tree, drafter.py:102-148) and the adaptive tree
  (draft_adaptive_tree, drafter.py:64-100): the branches fork from the MTP
  state where the reference forks them (checked against draft, draft_paths,
  draft_adaptive and the MTP logits from the same state); decoding with them
  emits the greedy stream, and planted trees make the position-0 and
  position-1 rescues win (generate.py:764-801).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


from oracle.torch_bridge import layer_np, u16, u32  # noqa: E402

SMALL = dict(n_layers=4, attn_every=2, hidden=512, inter=128, num_experts=64, top_k=4, vocab=4096, n_heads=4,
             n_kv_heads=2, n_k_heads=2, n_v_heads=4)


@pytest.fixture(scope="module")
def model(gpu):
    from vates_amd.workload import synth_spec_model
    return synth_spec_model(91, **SMALL, device=gpu)


def _prompt(gpu, n=8, seed=5):
    import torch
    rng = np.random.default_rng(seed)
    return torch.tensor(rng.integers(0, SMALL["vocab"], n), dtype=torch.int32, device=gpu)


def test_mtp_step_matches_oracle(gpu, orc, model):
    log("case: two chained MTP steps vs the oracle composition (reduced shape)")
    from model_oracle import check_mtp_steps
    check_mtp_steps(gpu, model, SMALL["hidden"], log)


class ScriptedDrafter:
    """Runs the MTP drafter (kernels and cache writes) and replaces its drafts by
    the true continuation for the first m tokens of each step and a wrong token
    after, cycling m through 0..K."""

    def __init__(self, inner, truth, prompt_len):
        self.inner, self.truth, self.P, self.n = inner, truth, prompt_len, 0
        self.cache, self.mtp = inner.cache, inner.mtp

    def _plant(self, d, start):
        import torch
        K = d.numel()
        base = start + 1 - self.P  # index of the next token in the greedy stream
        m = self.n % (K + 1)
        self.n += 1
        planted = [self.truth[base + i] if i < m else (self.truth[base + i] + 1) % SMALL["vocab"] for i in range(K)]
        d.copy_(torch.tensor(planted, dtype=torch.int32, device=d.device))
        return d

    def draft(self, H_last, x, K):
        start = self.cache.length
        return self._plant(self.inner.draft(H_last, x, K), start)

    def draft_adaptive(self, H_last, x, depth_max, tau):
        start = self.cache.length
        return self._plant(self.inner.draft_adaptive(H_last, x, depth_max, tau), start)

    def sync(self, start, h_seq, tokens):
        self.inner.sync(start, h_seq, tokens)


def _greedy_truth(gpu, model, prompt, n):
    from vates_amd.decode import greedy_decode, prefill
    caches = model.new_caches(256)
    x, h = prefill(model, prompt, caches)
    return greedy_decode(model, caches, x, prompt.numel(), n).tokens


def _fresh(gpu, model, prompt):
    from vates_amd.decode import prefill
    from vates_amd.mtp import MTPDrafter
    caches = model.new_caches(256)
    drafter = MTPDrafter(model.mtp, 256)
    x, h = prefill(model, prompt, caches, drafter)
    return caches, drafter, x, h


@pytest.mark.parametrize("layout", ["k+1", "k"])
def test_speculative_equals_greedy(gpu, model, layout):
    from vates_amd.decode import speculative_decode
    n_tok, K = 40, 3
    prompt = _prompt(gpu)
    truth = _greedy_truth(gpu, model, prompt, n_tok + K + 1)
    log(f"case: greedy stream {truth[:12]}...")
    for scripted in (True, False):
        log(f"case: speculative K=3 layout={layout} scripted={scripted}")
        caches, drafter, x, h = _fresh(gpu, model, prompt)
        d = ScriptedDrafter(drafter, truth, prompt.numel()) if scripted else drafter
        st = speculative_decode(model, d, caches, x, h, prompt.numel(), n_tok, K=K, layout=layout)
        assert st.tokens == truth[:n_tok], (st.tokens, truth[:n_tok])
        if scripted:
            assert set(st.accept_hist) == set(range(K + 1)), st.accept_hist
        log(f"accept_hist {st.accept_hist} steps {st.steps}")


def _adaptive_oracle_depth(probs, depth_max, tau):
    """draft_adaptive's rule (drafter.py:42-62) on float64 probabilities:
    (depth, whether some decision lay within 1e-4 of tau)."""
    conf, near = 1.0, False
    for i, p in enumerate(probs):
        if i + 1 >= depth_max:
            return depth_max, near
        conf *= p
        near |= abs(conf - tau) <= 1e-4 * max(tau, 1e-30)
        if conf < tau:
            return i + 1, near
    return len(probs), near


def _sample_probs(gpu, model, prompt, steps=12, K=3):
    """Draft probabilities of the first `steps` steps of a depth-K decode."""
    import torch
    from vates_amd.decode import speculative_decode
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    seen = []
    orig = drafter.draft_adaptive

    def rec(H_last, x_tok, depth_max, tau):
        lg = []
        d = orig(H_last, x_tok, depth_max, tau, logits_out=lg)
        for l in lg:
            v = l[0].double().cpu().numpy()
            seen.append(1.0 / np.exp(v - v.max()).sum())
        return d
    drafter.draft_adaptive = rec
    speculative_decode(model, drafter, caches, x, h, prompt.numel(), steps, K=K, layout="k", tau=0.0)
    torch.cuda.synchronize()
    return np.array(seen).reshape(-1, K)


def test_adaptive_depth_matches_tau_rule(gpu, model):
    """Eager adaptive decoding: depth per step from the fp32 probabilities the
    head fuses equals the tau rule on float64 softmax of the step's logits;
    tau = 0 always drafts K, tau > 1 always 1, a middle tau mixes depths;
    the stream equals greedy decoding in every case."""
    import torch
    from vates_amd.decode import speculative_decode
    n_tok, K = 40, 3
    prompt = _prompt(gpu, seed=12)
    truth = _greedy_truth(gpu, model, prompt, n_tok + K + 1)
    P = _sample_probs(gpu, model, prompt)
    # thresholds inside the spread of the first and of the two-draft confidence
    mids = (float(np.median(P[:, 0])), float(np.median(P[:, 0] * P[:, 1])))
    log(f"draft probabilities (first steps) {np.round(P[:4], 6).tolist()}, middle taus {mids}")
    seen = set()
    for tau in (0.0, 1.1) + mids:
        log(f"case: adaptive depth tau={tau:.3g}")
        caches, drafter, x, h = _fresh(gpu, model, prompt)
        orig = drafter.draft_adaptive
        oracle = []

        def rec(H_last, x_tok, depth_max, tau_):
            lg = []
            d = orig(H_last, x_tok, depth_max, tau_, logits_out=lg)
            probs = []
            for l in lg:
                v = l[0].double().cpu().numpy()
                probs.append(1.0 / np.exp(v - v.max()).sum())
            oracle.append(_adaptive_oracle_depth(probs, depth_max, tau_) + (d.numel(),))
            return d
        drafter.draft_adaptive = rec
        st = speculative_decode(model, drafter, caches, x, h, prompt.numel(), n_tok, K=K, layout="k", tau=tau)
        torch.cuda.synchronize()
        assert st.tokens == truth[:n_tok], (st.tokens, truth[:n_tok])
        for want, near, got in oracle:
            assert near or want == got, oracle
        assert st.depths == [o[2] for o in oracle]
        if tau == 0.0:
            assert set(st.depths) == {K}
        elif tau > 1.0:
            assert set(st.depths) == {1}
        seen |= set(st.depths)
        log(f"depths {st.depths}")
    assert seen == {1, 2, 3}


def test_draft_paths_top_p(gpu, model):
    log("case: draft_paths P=3 K=3")
    import torch
    from vates_amd.decode import prefill
    from vates_amd.mtp import MTPDrafter
    prompt = _prompt(gpu, seed=6)
    caches = model.new_caches(128)
    drafter = MTPDrafter(model.mtp, 128)
    x, h = prefill(model, prompt, caches, drafter)
    base = drafter.cache.length
    paths = drafter.draft_paths(h, x, 3, 3)
    drafter.cache.length = base
    _, _, logits = model.mtp.step(h, x, drafter.cache, want_logits=True)
    torch.cuda.synchronize()
    lg = logits[0].cpu().numpy()
    order = np.lexsort((np.arange(lg.size), -lg))[:3]
    assert paths[:, 0].cpu().tolist() == order.tolist()


@pytest.mark.parametrize("layout", ["k+1", "k"])
def test_graph_decode_equals_greedy(gpu, model, layout):
    """The captured-graph step (positions on the device) emits the greedy stream,
    with the MTP layer's drafts (identical to the eager drafter's from the same
    state, step for step) and with planted drafts that make every acceptance
    length 0..K occur."""
    from vates_amd.decode import GraphSpecDecoder, speculative_decode
    n_tok, K = 40, 3
    prompt = _prompt(gpu, seed=8)
    truth = _greedy_truth(gpu, model, prompt, n_tok + 2 * (K + 1))
    P = prompt.numel()
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    eager = speculative_decode(model, drafter, caches, x, h, P, n_tok, K=K, layout=layout, trace=True)
    for planted in (False, True):
        log(f"case: graph speculative K=3 layout={layout} planted={planted}")
        caches, drafter, x, h = _fresh(gpu, model, prompt)
        dec = GraphSpecDecoder(model, drafter, caches, K=K, planted=planted, layout=layout)
        dec.start(x, h, P)

        def plant(step, pos):
            m = step % (K + 1)
            base = pos - P  # greedy stream index of the token at position pos + 1
            return [truth[base + i] if i < m else (truth[base + i] + 1) % SMALL["vocab"] for i in range(K)]

        st = dec.run(n_tok, plant=plant if planted else None, trace=not planted)
        assert st.tokens == truth[:n_tok], (st.tokens, truth[:n_tok])
        if planted:
            assert set(st.accept_hist) == set(range(K + 1)), st.accept_hist
        else:  # the device-side handoff (H, x, MTP positions) drafts what the eager drafter does
            assert st.drafts == eager.drafts and st.accept_hist == eager.accept_hist
        log(f"accept_hist {st.accept_hist} steps {st.steps}")
        # the host view of the caches follows the device positions
        acc = [m + 1 if layout == "k+1" else min(m + 1, K) for m in st.accept_hist]
        assert all(c.length == P + sum(acc) for c in caches if c is not None)


def test_graph_adaptive_equals_eager(gpu, model):
    """Adaptive depth as graphs (one per draft step, one verify per depth)
    reproduces the eager adaptive decoder: tokens, depths, drafts."""
    from vates_amd.decode import GraphSpecDecoder, speculative_decode
    n_tok, K = 40, 3
    prompt = _prompt(gpu, seed=12)
    Pr = _sample_probs(gpu, model, prompt)
    tau = float(np.median(Pr[:, 0]))
    truth = _greedy_truth(gpu, model, prompt, n_tok + 2 * (K + 1))
    P = prompt.numel()
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    eager = speculative_decode(model, drafter, caches, x, h, P, n_tok, K=K, layout="k", tau=tau, trace=True)
    log(f"case: graph adaptive tau={tau:.3g}, eager depths {eager.depths}")
    caches, drafter, x, h = _fresh(gpu, model, prompt)
    dec = GraphSpecDecoder(model, drafter, caches, K=K, layout="k", tau=tau)
    dec.start(x, h, P)
    st = dec.run(n_tok, trace=True)
    assert st.tokens == truth[:n_tok]
    assert st.depths == eager.depths and st.drafts == eager.drafts and st.accept_hist == eager.accept_hist
    assert len(set(st.depths)) >= 2, st.depths


def test_tree_forward_equals_chains_and_commit(gpu, model):
    """forward_tree (one forward over P x K tokens) equals each path's chain
    forward bit for bit; TreeCommit leaves the caches exactly as a chain
    forward of the winner's accepted prefix would."""
    from model_oracle import check_tree_forward
    log("case: tree forward P=3 K=3 vs chains, commit vs the winner's chain")
    check_tree_forward(gpu, model, _prompt(gpu, seed=13), 3, 3, log)
    log("case: tree forward P=4 K=4 (16 tokens) vs chains")
    check_tree_forward(gpu, model, _prompt(gpu, seed=14), 4, 4, log, seed=1)


def test_tree_decode_equals_greedy(gpu, model):
    """Tree verification with P=3 paths of K=3 (the T = K layout) emits the
    greedy stream: with the MTP layer's paths, and with planted paths where a
    rotating path carries the true continuation for 0..K tokens and the others
    fewer (or tie), exercising the winner choice and every acceptance length."""
    from vates_amd.decode import greedy_decode, prefill, tree_speculative_decode
    from vates_amd.mtp import MTPDrafter
    n_tok, K, P = 30, 3, 3
    prompt = _prompt(gpu, seed=9)
    Pn = prompt.numel()
    caches = model.new_caches(256)
    x, h = prefill(model, prompt, caches)
    ref = greedy_decode(model, caches, x, Pn, n_tok + 2 * (K + 1))
    V = SMALL["vocab"]

    def plant(step, pos):
        base = pos - Pn  # greedy stream index of the token after position pos
        m = step % (K + 1)
        win = step % P
        rows = []
        for p in range(P):
            mp = m if p == win else (m - 1 if (p + step) % 2 else min(m, 1)) if m > 0 else 0
            mp = max(0, min(mp, m))
            rows.append([ref.tokens[base + i] if i < mp else (ref.tokens[base + i] + 1 + p) % V for i in range(K)])
        return rows

    for planted in (False, True):
        log(f"case: tree speculative K=3 P=3 planted={planted}")
        caches = model.new_caches(256)
        drafter = MTPDrafter(model.mtp, 256)
        x, h = prefill(model, prompt, caches, drafter)
        st = tree_speculative_decode(model, drafter, caches, x, h, Pn, n_tok, K=K, P=P,
                                     plant=plant if planted else None)
        assert st.tokens == ref.tokens[:n_tok], (st.tokens, ref.tokens[:n_tok])
        if planted:
            assert set(st.accept_hist) == set(range(K + 1)), st.accept_hist
        log(f"accept_hist {st.accept_hist}")


def _same_state(drafter, base):
    drafter.cache.length = base


def test_draft_tree_branches(gpu, model):
    """draft_tree's rows: A = the greedy chain (draft), B = the second-best
    first token continued greedily (draft_paths' second path), C = A's first
    token, then the second-best second token continued greedily."""
    log("case: draft_tree K=3 pos1")
    import torch
    from vates_amd.decode import prefill
    from vates_amd.mtp import MTPDrafter
    K = 3
    prompt = _prompt(gpu, seed=15)
    caches = model.new_caches(128)
    drafter = MTPDrafter(model.mtp, 128)
    x, h = prefill(model, prompt, caches, drafter)
    base = drafter.cache.length
    tree = drafter.draft_tree(h, x, K, pos1=True).cpu().numpy()
    _same_state(drafter, base)
    chain = drafter.draft(h, x, K).cpu().numpy()
    _same_state(drafter, base)
    two = drafter.draft_paths(h, x, K, 2).cpu().numpy()
    _same_state(drafter, base)
    _, h1, _ = model.mtp.step(h, x, drafter.cache)
    a0 = torch.tensor([int(tree[0, 0])], dtype=torch.int32, device=gpu)
    _, h2, lg2 = model.mtp.step(h1, a0, drafter.cache, want_logits=True)
    lg = lg2[0].cpu().numpy()
    second = int(np.lexsort((np.arange(lg.size), -lg))[1])
    cont = [int(tree[0, 0]), second]
    hh, tok = h2, torch.tensor([second], dtype=torch.int32, device=gpu)
    for _ in range(K - 2):
        am, hh, _ = model.mtp.step(hh, tok, drafter.cache)
        cont.append(int(am.cpu()[0]))
        tok = am
    torch.cuda.synchronize()
    assert tree.shape == (3, K)
    assert tree[0].tolist() == chain.tolist()
    assert tree[1].tolist() == two[1].tolist()
    assert tree[2].tolist() == cont
    log(f"tree {tree.tolist()}")
    _same_state(drafter, base)
    t2 = drafter.draft_tree(h, x, K, pos1=False).cpu().numpy()
    assert t2.shape == (2, K) and t2[0].tolist() == chain.tolist() and t2[1].tolist() == two[1].tolist()


def test_draft_adaptive_tree_branches(gpu, model):
    """draft_adaptive_tree: chain A equals draft_adaptive from the same state
    (tau at each end of the range and in between); chain B (when A is at least
    two long) is the second-best first token continued greedily to A's
    length."""
    from vates_amd.decode import prefill
    from vates_amd.mtp import MTPDrafter
    K = 3
    prompt = _prompt(gpu, seed=16)
    Pr = _sample_probs(gpu, model, prompt)
    caches = model.new_caches(128)
    drafter = MTPDrafter(model.mtp, 128)
    x, h = prefill(model, prompt, caches, drafter)
    base = drafter.cache.length
    seen = set()
    for tau in (0.0, float(np.median(Pr[:, 0])), float(Pr[:, 0].max()) * 0.999, 1.5):
        log(f"case: draft_adaptive_tree K=3 tau={tau:.3g}")
        _same_state(drafter, base)
        a, b = drafter.draft_adaptive_tree(h, x, K, tau)
        _same_state(drafter, base)
        ref = drafter.draft_adaptive(h, x, K, tau)
        n = a.numel()
        assert a.cpu().tolist() == ref.cpu().tolist()
        if n >= 2:
            _same_state(drafter, base)
            two = drafter.draft_paths(h, x, n, 2)
            assert b is not None and b.cpu().tolist() == two[1].cpu().tolist()
        else:
            assert b is None
        seen.add(n)
    assert 1 in seen and K in seen, seen


def test_tree_modes_equal_greedy(gpu, model):
    """Decoding with the minimal tree (with and without the position-1 branch)
    and with the adaptive tree emits the greedy stream; planted minimal trees
    make A, B (position-0 rescue) and C (position-1 rescue) win in turn."""
    from vates_amd.decode import greedy_decode, prefill, tree_speculative_decode
    from vates_amd.mtp import MTPDrafter
    n_tok, K = 30, 3
    prompt = _prompt(gpu, seed=17)
    Pn = prompt.numel()
    V = SMALL["vocab"]
    Pr = _sample_probs(gpu, model, prompt)
    caches = model.new_caches(256)
    x, h = prefill(model, prompt, caches)
    ref = greedy_decode(model, caches, x, Pn, n_tok + 2 * (K + 1))

    def plant(step, pos):
        base = pos - Pn
        t = [ref.tokens[base + i] for i in range(K)]
        bad = lambda v, d: (v + d) % V
        case = step % 4
        if case == 0:    # A matches two, B and C do not reach past it
            return [[t[0], t[1], bad(t[2], 1)], [bad(t[0], 2), t[1], t[2]], [t[0], bad(t[1], 3), t[2]]]
        if case == 1:    # A rejects at position 0, B's first token is the model's
            return [[bad(t[0], 1), t[1], t[2]], [t[0], t[1], bad(t[2], 2)], [bad(t[0], 1), t[1], t[2]]]
        if case == 2:    # A rejects at position 1, C's second token is the model's
            return [[t[0], bad(t[1], 1), t[2]], [bad(t[0], 2), t[1], t[2]], [t[0], t[1], t[2]]]
        # every path rejects at position 0: the lowest index, A, stands
        return [[bad(t[0], 1), t[1], t[2]], [bad(t[0], 2), t[1], t[2]], [bad(t[0], 1), bad(t[1], 3), t[2]]]

    runs = [("tree", dict(pos1=True), None), ("tree", dict(pos1=False), None), ("tree", dict(pos1=True), plant),
            ("adaptive_tree", dict(tau=float(np.median(Pr[:, 0]))), None)]
    for mode, kw, pl in runs:
        log(f"case: tree decode mode={mode} {kw} planted={pl is not None}")
        caches = model.new_caches(256)
        drafter = MTPDrafter(model.mtp, 256)
        x, h = prefill(model, prompt, caches, drafter)
        st = tree_speculative_decode(model, drafter, caches, x, h, Pn, n_tok, K=K, mode=mode, plant=pl, **kw)
        assert st.tokens == ref.tokens[:n_tok], (st.tokens, ref.tokens[:n_tok])
        log(f"accept_hist {st.accept_hist} winners {st.rescues} depths {st.depths}")
        if pl is not None:
            assert set(st.rescues) == {0, 1, 2}, st.rescues
            for i, w in enumerate(st.rescues):
                assert w == (0, 1, 2, 0)[i % 4], (i, w)
        if mode == "adaptive_tree":
            assert all(1 <= d <= K for d in st.depths)
