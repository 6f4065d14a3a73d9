"""GPU tests of the MTP draft step and the speculative decode loop.

* One MTP step (embedding norm, hidden norm, fc, attention block, MoE block,
  final norm, head argmax) against the CPU oracle's composition of the pinned
  pieces: hidden state relative L2 <= 2e-2 and cosine >= 0.999 (bf16
  activations through five blocks), draft token equal wherever the oracle's
  top-two logit margin exceeds 1e-2 of the logit scale.
* Speculative decoding with K=3 emits exactly the tokens of non-speculative
  greedy decoding (the reference's lossless invariant,
  tests/test_mtp_generate.py:421-489), with scripted drafts that make every
  acceptance length 0..K occur, and with the MTP layer's own drafts.
* draft_paths takes its first tokens from the top-P of the MTP logits.
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
    log("case: one MTP step vs the oracle composition")
    import torch
    from vates_amd.mtp import MTPDrafter
    mtp = model.mtp
    w = mtp.w
    H, V = SMALL["hidden"], SMALL["vocab"]
    drafter = MTPDrafter(mtp, 64)
    from vates_amd.synth import synth_bf16
    h = synth_bf16(91, 77, (1, H), device=gpu)
    tok = torch.tensor([123], dtype=torch.int32, device=gpu)
    am, Hn, logits = mtp.step(h, tok, drafter.cache, want_logits=True)
    torch.cuda.synchronize()
    # oracle: emb/hid norms -> fc -> attention -> MoE (post-attention norm inside) -> norm -> head
    emb = orc.rmsnorm_bf16(u16(w.embed)[123:124], u16(w.norm_emb), 1e-6)[0]
    hid = orc.rmsnorm_bf16(u16(h), u16(w.norm_hid), 1e-6)[0]
    cat = np.concatenate([emb, hid], axis=1)
    fc = w.fc
    x = orc.qgemv_f64(u32(fc.weight).reshape(H, -1), u16(fc.scales).reshape(H, -1), u16(fc.biases).reshape(H, -1),
                      H, 2 * H, orc.bf16_to_f32(cat))
    xb = orc.f32_to_bf16(x.astype(np.float32))
    at = w.attn
    A = {"H": H, "n_heads": SMALL["n_heads"], "n_kv": SMALL["n_kv_heads"], "rope_dim": 64, "theta": 1e7,
         "eps": 1e-6, "bits": 4}
    q, k, v, o, inn, qn, kn = at._keep
    for name, p in (("q", q), ("k", k), ("v", v), ("o", o)):
        A[name + "_w"], A[name + "_s"], A[name + "_b"] = u32(p.weight), u16(p.scales), u16(p.biases)
    A["in_norm"], A["q_norm"], A["k_norm"] = u16(inn), u16(qn), u16(kn)
    zero = np.zeros((SMALL["n_kv_heads"], 64, 256), np.uint16)
    ya, _, _ = orc.attention_layer(xb, A, 0, zero, zero)
    yab = orc.f32_to_bf16(ya.astype(np.float32))
    moe = w.moe
    mw = moe._keep
    L = {"H": H, "I": SMALL["inter"], "E": SMALL["num_experts"], "k": SMALL["top_k"], "group": 64, "norm": 1,
         "router_bits": moe.desc.router_bits, "bits": 4, "cap": moe.cap, "sg_bits": 8}
    L["router_w"], L["router_s"], L["router_b"] = u32(mw[0].weight), u16(mw[0].scales), u16(mw[0].biases)
    for key, p in (("gate", mw[1]), ("up", mw[2]), ("down", mw[3]), ("sh_gate", mw[4]), ("sh_up", mw[5]),
                   ("sh_down", mw[6])):
        L[key + "_w"], L[key + "_s"], L[key + "_b"] = u32(p.weight), u16(p.scales), u16(p.biases)
    L["sg_w"], L["sg_s"], L["sg_b"] = u32(mw[7].weight), u16(mw[7].scales), u16(mw[7].biases)
    L["table"] = None if mw[8] is None else mw[8].cpu().numpy()
    L["bias"] = None if mw[9] is None else mw[9].cpu().numpy()
    L["norm_w"] = u16(mw[10])
    L["norm_eps"] = 1e-6
    ym, ymb, _, _, _ = orc.moe_layer(yab, L, residual=True)
    Hr = orc.rmsnorm_bf16(ymb, u16(w.norm), 1e-6)[0]
    got = orc.bf16_to_f32(u16(Hn)).astype(np.float64).ravel()
    ref = orc.bf16_to_f32(Hr).astype(np.float64).ravel()
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    cos = got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref))
    assert rel <= 2e-2 and cos >= 0.999, (rel, cos)
    lg, _ = orc.lm_head(Hr, None, 1e-6, u16(w.lm_head))
    srt = np.sort(lg[0])
    if srt[-1] - srt[-2] > 1e-2 * np.abs(lg).max():
        assert am.item() == int(np.argmax(lg[0]))


class ScriptedDrafter:
    """Runs the MTP drafter (kernels and cache writes) and replaces its drafts by
    the true continuation for the first m tokens of each step and a wrong token
    after, cycling m through 0..K."""

    def __init__(self, inner, truth, prompt_len):
        self.inner, self.truth, self.P, self.n = inner, truth, prompt_len, 0
        self.cache, self.mtp = inner.cache, inner.mtp

    def draft(self, H_last, x, K):
        import torch
        d = self.inner.draft(H_last, x, K)
        base = self.cache.length - K + 1 - self.P  # index of the next token in the greedy stream
        m = self.n % (K + 1)
        self.n += 1
        planted = [self.truth[base + i] if i < m else (self.truth[base + i] + 1) % SMALL["vocab"] for i in range(K)]
        d.copy_(torch.tensor(planted, dtype=torch.int32, device=d.device))
        return d

    def sync(self, start, h_seq, tokens):
        self.inner.sync(start, h_seq, tokens)


def test_speculative_equals_greedy(gpu, model):
    import torch
    from vates_amd.decode import greedy_decode, prefill, speculative_decode
    from vates_amd.mtp import MTPDrafter
    n_tok, K = 40, 3
    prompt = _prompt(gpu)
    caches = model.new_caches(256)
    x, h = prefill(model, prompt, caches)
    ref = greedy_decode(model, caches, x, prompt.numel(), n_tok + K + 1)
    log(f"case: greedy stream {ref.tokens[:12]}...")
    for scripted in (True, False):
        log(f"case: speculative K=3 scripted={scripted}")
        caches = model.new_caches(256)
        drafter = MTPDrafter(model.mtp, 256)
        x, h = prefill(model, prompt, caches, drafter)
        d = ScriptedDrafter(drafter, ref.tokens, prompt.numel()) if scripted else drafter
        st = speculative_decode(model, d, caches, x, h, prompt.numel(), n_tok, K=K)
        assert st.tokens == ref.tokens[:n_tok], (st.tokens, ref.tokens[:n_tok])
        if scripted:
            assert set(st.accept_hist) == set(range(K + 1)), st.accept_hist
        log(f"accept_hist {st.accept_hist} steps {st.steps}")


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


def test_graph_decode_equals_greedy(gpu, model):
    """The captured-graph step (positions on the device) emits the greedy stream,
    with the MTP layer's drafts and with planted drafts that make every
    acceptance length 0..K occur."""
    import torch
    from vates_amd.decode import GraphSpecDecoder, greedy_decode, prefill
    from vates_amd.mtp import MTPDrafter
    n_tok, K = 40, 3
    prompt = _prompt(gpu, seed=8)
    caches = model.new_caches(256)
    x, h = prefill(model, prompt, caches)
    ref = greedy_decode(model, caches, x, prompt.numel(), n_tok + 2 * (K + 1))
    P = prompt.numel()
    for planted in (False, True):
        log(f"case: graph speculative K=3 planted={planted}")
        caches = model.new_caches(256)
        drafter = MTPDrafter(model.mtp, 256)
        x, h = prefill(model, prompt, caches, drafter)
        dec = GraphSpecDecoder(model, drafter, caches, K=K, planted=planted)
        dec.start(x, h, P)

        def plant(step, pos):
            m = step % (K + 1)
            base = pos - P  # greedy stream index of the token at position pos + 1
            return [ref.tokens[base + i] if i < m else (ref.tokens[base + i] + 1) % SMALL["vocab"] for i in range(K)]

        st = dec.run(n_tok, plant=plant if planted else None)
        assert st.tokens == ref.tokens[:n_tok], (st.tokens, ref.tokens[:n_tok])
        if planted:
            assert set(st.accept_hist) == set(range(K + 1)), st.accept_hist
        log(f"accept_hist {st.accept_hist} steps {st.steps}")
        # the host view of the caches follows the device positions
        assert all(c.length == P + sum(m + 1 for m in st.accept_hist) for c in caches if c is not None)


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
