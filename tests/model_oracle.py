"""The CPU oracle's composition of a whole decoder model and of the MTP step.

TEST INFRASTRUCTURE ONLY.  Exports the weights of a ``vates_amd.decode.SpecModel``
(device tensors) into the dictionaries the oracle's block functions take, and
composes them the way the reference's verify forward does
(mlx_streaming/mtp/generate.py:101-220, ``forward_with_hidden``): embedding
lookup, per decoder layer the full-attention or Gated DeltaNet block then the
routed MoE block with its shared expert (qwen3_next's decoder layer), the
final RMSNorm and the head; and the MTP step (mlx_streaming/mtp/
qwen3_next_mtp.py:34-57).  Every block output is rounded to bf16 before the
next block, as the activations between blocks are bf16 in the reference.
The oracle carries its own caches (attention keys/values rounded to bf16,
Gated DeltaNet conv rows and states in float64), so a composition never reads
a GPU result.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc
from oracle.torch_bridge import u16, u32


def attn_dict(layer, rope_dim: int = 64, theta: float = 1e7, eps: float = 1e-6) -> dict:
    q, k, v, o, inn, qn, kn = layer._keep
    A = {"H": layer.hidden, "n_heads": layer.n_heads, "n_kv": layer.n_kv, "rope_dim": rope_dim, "theta": theta,
         "eps": eps, "bits": 4}
    for name, p in (("q", q), ("k", k), ("v", v), ("o", o)):
        A[name + "_w"], A[name + "_s"], A[name + "_b"] = u32(p.weight), u16(p.scales), u16(p.biases)
    A["in_norm"], A["q_norm"], A["k_norm"] = u16(inn), u16(qn), u16(kn)
    return A


def gdn_dict(layer, eps: float = 1e-6) -> dict:
    qkvz, ba, out, inn, conv, A_log, dt_bias, nw = layer._keep
    G = {"H": layer.hidden, "n_k": layer.n_k, "n_v": layer.n_v, "dk": 128, "dv": 128, "eps": eps, "bits": 4,
         "in_norm": u16(inn), "conv_w": u16(conv).reshape(-1, 4), "A_log": A_log.cpu().numpy(),
         "dt_bias": dt_bias.cpu().numpy(), "norm_w": u16(nw)}
    for name, p in (("qkvz", qkvz), ("ba", ba), ("out", out)):
        G[name + "_w"], G[name + "_s"], G[name + "_b"] = u32(p.weight), u16(p.scales), u16(p.biases)
    return G


def moe_dict(moe) -> dict:
    """vates_amd.moe.MoELayer -> oracle.moe_layer's dict (expert stacks taken
    back to the reference's pool layout: the layer stores them re-laid)."""
    mw = moe.reference_weights()
    d = moe.desc
    L = {"H": d.hidden, "I": d.inter, "E": d.num_experts, "k": d.top_k, "group": 64, "norm": int(d.norm_topk_prob),
         "router_bits": d.router_bits, "bits": 4, "cap": moe.cap, "sg_bits": d.shared_expert_gate_bits}
    r = mw["router"]
    L["router_w"], L["router_s"], L["router_b"] = u32(r.weight), u16(r.scales), u16(r.biases)
    for key, name in (("gate", "gate"), ("up", "up"), ("down", "down"), ("sh_gate", "shared_gate"),
                      ("sh_up", "shared_up"), ("sh_down", "shared_down")):
        p = mw[name]
        L[key + "_w"], L[key + "_s"], L[key + "_b"] = u32(p.weight), u16(p.scales), u16(p.biases)
    sg = mw["shared_expert_gate"]
    L["sg_w"], L["sg_s"], L["sg_b"] = u32(sg.weight), u16(sg.scales), u16(sg.biases)
    L["table"] = None if mw["slot_table"] is None else mw["slot_table"].cpu().numpy()
    L["bias"] = None if mw["router_logit_bias"] is None else mw["router_logit_bias"].cpu().numpy()
    L["norm_w"] = None if mw["norm_weight"] is None else u16(mw["norm_weight"])
    L["norm_eps"] = float(d.norm_eps)
    return L


def bf16(a: np.ndarray) -> np.ndarray:
    """float64/float32 -> bf16 bit patterns (round to nearest even)."""
    return orc.f32_to_bf16(np.asarray(a, np.float32))


class OracleAttnCache:
    def __init__(self, n_kv: int, max_len: int):
        self.k = np.zeros((n_kv, max_len, 256), np.uint16)
        self.v = np.zeros((n_kv, max_len, 256), np.uint16)


class OracleGdnCache:
    def __init__(self):
        self.conv = None    # float64 [3, conv_dim]: conv inputs of the last three positions
        self.state = None   # float64 [n_v, dv, dk]


class OracleModel:
    """The oracle's forward of a SpecModel (weights copied to host once)."""

    def __init__(self, model, max_len: int = 64):
        self.embed = u16(model.embed)
        self.head = u16(model.head)
        self.final_norm = u16(model.final_norm)
        self.eps = model.eps
        self.blocks = []
        for layer in model.layers:
            if layer.attn is not None:
                kind, d = "attn", attn_dict(layer.attn)
            elif layer.gdn is not None:
                kind, d = "gdn", gdn_dict(layer.gdn)
            else:
                kind, d = None, None
            self.blocks.append((kind, d, moe_dict(layer.moe)))
        self.max_len = max_len
        self.mtp = None
        if model.mtp is not None:
            w = model.mtp.w
            self.mtp = {"norm_emb": u16(w.norm_emb), "norm_hid": u16(w.norm_hid), "fc_w": u32(w.fc.weight),
                        "fc_s": u16(w.fc.scales), "fc_b": u16(w.fc.biases), "attn": attn_dict(w.attn),
                        "moe": moe_dict(w.moe), "norm": u16(w.norm)}

    def new_caches(self):
        caches = []
        for kind, d, _ in self.blocks:
            caches.append(OracleAttnCache(d["n_kv"], self.max_len) if kind == "attn" else
                          OracleGdnCache() if kind == "gdn" else None)
        return caches

    def block_attn(self, d, x, cache, pos0):
        T = x.shape[0]
        y, kn, vn = orc.attention_layer(x, d, pos0, cache.k, cache.v)
        cache.k[:, pos0:pos0 + T] = bf16(kn).transpose(1, 0, 2)
        cache.v[:, pos0:pos0 + T] = bf16(vn).transpose(1, 0, 2)
        return y

    @staticmethod
    def block_gdn(d, x, cache):
        T = x.shape[0]
        cd = 2 * d["n_k"] * 128 + d["n_v"] * 128
        conv_in = cache.conv if cache.conv is not None else np.zeros((3, cd))
        y, rows, states = orc.gdn_layer(x, d, conv_in=conv_in, state_in=cache.state)
        cache.conv = np.concatenate([conv_in, rows])[-3:]
        cache.state = states[-1]
        return y

    def forward(self, ids, caches, pos0: int, trace=None):
        """ids int [T] at positions pos0..; returns (logits float64 [T, V],
        pre-norm hidden bf16 bits [T, H]).  trace (a list) receives each
        block's bf16 output."""
        x = self.embed[np.asarray(ids, np.int64)]
        for (kind, d, L), cache in zip(self.blocks, caches):
            if kind == "attn":
                x = bf16(self.block_attn(d, x, cache, pos0))
            elif kind == "gdn":
                x = bf16(self.block_gdn(d, x, cache))
            if trace is not None and kind is not None:
                trace.append(x)
            _, x, _, _, _ = orc.moe_layer(x, L, residual=True)
            if trace is not None:
                trace.append(x)
        logits, _ = orc.lm_head(x, self.final_norm, self.eps, self.head)
        return logits, x

    def mtp_step(self, hidden_bf16, tok: int, cache: OracleAttnCache, pos0: int):
        """One MTP step: (MTP hidden after its final norm, bf16 bits [1, H],
        logits float64 [1, V])."""
        m = self.mtp
        H = self.embed.shape[1]
        emb = orc.rmsnorm_bf16(self.embed[tok:tok + 1], m["norm_emb"], self.eps)[0]
        hid = orc.rmsnorm_bf16(hidden_bf16, m["norm_hid"], self.eps)[0]
        cat = np.concatenate([emb, hid], axis=1)
        x = orc.qgemv_f64(m["fc_w"].reshape(H, -1), m["fc_s"].reshape(H, -1), m["fc_b"].reshape(H, -1), H, 2 * H,
                          orc.bf16_to_f32(cat))
        x = bf16(x)
        x = bf16(self.block_attn(m["attn"], x, cache, pos0))
        _, x, _, _, _ = orc.moe_layer(x, m["moe"], residual=True)
        Hn = orc.rmsnorm_bf16(x, m["norm"], self.eps)[0]
        logits, _ = orc.lm_head(Hn, None, self.eps, self.head)
        return Hn, logits


def rel_cos(got, ref):
    g = np.asarray(got, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    rel = float(np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30))
    cos = float(g @ r / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-30))
    return rel, cos


def clear_margin(logits_row, frac: float = 1e-2) -> bool:
    """True when the top-two margin of a float64 logit row exceeds frac of its
    largest magnitude (the argmax is then fixed against fp32/bf16 rounding)."""
    s = np.sort(logits_row)
    return bool(s[-1] - s[-2] > frac * np.abs(logits_row).max())


def check_mtp_steps(gpu, model, H, log):
    """Two chained MTP steps (the second at position 1, fed the first step's
    hidden and draft) against the oracle's composition: hidden rel <= 2e-2,
    cos >= 0.999; draft equal wherever the oracle's margin is clear."""
    import torch
    from vates_amd.mtp import MTPDrafter
    from vates_amd.synth import synth_bf16
    om = OracleModel(model, max_len=64)
    drafter = MTPDrafter(model.mtp, 64)
    ocache = OracleAttnCache(model.mtp.w.attn.n_kv, 64)
    h = synth_bf16(91, 77, (1, H), device=gpu)
    tok = torch.tensor([123], dtype=torch.int32, device=gpu)
    h_np, tok_np = u16(h), 123
    for step in range(2):
        am, Hn, logits = model.mtp.step(h, tok, drafter.cache, want_logits=True)
        torch.cuda.synchronize()
        Hr, lg = om.mtp_step(h_np, tok_np, ocache, step)
        rel, cos = rel_cos(orc.bf16_to_f32(u16(Hn)), orc.bf16_to_f32(Hr))
        log(f"mtp step {step}: rel={rel:.3g} cos={cos:.6f} draft={am.item()} oracle={int(np.argmax(lg[0]))}")
        assert rel <= 2e-2 and cos >= 0.999, (step, rel, cos)
        if clear_margin(lg[0]):
            assert am.item() == int(np.argmax(lg[0]))
        # chain both on the GPU's draft so the two compositions see the same tokens
        h, tok = Hn, am[:1].clone()
        h_np, tok_np = u16(Hn), int(am.item())


def check_tree_forward(gpu, model, prompt, P, K, log, seed=0):
    """forward_tree over P paths of K tokens against chain forwards of each
    path (bit for bit: argmax and hidden rows), then TreeCommit of a winner
    against a chain forward of the winner's accepted prefix: attention keys
    and values, Gated DeltaNet conv rows and the state before the next
    position, bit for bit.  Two cache sets filled by the same prefill."""
    import torch
    from vates_amd.accept import accept_greedy
    from vates_amd.attention import KVCache
    from vates_amd.decode import TreeCommit, prefill
    V = model.embed.shape[0]
    n = prompt.numel()
    A = model.new_caches(128)
    B = model.new_caches(128)
    x, _ = prefill(model, prompt, A)
    prefill(model, prompt, B)
    rng = np.random.default_rng(seed)
    paths = torch.tensor(rng.integers(0, V, (P, K)), dtype=torch.int32, device=gpu)
    verify = torch.cat([x.view(1, 1).expand(P, 1), paths[:, :K - 1]], dim=1).contiguous()
    am_t, hid_t, _ = model.forward_tree(verify.view(-1), A, n, P)
    torch.cuda.synchronize()
    assert all(c.length == n for c in A if c is not None), "a tree forward must not move the caches"
    for p in range(P):
        am_c, hid_c, _ = model.forward(verify[p], B, n)
        torch.cuda.synchronize()
        assert torch.equal(am_t[p * K:(p + 1) * K], am_c), f"path {p}: argmax differs from its chain forward"
        assert torch.equal(hid_t[p * K:(p + 1) * K].view(torch.int16), hid_c.view(torch.int16)), f"path {p}: hidden"
    log(f"  tree rows equal chain rows for {P} paths of {K}")
    # a winner: plant the model's own predictions into one path so that it matches m drafts
    for w, m in ((P - 1, K), (0, 0), (P // 2, 1)):
        drafts = paths.clone()
        preds = am_t.view(P, K).clone()
        drafts[w, :m] = preds[w, :m]
        if m < K:
            drafts[w, m] = (preds[w, m] + 1) % V
        for q in range(P):
            if q != w:
                drafts[q, 0] = (preds[q, 0] + 1) % V  # other paths match nothing
        rec = accept_greedy(drafts, preds.view(-1), mode=0)
        r = rec.cpu().tolist()
        acc = min(m + 1, K)
        assert r[1] == m and r[2] == acc and r[3] == (w if m > 0 else 0), r
        w = r[3]
        A2 = model.new_caches(128)
        B2 = model.new_caches(128)
        prefill(model, prompt, A2)
        prefill(model, prompt, B2)
        model.forward_tree(verify.view(-1), A2, n, P)
        TreeCommit(A2, P, K)(rec, pos0=n)
        model.forward(verify[w, :acc].contiguous(), B2, n)
        torch.cuda.synchronize()
        for li, (ca, cb) in enumerate(zip(A2, B2)):
            if ca is None:
                continue
            if isinstance(ca, KVCache):
                for name in ("keys", "values"):
                    ga = getattr(ca, name)(n, n + acc)
                    gb = getattr(cb, name)(n, n + acc)
                    assert torch.equal(ga.view(torch.int16), gb.view(torch.int16)), (li, name, w, acc)
            else:
                assert torch.equal(ca.conv_rows(n + acc).view(torch.int16), cb.conv_rows(n + acc).view(torch.int16)), \
                    (li, "conv", w, acc)
                assert torch.equal(ca.state_before(n + acc).view(torch.int32),
                                   cb.state_before(n + acc).view(torch.int32)), (li, "state", w, acc)
        log(f"  commit of path {w} with {acc} accepted equals the chain forward of its prefix")
