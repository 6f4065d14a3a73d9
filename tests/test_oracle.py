"""Pins the CPU oracle against the reference's known answers, closed forms,
library routines (numpy/scipy) and invariants.  CPU only."""
import json
from pathlib import Path

import numpy as np
import pytest
from scipy.special import softmax as sp_softmax

GOLD = Path(__file__).resolve().parent / "golden"
KA = json.loads((GOLD / "reference_known_answers.json").read_text())


# ----------------------------------------------------------------- RNG / bf16
def test_philox_known_answers(orc):
    for case in KA["philox4x32_10"]:
        assert orc.philox(case["ctr"], case["key"]) == case["out"]


def test_bf16_round_to_nearest_even(orc):
    cases = {1.0: 0x3F80, -2.0: 0xC000, 1.00390625: 0x3F80,  # exact tie -> even
             1.01171875: 0x3F82,  # tie between 0x3F81 and 0x3F82 -> even
             3.0e38: 0x7F62, 0.0: 0x0000}
    for v, bits in cases.items():
        assert orc.lib().orc_f32_to_bf16(v) == bits, v
    x = np.random.default_rng(0).normal(size=4096).astype(np.float32)
    b = orc.f32_to_bf16(x)
    back = orc.bf16_to_f32(b)
    # round trip error below half an ulp of bf16 (8 significant bits)
    assert np.all(np.abs(back - x) <= np.abs(x) * 2.0 ** -8 + 1e-38)


def test_synth_statistics(orc):
    v = orc.synth_normal(11, 3, 1 << 20, 0.02)
    assert abs(v.mean()) < 1e-4
    assert abs(v.std() - 0.02) < 2e-4
    # Irwin-Hall(4) support is +-131070 * scale = +-3.46 std
    assert np.abs(v).max() <= 131070 * orc.scale_for(0.02) * (1 + 1e-6)
    # deterministic, and distinct streams differ
    assert np.array_equal(v[:1000], orc.synth_normal(11, 3, 1000, 0.02))
    assert not np.array_equal(v[:1000], orc.synth_normal(11, 4, 1000, 0.02))


# ------------------------------------------------------------------- dequant
def test_dequant_nibble_order_known_answers(orc):
    for case in KA["dequant_words"]:
        bits = case["bits"]
        cols = 32 // bits
        # pad to a full 64-column group: row = [word, 0, ...]
        words = np.zeros((1, 64 * bits // 32), dtype=np.uint32)
        words[0, 0] = case["word"]
        one = orc.f32_to_bf16(np.array([1.0], np.float32))
        zero = orc.f32_to_bf16(np.array([0.0], np.float32))
        s = np.full((1, 1), one[0], np.uint16)
        b = np.full((1, 1), zero[0], np.uint16)
        d = orc.dequant(words, s, b, 1, 64, 64, bits)
        assert list(d[0, :cols]) == case["q"]


def test_dequant_affine_known_values(orc):
    words = np.full((1, 8), 0x76543210, dtype=np.uint32)  # q = 0..7 repeating
    s = orc.f32_to_bf16(np.array([[0.5]], np.float32))
    b = orc.f32_to_bf16(np.array([[-1.0]], np.float32))
    d = orc.dequant(words, s, b, 1, 64, 64, 4)
    assert list(d[0, :8]) == [-1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 2.5]


def test_dequant_reference_fixture(orc):
    """test_native_moe_ext.py:20-47 writes weight = arange words, scale =
    bf16(0.001), bias = 0 for a [8, 32, 64] 6-bit stack; the same fixture at
    4 bits: every value is q * bf16(0.001) with q the nibble of the word."""
    out_dim, in_dim = 4, 64
    words = np.arange(out_dim * in_dim // 8, dtype=np.uint32).reshape(out_dim, in_dim // 8)
    s = np.full((out_dim, 1), orc.f32_to_bf16(np.array([0.001], np.float32))[0], np.uint16)
    b = np.zeros((out_dim, 1), np.uint16)
    d = orc.dequant(words, s, b, out_dim, in_dim, 64, 4)
    sc = float(orc.bf16_to_f32(s[0])[0])
    # word w holds nibbles of w: column 8*i + j of row r has nibble j of word 8*r + i
    assert d[0, 0:8].tolist() == [0.0] * 8
    assert d[0, 8:16].tolist() == [np.float32(sc)] + [0.0] * 7
    assert d[3, 56:64].tolist() == [np.float32(v * sc) for v in (15, 1, 0, 0, 0, 0, 0, 0)]


def test_quantize_minimises_error_and_round_trips(orc):
    rng = np.random.default_rng(1)
    w = (rng.normal(size=(8, 256)) * 0.02).astype(np.float32)
    for bits in (4, 8):
        wq, s, b = orc.quantize(w, 64, bits)
        d = orc.dequant(wq, s, b, 8, 256, 64, bits)
        sf = orc.bf16_to_f32(s).repeat(64, axis=1)
        bf = orc.bf16_to_f32(b).repeat(64, axis=1)
        # brute force: the stored q is the nearest level in [0, qmax]
        levels = np.arange(2 ** bits, dtype=np.float64)
        cand = levels[None, None, :] * sf[..., None].astype(np.float64) + bf[..., None].astype(np.float64)
        best = np.abs(cand - w[..., None]).min(axis=-1)
        err = np.abs(d.astype(np.float64) - w)
        assert np.all(err <= best + 1e-7 * np.abs(w) + 1e-12)
        # and within half a step plus what rounding scale and bias to bf16 moves the grid
        g = w.reshape(8, 4, 64)
        mn, mx = g.min(-1).repeat(64, 1), g.max(-1).repeat(64, 1)
        qmax = 2 ** bits - 1
        slack = np.abs(bf - mn) + qmax * np.abs(sf - (mx - mn) / qmax)
        assert np.all(err <= 0.5 * sf + slack + 1e-7)


def test_synth_quantized_matches_quantize_of_synth(orc):
    rows, cols = 5, 128
    wq, s, b = orc.synth_quantized(3, 9, rows, cols, 64, 4, 0.02)
    raw = orc.synth_normal(3, 9, rows * cols, 0.02).reshape(rows, cols)
    wq2, s2, b2 = orc.quantize(raw, 64, 4)
    assert np.array_equal(wq, wq2) and np.array_equal(s, s2) and np.array_equal(b, b2)


# --------------------------------------------------------- GEMV and routing
def test_qgemv_matches_numpy_float64(orc):
    rng = np.random.default_rng(2)
    rows, cols = 24, 512
    wq, s, b = orc.quantize((rng.normal(size=(rows, cols)) * 0.02).astype(np.float32), 64, 4)
    x = rng.normal(size=(3, cols)).astype(np.float32)
    y = orc.qgemv_f64(wq, s, b, rows, cols, x)
    ref = x.astype(np.float64) @ orc.dequant(wq, s, b, rows, cols).astype(np.float64).T
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)


def test_router_logits_fp32_order_close_to_float64(orc):
    E, H = 64, 512
    wq, s, b = orc.synth_quantized(4, 1, E, H, bits=8)
    x = orc.synth_bf16(4, 2, (2, H), 1.0)
    bias = np.linspace(-1, 1, E).astype(np.float32)
    lg = orc.router_logits(wq, s, b, x, E, H, bits=8, bias=bias)
    ref = orc.bf16_to_f32(x).astype(np.float64) @ orc.dequant(wq, s, b, E, H, 64, 8).astype(np.float64).T + bias
    np.testing.assert_allclose(lg, ref, rtol=1e-5, atol=1e-5)
    # same inputs, same bits
    assert np.array_equal(lg, orc.router_logits(wq, s, b, x, E, H, bits=8, bias=bias))


def _topk_bruteforce(logits, k, norm):
    T, E = logits.shape
    ids = np.zeros((T, k), np.int64)
    scores = np.zeros((T, k))
    for t in range(T):
        order = np.lexsort((np.arange(E), -logits[t].astype(np.float64)))  # value desc, index asc
        ids[t] = order[:k]
        p = sp_softmax(logits[t].astype(np.float64))
        sel = p[ids[t]]
        scores[t] = sel / sel.sum() if norm else sel
    return ids, scores


def test_topk_softmax_matches_bruteforce(orc):
    rng = np.random.default_rng(3)
    logits = rng.normal(size=(6, 512)).astype(np.float32)
    logits[2, 17] = logits[2, 400] = logits[2].max() + 1  # tie -> lower index first
    for norm in (True, False):
        ids, sc = orc.topk_softmax(logits, 10, norm)
        rid, rsc = _topk_bruteforce(logits, 10, norm)
        assert np.array_equal(ids, rid)
        np.testing.assert_allclose(sc, rsc, rtol=1e-6)
    assert ids[2, 0] == 17 and ids[2, 1] == 400


def test_topk_nan_ranks_last(orc):
    logits = np.array([[np.nan, 1.0, 3.0, np.nan, 2.0]], np.float32)
    ids, _ = orc.topk_softmax(logits, 4, True)
    assert ids[0].tolist() == [2, 4, 1, 0]


# ------------------------------------------------------------------ experts
def _pool(orc, seed, cap, H, I):
    P = {}
    P["gate_w"], P["gate_s"], P["gate_b"] = orc.synth_quantized(seed, 2, cap * I, H)
    P["up_w"], P["up_s"], P["up_b"] = orc.synth_quantized(seed, 3, cap * I, H)
    P["down_w"], P["down_s"], P["down_b"] = orc.synth_quantized(seed, 4, cap * H, I)
    return P


def _expert_np(orc, P, slot, x, H, I):
    sl = slice(slot * I, (slot + 1) * I)
    g = x @ orc.dequant(P["gate_w"][sl], P["gate_s"][sl], P["gate_b"][sl], I, H).astype(np.float64).T
    u = x @ orc.dequant(P["up_w"][sl], P["up_s"][sl], P["up_b"][sl], I, H).astype(np.float64).T
    a = g / (1 + np.exp(-g)) * u  # test_fused_moe_runtime.py:53: gate*sigmoid(gate)*up
    dl = slice(slot * H, (slot + 1) * H)
    return a @ orc.dequant(P["down_w"][dl], P["down_s"][dl], P["down_b"][dl], H, I).astype(np.float64).T


def test_fused_moe_slots_matches_numpy(orc):
    H, I, cap, T, k = 256, 128, 6, 3, 3
    P = _pool(orc, 5, cap, H, I)
    rng = np.random.default_rng(5)
    x = rng.normal(size=(T, H)).astype(np.float32)
    slots = np.array([[0, 5, 2], [2, 2, 1], [4, 0, 3]], np.int32)  # duplicates allowed
    scores = rng.random((T, k)).astype(np.float32)
    out = orc.fused_moe_slots(x, slots, scores, P, T, k, H, I, cap)
    ref = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            ref[t] += scores[t, j] * _expert_np(orc, P, slots[t, j], x[t].astype(np.float64), H, I)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-7)
    bad = slots.copy()
    bad[1, 1] = cap
    with pytest.raises(RuntimeError):
        orc.fused_moe_slots(x, bad, scores, P, T, k, H, I, cap)


def test_moe_layer_is_router_topk_experts_shared(orc):
    """Full layer == router -> top-k -> table -> experts -> combine -> shared,
    each piece pinned above, composed with numpy."""
    H, I, E, k, T, cap = 512, 128, 64, 4, 2, 64
    L = {"H": H, "I": I, "E": E, "k": k, "group": 64, "norm": 1, "router_bits": 8, "bits": 4, "cap": cap,
         "sg_bits": 8}
    L["router_w"], L["router_s"], L["router_b"] = orc.synth_quantized(8, 1, E, H, bits=8)
    L.update(_pool(orc, 8, cap, H, I))
    sh = _pool(orc, 9, 1, H, I)
    for key, v in sh.items():
        L["sh_" + key] = v
    L["sg_w"], L["sg_s"], L["sg_b"] = orc.synth_quantized(8, 8, 1, H, bits=8)
    L["table"] = np.random.default_rng(8).permutation(E).astype(np.int32)
    L["bias"] = np.log(1.0 / np.arange(1, E + 1) ** 1.1).astype(np.float32)
    x = orc.synth_bf16(8, 9, (T, H), 1.0)
    out_f32, out_bf16, ids, sc, sl = orc.moe_layer(x, L, residual=True)
    lg = orc.router_logits(L["router_w"], L["router_s"], L["router_b"], x, E, H, bits=8, bias=L["bias"])
    rid, rsc = orc.topk_softmax(lg, k, True)
    assert np.array_equal(ids, rid) and np.array_equal(sc, rsc)
    assert np.array_equal(sl, L["table"][ids])
    xf = orc.bf16_to_f32(x).astype(np.float64)
    sgw = orc.dequant(L["sg_w"], L["sg_s"], L["sg_b"], 1, H, 64, 8).astype(np.float64)
    for t in range(T):
        ref = xf[t].copy()
        for j in range(k):
            ref += float(sc[t, j]) * _expert_np(orc, L, int(sl[t, j]), xf[t], H, I)
        gate = 1 / (1 + np.exp(-(sgw[0] @ xf[t])))
        shp = {kk[3:]: v for kk, v in L.items() if kk.startswith("sh_")}
        ref += gate * _expert_np(orc, shp, 0, xf[t], H, I)
        np.testing.assert_allclose(out_f32[t], ref, rtol=1e-5, atol=1e-6)
    assert np.array_equal(out_bf16, orc.f32_to_bf16(out_f32))
    # the same layer with its own routing given reproduces every bit
    r32, r16 = orc.moe_layer_routed(x, L, ids, sc, residual=True)
    assert np.array_equal(r32.view(np.uint32), out_f32.view(np.uint32)) and np.array_equal(r16, out_bf16)
    # and a different routing changes it
    ids2 = ids.copy()
    ids2[0, 0] = (ids2[0, 0] + 1) % E
    while ids2[0, 0] in ids[0]:
        ids2[0, 0] = (ids2[0, 0] + 1) % E
    d32, _ = orc.moe_layer_routed(x, L, ids2, sc, residual=True)
    assert not np.array_equal(d32[0], out_f32[0]) and np.array_equal(d32[1], out_f32[1])


def test_oracle_small_fixture_unchanged(orc):
    from tests.golden.make_fixtures import oracle_small
    gold = np.load(GOLD / "oracle_small.npz")
    now = oracle_small()
    for key in gold.files:
        assert np.array_equal(gold[key], now[key]), key


# ---------------------------------------------------- expert-major prefill
def test_route_reduce_known_answer(orc):
    c = KA["route_reduce"]
    out = orc.route_reduce(np.array(c["previous"], np.float32), np.array(c["weighted"], np.float32),
                           np.array(c["assignment_pos"], np.int32), c["routes_per_token"])
    assert out.tolist() == c["expected"]


def _bf16(orc, a):
    return orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(a, np.float32)))


def test_route_reduce_equals_bf16_scatter_chain(orc):
    """test_expert_major_prefill.py:106-132: the per-token canonical-order
    reduce equals a bf16 scatter chain applied rank by rank."""
    tokens, routes, hidden = 17, 4, 8
    prev = _bf16(orc, _bf16(orc, np.arange(tokens * hidden).reshape(tokens, hidden) % 31) / 31)
    pos = (np.arange(37) * 11) % (tokens * routes)
    w = _bf16(orc, _bf16(orc, np.arange(37 * hidden).reshape(37, hidden) % 43) / 43)
    chain = prev.copy()
    for rank in range(routes):
        for i, p in enumerate(pos):
            if p % routes == rank:
                chain[p // routes] = _bf16(orc, chain[p // routes] + w[i])
    got = orc.route_reduce(prev, w, pos.astype(np.int32), routes, bf16_acc=True)
    assert np.array_equal(got, chain)


def test_expert_major_toy_known_answer(orc):
    c = KA["expert_major_toy"]
    x = np.array(c["x"], np.float32)
    inds = np.array(c["inds"], np.int32)
    scores = np.array(c["scores"], np.float32)
    k = inds.shape[1]
    counts, groups = orc.expert_major_groups(inds, c["num_experts"], c["layer_cap"])
    assert [list(g[0]) for g in groups] == c["group_loads"]
    out = np.zeros_like(x)
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")
    prefix = 0
    for experts, n in groups:
        pos = order[prefix:prefix + n]
        prefix += n
        y = x[pos // k] + (flat[pos][:, None] + 1).astype(np.float32)  # y_e(x) = x + e + 1
        out = orc.route_reduce(out, y * scores.reshape(-1)[pos][:, None], pos.astype(np.int32), k)
    np.testing.assert_allclose(out, np.array(c["expected"], np.float32), rtol=1e-6, atol=1e-6)


def test_expert_major_groups_respect_limits(orc):
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 512, size=20480)
    counts, groups = orc.expert_major_groups(ids, 512, 128, 32768)
    assert np.array_equal(counts, np.bincount(ids, minlength=512))
    seen = [e for g, _ in groups for e in g]
    assert seen == sorted(np.nonzero(counts)[0].tolist())
    for g, n in groups:
        assert len(g) <= 128 and n == counts[list(g)].sum()
        assert n <= 32768 or len(g) == 1


# --------------------------------------------------------------- acceptance
def test_accept_prefix_known_answers(orc):
    for c in KA["accept_prefix"]:
        emitted, m, acc = orc.accept_greedy(c["drafts"], c["preds"], mode=0)
        assert m == c["matched"]


def test_accept_emission_rules(orc):
    d = [11, 22, 33]
    # T=K mode (generate.py:819, :850-856)
    assert orc.accept_greedy(d, [11, 22, 99], 0) == ([11, 22, 99], 2, 3)
    assert orc.accept_greedy(d, [99, 22, 33], 0) == ([99], 0, 1)
    assert orc.accept_greedy(d, [11, 22, 33], 0) == ([11, 22, 33], 3, 3)
    # T=K+1 mode: bonus token after a full match
    assert orc.accept_greedy(d, [11, 22, 33, 44], 1) == ([11, 22, 33, 44], 3, 4)
    assert orc.accept_greedy(d, [11, 5, 33, 44], 1) == ([11, 5], 1, 2)


def test_accept_tree_prefers_longest_then_lowest_path(orc):
    paths = np.array([[1, 2, 3], [1, 2, 9], [1, 2, 3]], np.int32)
    preds = np.array([[1, 2, 7], [1, 2, 9], [1, 2, 9]], np.int32)
    best, emitted, m, acc = orc.accept_tree(paths, preds)
    assert (best, m) == (1, 3) and emitted == [1, 2, 9] and acc == 3
    preds2 = np.array([[1, 5, 0], [1, 6, 0], [1, 2, 0]], np.int32)
    best, emitted, m, acc = orc.accept_tree(paths, preds2)
    assert (best, m) == (2, 2) and emitted == [1, 2, 0]
    preds3 = np.array([[1, 5, 0], [1, 6, 0], [1, 7, 0]], np.int32)
    assert orc.accept_tree(paths, preds3)[0] == 0  # tie at matched=1 -> lowest path index


def test_argmax_rows_ties_and_nan(orc):
    lg = np.array([[0.0, 2.0, 2.0, np.nan], [np.nan, np.nan, -1.0, -1.0]], np.float32)
    assert orc.argmax_rows(lg).tolist() == [1, 2]


def test_rmsnorm_and_head_match_torch_float64(orc):
    """The head's norm and product against torch's rms_norm and a float64 matmul
    (mlx RMSNorm semantics: x / sqrt(mean(x^2) + eps) * w, rounded to bf16 once).
    Error bars: the bf16 rounding of the normalised value (half an ulp, 2^-9
    relative) and nothing for the product, which the oracle sums in double."""
    import torch
    rng = np.random.default_rng(17)
    T, H, V = 3, 512, 700
    x = orc.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32) * 3)
    w = orc.f32_to_bf16(1.0 + 0.1 * rng.standard_normal(H).astype(np.float32))
    W = orc.f32_to_bf16(0.05 * rng.standard_normal((V, H)).astype(np.float32))
    xn, inv = orc.rmsnorm_bf16(x, w, 1e-6)
    ref = torch.nn.functional.rms_norm(torch.tensor(orc.bf16_to_f32(x), dtype=torch.float64), (H,),
                                       torch.tensor(orc.bf16_to_f32(w), dtype=torch.float64), eps=1e-6).numpy()
    got = orc.bf16_to_f32(xn).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-30)
    # the sign and the position of every element survive (no transposed or dropped term)
    assert np.array_equal(np.sign(got), np.sign(ref))
    logits, absdot = orc.lm_head(x, w, 1e-6, W)
    np.testing.assert_allclose(logits, got @ orc.bf16_to_f32(W).astype(np.float64).T, rtol=0, atol=1e-9)
    assert np.all(absdot >= np.abs(logits))
    # no norm: plain product
    lg2, _ = orc.lm_head(x, None, 1e-6, W)
    np.testing.assert_allclose(lg2, orc.bf16_to_f32(x).astype(np.float64) @ orc.bf16_to_f32(W).astype(np.float64).T,
                               rtol=0, atol=1e-9)
