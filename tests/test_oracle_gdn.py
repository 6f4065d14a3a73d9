"""Pins the oracle's Gated DeltaNet block (CPU only).

Checked against Hugging Face transformers' Qwen3NextGatedDeltaNet (the
published Qwen3-Next linear-attention block: grouped qkvz/ba projections,
causal depthwise conv of width 4 with SiLU, per-head q/k normalisation,
g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b), the gated delta rule,
gated RMSNorm, out_proj) run in float64 with the oracle's dequantised weights.
The one convention that differs: the reference normalises q and k with
rms_norm(., eps=1e-6) times dk^-1/2 (mlx_streaming/mtp/kv_cache.py:61-63),
which equals transformers' l2norm with eps = dk * 1e-6; the test runs
transformers with that eps.  The state path is checked against itself: a
batch continued from the conv rows and state of an earlier call equals one call
over the whole sequence, and a T-token call equals T one-token calls (the
reference's multistate invariant, tests/test_gated_delta_multistate.py:29-57).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

DIMS = dict(H=512, n_k=2, n_v=4, dk=128, dv=128)


def gdn_weights(orc, seed, H, n_k, n_v, dk, dv, bits=4):
    r = n_v // n_k
    G = {"H": H, "n_k": n_k, "n_v": n_v, "dk": dk, "dv": dv, "eps": 1e-6, "bits": bits}
    cd = 2 * n_k * dk + n_v * dv
    for i, (name, rows, cols) in enumerate((("qkvz", n_k * (2 * dk + 2 * r * dv), H), ("ba", 2 * n_v, H),
                                            ("out", H, n_v * dv))):
        G[name + "_w"], G[name + "_s"], G[name + "_b"] = orc.synth_quantized(seed, 30 + i, rows, cols, bits=bits)
    rng = np.random.default_rng(seed)
    G["in_norm"] = orc.f32_to_bf16((1.0 + 0.1 * rng.normal(size=H)).astype(np.float32))
    G["conv_w"] = orc.f32_to_bf16((0.4 * rng.normal(size=(cd, 4))).astype(np.float32))
    G["A_log"] = np.log(rng.uniform(1.0, 16.0, n_v)).astype(np.float32)
    G["dt_bias"] = rng.normal(size=n_v).astype(np.float32)
    G["norm_w"] = orc.f32_to_bf16((1.0 + 0.1 * rng.normal(size=dv)).astype(np.float32))
    return G


def test_gdn_matches_transformers_qwen3_next(orc, monkeypatch):
    from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig
    from transformers.models.qwen3_next import modeling_qwen3_next as M
    H, n_k, n_v, dk, dv = DIMS.values()
    T = 11
    G = gdn_weights(orc, 71, **DIMS)
    cfg = Qwen3NextConfig(hidden_size=H, linear_num_key_heads=n_k, linear_num_value_heads=n_v,
                          linear_key_head_dim=dk, linear_value_head_dim=dv, linear_conv_kernel_dim=4,
                          rms_norm_eps=1e-6)
    net = M.Qwen3NextGatedDeltaNet(cfg, layer_idx=0).double()
    r = n_v // n_k
    deq = lambda n, rows, cols: torch.from_numpy(orc.dequant(G[n + "_w"], G[n + "_s"], G[n + "_b"], rows, cols, 64, 4)
                                                 .astype(np.float64))
    with torch.no_grad():
        net.in_proj_qkvz.weight.copy_(deq("qkvz", n_k * (2 * dk + 2 * r * dv), H))
        net.in_proj_ba.weight.copy_(deq("ba", 2 * n_v, H))
        net.out_proj.weight.copy_(deq("out", H, n_v * dv))
        net.conv1d.weight.copy_(torch.from_numpy(orc.bf16_to_f32(G["conv_w"]).astype(np.float64))[:, None, :])
        net.A_log.copy_(torch.from_numpy(G["A_log"].astype(np.float64)))
        net.dt_bias.copy_(torch.from_numpy(G["dt_bias"].astype(np.float64)))
        net.norm.weight.copy_(torch.from_numpy(orc.bf16_to_f32(G["norm_w"]).astype(np.float64)))
    l2 = M.l2norm
    monkeypatch.setattr(M, "l2norm", lambda x, dim=-1, eps=1e-6: l2(x, dim=dim, eps=dk * 1e-6))
    x = orc.synth_bf16(71, 1, (T, H), 1.0)
    xn = orc.rmsnorm_bf16(x, G["in_norm"], 1e-6)[0]
    hs = torch.from_numpy(orc.bf16_to_f32(xn).astype(np.float64))[None]
    with torch.no_grad():
        ref = net(hs)[0].numpy()
    out, rows, states = orc.gdn_layer(x, G)
    got = out - orc.bf16_to_f32(x).astype(np.float64)
    # transformers computes g and runs the delta rule in float32 (.float(), .to(torch.float32)):
    # agreement to ~1e-6 relative; a wrong layout, tap order, head map or gate is O(1)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())
    assert np.abs(ref).max() > 1e-2


def test_gdn_state_path_equals_full_sequence(orc):
    G = gdn_weights(orc, 72, **DIMS)
    L, T = 13, 4
    x = orc.synth_bf16(72, 2, (L, DIMS["H"]), 1.0)
    full, rows, states = orc.gdn_layer(x, G)
    conv_in = rows[L - T - 3:L - T]
    tail, rows_t, states_t = orc.gdn_layer(x[L - T:], G, conv_in=conv_in, state_in=states[L - T - 1])
    np.testing.assert_array_equal(tail, full[L - T:])
    np.testing.assert_array_equal(states_t, states[L - T:])
    np.testing.assert_array_equal(rows_t, rows[L - T:])
    # one token at a time, carrying conv rows and state
    prev_rows = np.zeros((3, rows.shape[1]))
    st = None
    for t in range(L):
        o1, r1, s1 = orc.gdn_layer(x[t:t + 1], G, conv_in=prev_rows, state_in=st)
        np.testing.assert_array_equal(o1[0], full[t])
        np.testing.assert_array_equal(s1[0], states[t])
        prev_rows = np.concatenate([prev_rows[1:], r1])
        st = s1[0]


def test_gdn_decay_and_gate_extremes(orc):
    """g -> 0 (huge A_log) erases the carried state: the output no longer depends on it."""
    G = gdn_weights(orc, 73, **DIMS)
    G["A_log"] = np.full(DIMS["n_v"], 8.0, np.float32)
    G["dt_bias"] = np.full(DIMS["n_v"], 10.0, np.float32)
    x = orc.synth_bf16(73, 3, (1, DIMS["H"]), 1.0)
    s0 = np.random.default_rng(3).normal(size=(DIMS["n_v"], DIMS["dv"], DIMS["dk"]))
    a, _, sa = orc.gdn_layer(x, G, state_in=s0)
    b, _, sb = orc.gdn_layer(x, G, state_in=None)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)
    np.testing.assert_allclose(sa, sb, rtol=0, atol=1e-12)
