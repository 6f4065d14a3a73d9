"""Pins the oracle's full-attention block (CPU only).

Checked against Hugging Face transformers' Qwen3NextAttention (the published
Qwen3-Next architecture: [q | gate] per head, q/k RMSNorm with (1 + w), partial
rotary with rotate_half, GQA, causal softmax, sigmoid gate, o_proj) run in
float64 with the oracle's dequantised weights; and for the KV-cache path,
against itself: attending over a cache filled by an earlier call equals one
call over the whole sequence.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")


def _attn_weights(orc, seed, H, n_heads, n_kv, bits=4):
    A = {"H": H, "n_heads": n_heads, "n_kv": n_kv, "rope_dim": 64, "theta": 1e7, "eps": 1e-6, "bits": bits}
    for i, (name, rows, cols) in enumerate((("q", n_heads * 512, H), ("k", n_kv * 256, H), ("v", n_kv * 256, H),
                                            ("o", H, n_heads * 256))):
        A[name + "_w"], A[name + "_s"], A[name + "_b"] = orc.synth_quantized(seed, 10 + i, rows, cols, bits=bits)
    A["in_norm"] = orc.f32_to_bf16((1.0 + 0.1 * np.random.default_rng(seed).normal(size=H)).astype(np.float32))
    A["q_norm"] = orc.f32_to_bf16((1.0 + 0.1 * np.random.default_rng(seed + 1).normal(size=256)).astype(np.float32))
    A["k_norm"] = orc.f32_to_bf16((1.0 + 0.1 * np.random.default_rng(seed + 2).normal(size=256)).astype(np.float32))
    return A


def test_attention_matches_transformers_qwen3_next(orc):
    from transformers.models.qwen3_next.configuration_qwen3_next import Qwen3NextConfig
    from transformers.models.qwen3_next import modeling_qwen3_next as M
    H, n_heads, n_kv, T = 512, 4, 2, 9
    A = _attn_weights(orc, 61, H, n_heads, n_kv)
    cfg = Qwen3NextConfig(hidden_size=H, num_attention_heads=n_heads, num_key_value_heads=n_kv, head_dim=256,
                          rms_norm_eps=1e-6, attention_bias=False,
                          rope_parameters={"rope_type": "default", "rope_theta": 1e7, "partial_rotary_factor": 0.25})
    cfg._attn_implementation = "eager"
    att = M.Qwen3NextAttention(cfg, layer_idx=3).double()
    deq = lambda n, r, c: torch.from_numpy(orc.dequant(A[n + "_w"], A[n + "_s"], A[n + "_b"], r, c, 64, 4)
                                           .astype(np.float64))
    with torch.no_grad():
        att.q_proj.weight.copy_(deq("q", n_heads * 512, H))
        att.k_proj.weight.copy_(deq("k", n_kv * 256, H))
        att.v_proj.weight.copy_(deq("v", n_kv * 256, H))
        att.o_proj.weight.copy_(deq("o", H, n_heads * 256))
        att.q_norm.weight.copy_(torch.from_numpy(orc.bf16_to_f32(A["q_norm"]).astype(np.float64) - 1.0))
        att.k_norm.weight.copy_(torch.from_numpy(orc.bf16_to_f32(A["k_norm"]).astype(np.float64) - 1.0))
    x = orc.synth_bf16(61, 1, (T, H), 1.0)
    xn = orc.rmsnorm_bf16(x, A["in_norm"], 1e-6)[0]
    rope = M.Qwen3NextRotaryEmbedding(cfg)
    hs = torch.from_numpy(orc.bf16_to_f32(xn).astype(np.float64))[None]
    pos = torch.arange(T)[None]
    cos, sin = rope(hs, pos)
    mask = torch.full((T, T), float("-inf"), dtype=torch.float64).triu(1)[None, None]
    with torch.no_grad():
        ref, _ = att(hs, (cos.double(), sin.double()), mask)
    empty = np.zeros((n_kv, T, 256), np.uint16)
    out, kn, vn = orc.attention_layer(x, A, 0, empty, empty)
    got = out - orc.bf16_to_f32(x).astype(np.float64)
    # transformers builds its rotary cos/sin tables in float32 (the oracle's angles are double):
    # agreement to ~3e-7 relative; a wrong convention (pairing, gate, norm, GQA map) is O(1)
    np.testing.assert_allclose(got, ref[0].numpy(), rtol=1e-6, atol=1e-6 * np.abs(got).max())
    assert np.abs(got).max() > 1e-2


def test_attention_cache_path_equals_full_sequence(orc):
    H, n_heads, n_kv, L, T = 512, 4, 2, 40, 3
    A = _attn_weights(orc, 62, H, n_heads, n_kv)
    x = orc.synth_bf16(62, 1, (L, H), 1.0)
    max_len = 64
    zero = np.zeros((n_kv, max_len, 256), np.uint16)
    full, kn, vn = orc.attention_layer(x, A, 0, zero, zero)
    # a cache holding the first L-T positions (the exact k and v, which are bf16-exact here only
    # up to rounding, so compare against a full run that sees the same rounded prefix)
    kc = zero.copy()
    vc = zero.copy()
    kc[:, :L - T] = orc.f32_to_bf16(kn[:L - T].transpose(1, 0, 2).astype(np.float32))
    vc[:, :L - T] = orc.f32_to_bf16(vn[:L - T].transpose(1, 0, 2).astype(np.float32))
    tail, _, _ = orc.attention_layer(x[L - T:], A, L - T, kc, vc)
    np.testing.assert_allclose(tail, full[L - T:], rtol=2e-2, atol=2e-2 * np.abs(full).max())
    # causality: the first rows do not see later tokens
    head, _, _ = orc.attention_layer(x[:5], A, 0, zero, zero)
    np.testing.assert_allclose(head, full[:5], rtol=1e-12, atol=1e-12)
