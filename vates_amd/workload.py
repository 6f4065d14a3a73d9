"""Synthetic Qwen3-Next-shaped MoE layers resident in HBM.

A layer holds an 8-bit router [E, H], a pool of ``cap`` 4-bit SwiGLU experts
(gate/up [cap, I, H], down [cap, H, I]), a 4-bit shared expert, an 8-bit
shared-expert gate [1, H], an expert->slot table (a seeded permutation when
cap == E, as the resident pool's table in resident_pool.py:549-580) and an
optional per-expert router logit bias ``alpha * log z(e)`` where z is a
Zipf(s) pmf over a seeded expert ranking, which skews routing the way real
expert popularity does.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from .moe import MoELayer, QuantizedProj
from .synth import synth_proj

# stream ids of one layer's tensors: layer * 16 + index
_ROUTER, _GATE, _UP, _DOWN, _SH_GATE, _SH_UP, _SH_DOWN, _SGATE = range(8)


@dataclass
class LayerWeights:
    router: QuantizedProj
    gate: QuantizedProj
    up: QuantizedProj
    down: QuantizedProj
    sh_gate: QuantizedProj
    sh_up: QuantizedProj
    sh_down: QuantizedProj
    sgate: QuantizedProj
    table: Optional[torch.Tensor]
    bias: Optional[torch.Tensor]
    norm: Optional[torch.Tensor]
    hidden: int
    inter: int
    num_experts: int
    router_bits: int
    sgate_bits: int


def zipf_bias(seed: int, layer: int, num_experts: int, s: float, alpha: float) -> np.ndarray:
    """alpha * log z(e), z = Zipf(s) pmf over a seeded ranking of the experts."""
    rng = np.random.default_rng([seed, layer, 0x21BF])
    rank = rng.permutation(num_experts)
    z = 1.0 / np.arange(1, num_experts + 1, dtype=np.float64) ** s
    z /= z.sum()
    bias = np.empty(num_experts, dtype=np.float32)
    bias[rank] = (alpha * np.log(z)).astype(np.float32)
    return bias


def norm_weight(seed: int, layer: int, hidden: int) -> np.ndarray:
    """RMSNorm weight as bf16 bit patterns: 1 + N(0, 0.1^2), rounded to nearest even."""
    rng = np.random.default_rng([seed, layer, 0x4E0A])
    w = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    u = w.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def slot_permutation(seed: int, layer: int, num_experts: int) -> np.ndarray:
    rng = np.random.default_rng([seed, layer, 0x5107])
    return rng.permutation(num_experts).astype(np.int32)


def synth_layer(seed: int, layer: int, *, hidden: int = 2048, inter: int = 512, num_experts: int = 512,
                cap: Optional[int] = None, router_bits: int = 8, sgate_bits: int = 8, std: float = 0.02,
                zipf_s: float = 1.1, zipf_alpha: float = 0.0, permute_slots: bool = True, with_norm: bool = True,
                device=None) -> LayerWeights:
    cap = num_experts if cap is None else cap
    device = torch.device(device or "cuda")
    base = layer * 16
    mk = lambda idx, n, o, i, bits=4: synth_proj(seed, base + idx, n, o, i, bits=bits, std=std, device=device)
    router = mk(_ROUTER, 1, num_experts, hidden, router_bits)
    gate = mk(_GATE, cap, inter, hidden)
    up = mk(_UP, cap, inter, hidden)
    down = mk(_DOWN, cap, hidden, inter)
    sh_gate = mk(_SH_GATE, 1, inter, hidden)
    sh_up = mk(_SH_UP, 1, inter, hidden)
    sh_down = mk(_SH_DOWN, 1, hidden, inter)
    sgate = mk(_SGATE, 1, 1, hidden, sgate_bits)
    table = None
    if permute_slots and cap == num_experts:
        table = torch.from_numpy(slot_permutation(seed, layer, num_experts)).to(device)
    elif cap != num_experts:
        table = torch.from_numpy((np.arange(num_experts) % cap).astype(np.int32)).to(device)
    bias = None
    if zipf_alpha:
        bias = torch.from_numpy(zipf_bias(seed, layer, num_experts, zipf_s, zipf_alpha)).to(device)
    norm = None
    if with_norm:
        norm = torch.from_numpy(norm_weight(seed, layer, hidden).view(np.int16)).to(device).view(torch.bfloat16)
    return LayerWeights(router, gate, up, down, sh_gate, sh_up, sh_down, sgate, table, bias, norm, hidden, inter,
                        num_experts, router_bits, sgate_bits)


def make_layer(w: LayerWeights, top_k: int = 10, norm_topk_prob: bool = True) -> MoELayer:
    return MoELayer(w.router, w.gate, w.up, w.down, top_k=top_k, norm_topk_prob=norm_topk_prob,
                    router_bits=w.router_bits, shared_gate=w.sh_gate, shared_up=w.sh_up, shared_down=w.sh_down,
                    shared_expert_gate=w.sgate, shared_expert_gate_bits=w.sgate_bits, slot_table=w.table,
                    router_logit_bias=w.bias, norm_weight=w.norm)


def bf16_norm(seed: int, layer: int, n: int, device) -> torch.Tensor:
    return torch.from_numpy(norm_weight(seed, layer, n).view(np.int16)).to(device).view(torch.bfloat16)


def synth_attention(seed: int, layer: int, *, hidden: int = 2048, n_heads: int = 16, n_kv_heads: int = 2,
                    std: float = 0.02, device=None):
    """Qwen3-Next full-attention block: 4-bit q|gate, k, v, o projections, bf16 norms."""
    from .attention import AttentionLayer
    device = torch.device(device or "cuda")
    base = layer * 16 + 8
    q = synth_proj(seed, base, 1, n_heads * 512, hidden, std=std, device=device)
    k = synth_proj(seed, base + 1, 1, n_kv_heads * 256, hidden, std=std, device=device)
    v = synth_proj(seed, base + 2, 1, n_kv_heads * 256, hidden, std=std, device=device)
    o = synth_proj(seed, base + 3, 1, hidden, n_heads * 256, std=std, device=device)
    return AttentionLayer(q, k, v, o, bf16_norm(seed, 1000 + layer, hidden, device),
                          bf16_norm(seed, 2000 + layer, 256, device), bf16_norm(seed, 3000 + layer, 256, device),
                          n_heads=n_heads, n_kv_heads=n_kv_heads)


def synth_gdn(seed: int, layer: int, *, hidden: int = 2048, n_k_heads: int = 16, n_v_heads: int = 32,
              std: float = 0.02, device=None):
    """Qwen3-Next Gated DeltaNet block: 4-bit qkvz, ba and out projections,
    bf16 conv weights [conv_dim, 4] (std 0.3), A_log = log U(1, 16),
    dt_bias ~ N(0, 1), bf16 norms."""
    from .gdn import GatedDeltaNetLayer
    from .synth import synth_bf16
    device = torch.device(device or "cuda")
    base = layer * 16 + 12
    r = n_v_heads // n_k_heads
    qkvz = synth_proj(seed, base, 1, n_k_heads * (256 + 256 * r), hidden, std=std, device=device)
    ba = synth_proj(seed, base + 1, 1, 2 * n_v_heads, hidden, std=std, device=device)
    out = synth_proj(seed, base + 2, 1, hidden, n_v_heads * 128, std=std, device=device)
    conv_dim = 2 * n_k_heads * 128 + n_v_heads * 128
    conv = synth_bf16(seed, 0xC0000 + layer, (conv_dim, 4), std=0.3, device=device)
    rng = np.random.default_rng([seed, layer, 0x6D17])
    A_log = torch.from_numpy(np.log(rng.uniform(1.0, 16.0, n_v_heads)).astype(np.float32)).to(device)
    dt_bias = torch.from_numpy(rng.standard_normal(n_v_heads).astype(np.float32)).to(device)
    return GatedDeltaNetLayer(qkvz, ba, out, bf16_norm(seed, 5000 + layer, hidden, device), conv, A_log, dt_bias,
                              bf16_norm(seed, 6000 + layer, 128, device), n_k_heads=n_k_heads, n_v_heads=n_v_heads)


def synth_spec_model(seed: int, *, n_layers: int = 4, attn_every: int = 4, hidden: int = 2048, inter: int = 512,
                     num_experts: int = 512, top_k: int = 10, vocab: int = 151936, n_heads: int = 16,
                     n_kv_heads: int = 2, zipf_alpha: float = 0.5, linear_attention: bool = True,
                     n_k_heads: int = 16, n_v_heads: int = 32, device=None):
    """A random-init Qwen3-Next-shaped model for speculative decoding: bf16
    embedding and head [vocab, hidden], n_layers decoder layers (a full-attention
    block on every attn_every-th layer, as layer_types' interval pattern, a
    Gated DeltaNet block on the others unless linear_attention is False, then
    the routed MoE with the shared expert), the final norm, and the MTP layer
    (layer id 100: fc [hidden, 2 hidden], attention, MoE, norms)."""
    from .decode import DecoderLayer, SpecModel
    from .mtp import MTPLayer, MTPWeights
    from .synth import synth_bf16
    device = torch.device(device or "cuda")
    embed = synth_bf16(seed, 0xE0000, (vocab, hidden), std=1.0, device=device)
    head = synth_bf16(seed, 0xE0001, (vocab, hidden), std=0.02, device=device)
    layers = []
    for l in range(n_layers):
        w = synth_layer(seed, l, hidden=hidden, inter=inter, num_experts=num_experts, zipf_alpha=zipf_alpha,
                        device=device)
        full = (l + 1) % attn_every == 0
        attn = synth_attention(seed, l, hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv_heads, device=device) \
            if full else None
        gdn = synth_gdn(seed, l, hidden=hidden, n_k_heads=n_k_heads, n_v_heads=n_v_heads, device=device) \
            if linear_attention and not full else None
        layers.append(DecoderLayer(make_layer(w, top_k=top_k), attn, gdn))
    mw = synth_layer(seed, 100, hidden=hidden, inter=inter, num_experts=num_experts, zipf_alpha=zipf_alpha,
                     device=device)
    mtp = MTPLayer(MTPWeights(
        embed=embed, norm_emb=bf16_norm(seed, 4000, hidden, device), norm_hid=bf16_norm(seed, 4001, hidden, device),
        fc=synth_proj(seed, 100 * 16 + 15, 1, hidden, 2 * hidden, device=device),
        attn=synth_attention(seed, 100, hidden=hidden, n_heads=n_heads, n_kv_heads=n_kv_heads, device=device),
        moe=make_layer(mw, top_k=top_k), norm=bf16_norm(seed, 4002, hidden, device), lm_head=head))
    return SpecModel(embed, layers, bf16_norm(seed, 4003, hidden, device), head, mtp)
