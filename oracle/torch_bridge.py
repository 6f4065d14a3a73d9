"""Copies GPU-resident weights (torch tensors) into the numpy layout the
oracle takes.  TEST INFRASTRUCTURE ONLY (tests/, smoke(), bench cpu_baseline)."""
from __future__ import annotations

import numpy as np


def u32(t) -> np.ndarray:
    """Bit pattern of a 4-byte tensor as uint32."""
    import torch
    return t.detach().view(torch.int32).cpu().numpy().view(np.uint32)


def u16(t) -> np.ndarray:
    """Bit pattern of a 2-byte tensor (int16 / bf16) as uint16."""
    import torch
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def pool_np(gate, up, down) -> dict:
    return {"gate_w": u32(gate.weight), "gate_s": u16(gate.scales), "gate_b": u16(gate.biases),
            "up_w": u32(up.weight), "up_s": u16(up.scales), "up_b": u16(up.biases),
            "down_w": u32(down.weight), "down_s": u16(down.scales), "down_b": u16(down.biases)}


def layer_np(w, top_k: int, norm: bool = True) -> dict:
    """vates_amd.workload.LayerWeights -> oracle.moe_layer's dict."""
    L = {"H": w.hidden, "I": w.inter, "E": w.num_experts, "k": top_k, "group": 64, "norm": int(norm),
         "router_bits": w.router_bits, "bits": 4, "cap": w.gate.weight.shape[0], "sg_bits": w.sgate_bits}
    L["router_w"], L["router_s"], L["router_b"] = u32(w.router.weight), u16(w.router.scales), u16(w.router.biases)
    L.update(pool_np(w.gate, w.up, w.down))
    for key, v in pool_np(w.sh_gate, w.sh_up, w.sh_down).items():
        L["sh_" + key] = v
    L["sg_w"], L["sg_s"], L["sg_b"] = u32(w.sgate.weight), u16(w.sgate.scales), u16(w.sgate.biases)
    L["table"] = None if w.table is None else w.table.cpu().numpy()
    L["bias"] = None if w.bias is None else w.bias.cpu().numpy()
    L["norm_w"] = None if w.norm is None else u16(w.norm)
    L["norm_eps"] = 1e-6
    return L
