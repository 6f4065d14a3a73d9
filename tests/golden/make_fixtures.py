"""Writes the golden fixtures under tests/golden/.

reference_known_answers.json holds the literal inputs and expected outputs
that the reference's own tests state (paths relative to the AMOS144/Vates
checkout); nothing here runs reference code.  oracle_small.npz holds small
oracle outputs on seeded inputs so that later changes to the oracle are caught.

Run:  python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import json
import sys
from fractions import Fraction
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))


def reference_known_answers() -> dict:
    out = {}
    # mlx_streaming/tests/test_mtp_generate.py:211-223
    out["accept_prefix"] = [
        {"drafts": [11, 22, 33], "preds": [11, 22, 99], "matched": 2},
        {"drafts": [11, 22, 33], "preds": [99, 22, 33], "matched": 0},
        {"drafts": [11, 22, 33], "preds": [11, 22, 33], "matched": 3},
    ]
    # mlx_streaming/tests/test_expert_major_prefill.py:89-103
    out["route_reduce"] = {
        "previous": [[1.0, -1.0], [2.0, -2.0]],
        "assignment_pos": [3, 0, 2],
        "weighted": [[30.0, 300.0], [10.0, 100.0], [20.0, 200.0]],
        "routes_per_token": 2,
        "expected": [[11.0, 99.0], [52.0, 498.0]],
    }
    # mlx_streaming/tests/test_expert_major_prefill.py:33-86: toy experts
    # y_e(x) = x + (e + 1), capacity 2 -> group loads [(0, 1), (2, 3)].
    x = [[1, 2], [3, 4], [5, 6]]
    inds = [[0, 3], [1, 0], [3, 2]]
    scores = [["1/4", "3/4"], ["3/5", "2/5"], ["1/10", "9/10"]]
    expected = []
    for xt, it, st in zip(x, inds, scores):
        expected.append([float(sum((Fraction(v) + e + 1) * Fraction(s) for e, s in zip(it, st))) for v in xt])
    out["expert_major_toy"] = {
        "x": x, "inds": inds, "scores": [[float(Fraction(s)) for s in row] for row in scores],
        "num_experts": 4, "layer_cap": 2, "expected": expected, "group_loads": [[0, 1], [2, 3]],
    }
    # mlx_streaming/tests/test_mtp_generate.py:575-606
    out["commit_kv_trim"] = {"tokens": 5, "verified_len": 5, "accepted_len": 3, "offset_after": 3}
    out["commit_checkpoint"] = {
        "verified_len": 3, "accepted_len": 2,
        "checkpoints": [[1.0, 10.0], [2.0, 20.0], [3.0, 30.0]],
        "shapes": [[1, 3, 4], [1, 2, 2]],
        "sums_after": [24.0, 80.0],
    }
    # mlx_streaming/tests/test_native_moe_ext.py:50-72 (slot pool, cap 4)
    out["slot_pool"] = {"cap": 4, "calls": [[1, 2, 1], [2, 1]], "local": [[0, 1, 0], [1, 0]], "rebuilds_after": [1, 1]}
    # Random123 known-answer vectors for Philox4x32-10 (kat_vectors)
    out["philox4x32_10"] = [
        {"ctr": [0, 0, 0, 0], "key": [0, 0], "out": [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]},
        {"ctr": [0xFFFFFFFF] * 4, "key": [0xFFFFFFFF] * 2, "out": [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]},
        {"ctr": [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], "key": [0xA4093822, 0x299F31D0],
         "out": [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]},
    ]
    # Nibble order of the packed format (fused_moe.cpp:131-145, LSB first).
    out["dequant_words"] = [
        {"word": 0x76543210, "bits": 4, "q": [0, 1, 2, 3, 4, 5, 6, 7]},
        {"word": 0xFEDCBA98, "bits": 4, "q": [8, 9, 10, 11, 12, 13, 14, 15]},
        {"word": 0x04030201, "bits": 8, "q": [1, 2, 3, 4]},
        {"word": 0xFF80017F, "bits": 8, "q": [127, 1, 128, 255]},
    ]
    return out


def oracle_small() -> dict:
    """A small full MoE layer (hidden 512, inter 128, 64 experts, top-4, T=3)."""
    from oracle import oracle as o
    H, I, E, k, T = 512, 128, 64, 4, 3
    L = {"H": H, "I": I, "E": E, "k": k, "group": 64, "norm": 1, "router_bits": 8, "bits": 4, "cap": E,
         "bias": None, "table": None, "sg_bits": 8}
    L["router_w"], L["router_s"], L["router_b"] = o.synth_quantized(7, 1, E, H, bits=8)
    L["gate_w"], L["gate_s"], L["gate_b"] = o.synth_quantized(7, 2, E * I, H)
    L["up_w"], L["up_s"], L["up_b"] = o.synth_quantized(7, 3, E * I, H)
    L["down_w"], L["down_s"], L["down_b"] = o.synth_quantized(7, 4, E * H, I)
    L["sh_gate_w"], L["sh_gate_s"], L["sh_gate_b"] = o.synth_quantized(7, 5, I, H)
    L["sh_up_w"], L["sh_up_s"], L["sh_up_b"] = o.synth_quantized(7, 6, I, H)
    L["sh_down_w"], L["sh_down_s"], L["sh_down_b"] = o.synth_quantized(7, 7, H, I)
    L["sg_w"], L["sg_s"], L["sg_b"] = o.synth_quantized(7, 8, 1, H, bits=8)
    x = o.synth_bf16(7, 9, (T, H), 1.0)
    out_f32, out_bf16, ids, sc, sl = o.moe_layer(x, L)
    return {"x": x, "out_f32": out_f32, "out_bf16": out_bf16, "ids": ids, "scores": sc,
            "router_w_sum": np.array([int(L["router_w"].astype(np.uint64).sum())], dtype=np.uint64),
            "gate_w_sum": np.array([int(L["gate_w"].astype(np.uint64).sum())], dtype=np.uint64)}


def main() -> None:
    (HERE / "reference_known_answers.json").write_text(json.dumps(reference_known_answers(), indent=1) + "\n")
    np.savez(HERE / "oracle_small.npz", **oracle_small())
    print("wrote", HERE / "reference_known_answers.json", HERE / "oracle_small.npz")


if __name__ == "__main__":
    main()
