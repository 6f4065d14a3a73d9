"""ctypes binding of libvmi.so (declared in include/vmi.h).

The library is the only compute path: if it is missing or fails to load,
every entry point raises VmiError.  There is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libvmi.so"

VMI_OK = 0
VMI_ERR_INVALID = -1
VMI_ERR_UNSUPPORTED = -2
VMI_ERR_HIP = -3
VMI_ERR_WORKSPACE = -4
VMI_F32 = 0
VMI_BF16 = 1
VMI_STATUS_BAD_SLOT = 0x1
VMI_STATUS_BAD_ROUTE = 0x2
VMI_STATUS_BAD_POS = 0x4
VMI_STATUS_BAD_RECORD = 0x8
VMI_STATUS_WAIT_GAVE_UP = 0x10
VMI_STATUS_BAD_LOGITS = 0x20


class VmiError(RuntimeError):
    """Raised for any non-zero libvmi status or a missing library."""

    def __init__(self, msg: str, code: int = VMI_ERR_INVALID):
        super().__init__(msg)
        self.code = code


class QMat(ctypes.Structure):
    _fields_ = [("w", c_void_p), ("s", c_void_p), ("b", c_void_p)]


VMI_TREE_ATTENTION = 1
VMI_TREE_GDN = 2


class TreeLayer(ctypes.Structure):
    """vmi_tree_layer: one layer's entry of vmi_tree_commit's table."""
    _fields_ = [("kind", c_int), ("n_kv_heads", c_int), ("max_len", c_int), ("n_k_heads", c_int),
                ("n_v_heads", c_int), ("n_slots", c_int), ("k_cache", c_void_p), ("v_cache", c_void_p),
                ("tree_kv", c_void_p), ("conv_ring", c_void_p), ("state_ring", c_void_p), ("tree_conv", c_void_p),
                ("tree_side", c_void_p)]


class MoeLayerDesc(ctypes.Structure):
    _fields_ = [
        ("hidden", c_int), ("inter", c_int), ("num_experts", c_int), ("top_k", c_int),
        ("group", c_int), ("bits", c_int), ("norm_topk_prob", c_int), ("router_bits", c_int),
        ("cap", c_int),
        ("router", QMat), ("router_logit_bias", c_void_p), ("slot_table", c_void_p),
        ("gate", QMat), ("up", QMat), ("down", QMat),
        ("shared_gate", QMat), ("shared_up", QMat), ("shared_down", QMat),
        ("shared_expert_gate", QMat), ("shared_expert_gate_bits", c_int),
        ("norm_weight", c_void_p), ("norm_eps", c_float), ("prefill_tables", c_void_p),
    ]


# name -> (restype, argtypes)
_SIGNATURES = {
    "vmi_last_error": (c_char_p, []),
    "vmi_version": (c_int, []),
    "vmi_fused_moe_slots_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "vmi_fused_moe_slots": (c_int, [c_void_p, c_int, c_void_p, c_void_p, QMat, QMat, QMat, c_int, c_int, c_int,
                                    c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "vmi_fused_moe_staged": (c_int, [c_void_p, c_int, c_void_p, QMat, QMat, QMat, c_int, c_int, c_int, c_int, c_int,
                                     c_int, c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "vmi_moe_layer_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "vmi_moe_layer": (c_int, [POINTER(MoeLayerDesc), c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_void_p, c_size_t, c_void_p]),
    "vmi_moe_layer_noalloc": (c_int, [POINTER(MoeLayerDesc), c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p]),
    "vmi_moe_prefill_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "vmi_moe_prefill": (c_int, [POINTER(MoeLayerDesc), c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_size_t, c_void_p]),
    "vmi_moe_prefill_tables_bytes": (c_size_t, [c_int, c_int, c_int]),
    "vmi_moe_prefill_tables": (c_int, [POINTER(MoeLayerDesc), c_void_p, c_size_t, c_void_p]),
    "vmi_workspace_status": (c_int, [c_void_p, c_void_p, POINTER(c_uint32)]),
    "vmi_dequant_affine": (c_int, [QMat, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "vmi_synth_quantized": (c_int, [c_uint64, c_uint32, c_int64, c_int, c_int, c_int, c_float, c_void_p, c_void_p,
                                    c_void_p, c_void_p]),
    "vmi_synth_bf16": (c_int, [c_uint64, c_uint32, c_int64, c_float, c_void_p, c_void_p]),
    "vmi_accept_greedy": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
    "vmi_spec_commit": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_void_p]),
    "vmi_accept_stochastic_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "vmi_accept_stochastic": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_float, c_float, c_uint64,
                                      c_uint64, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p, c_void_p]),
    "vmi_sample_top_p_workspace_bytes": (c_size_t, [c_int, c_int]),
    "vmi_sample_top_p": (c_int, [c_void_p, c_int, c_int, c_float, c_float, c_uint64, c_uint64, c_void_p, c_void_p,
                                 c_void_p, c_size_t, c_void_p, c_void_p]),
    "vmi_set_wait_limit": (c_int, [c_int]),
    "vmi_qgemv": (c_int, [c_void_p, c_int, c_int, QMat, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p,
                          c_void_p]),
    "vmi_attention_layer_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "vmi_attention_layer": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                    c_void_p, c_size_t, c_void_p]),
    "vmi_attention_tree_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "vmi_attention_tree": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int,
                                   c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "vmi_gdn_tree": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                             c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "vmi_tree_commit": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "vmi_gdn_layer_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "vmi_gdn_layer": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                              c_void_p, c_size_t, c_void_p]),
    "vmi_rmsnorm": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_void_p, c_float, c_void_p, c_int, c_void_p,
                            c_void_p]),
    "vmi_topk_rows": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "vmi_stream_read": (c_int, [c_void_p, c_size_t, c_int, c_int, c_void_p, c_void_p]),
    "vmi_mfma_peak": (c_int, [c_int, c_int, c_void_p, c_void_p]),
    "vmi_lm_head_workspace_bytes": (c_size_t, [c_int, c_int]),
    "vmi_lm_head": (c_int, [c_void_p, c_int, c_int, c_void_p, c_float, c_void_p, c_int, c_void_p, c_void_p,
                            c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "vmi_head_tiles_bytes": (c_size_t, [c_int, c_int]),
    "vmi_head_tiles": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "vmi_lm_head_tiled": (c_int, [c_void_p, c_int, c_int, c_void_p, c_float, c_void_p, c_int, c_void_p, c_void_p,
                                  c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Loads libvmi.so once; raises VmiError when it is absent or incomplete."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise VmiError(f"{LIB_PATH} is not built; run `python -m vates_amd.build` (hipcc, gfx950)",
                       VMI_ERR_UNSUPPORTED)
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        raise VmiError(f"cannot load {LIB_PATH}: {exc}", VMI_ERR_UNSUPPORTED) from exc
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != VMI_OK:
        msg = load().vmi_last_error().decode(errors="replace")
        raise VmiError(f"{what}: {msg} (status {rc})", rc)


def exported_names() -> list[str]:
    return list(_SIGNATURES)
