"""vates_amd: MI355X-native speculative-decode MoE hot path (HIP kernels behind a C ABI).

Public surface:
  fused_moe_slots   -- mirror of the reference native_moe_ext.fused_moe_slots
  fused_moe_staged  -- mirror of native_moe_ext.fused_moe_staged (pre-sliced weights)
  MoELayer          -- routed MoE layer (router, top-k, experts, shared expert)
  QuantizedProj     -- one affine-quantised projection stack
"""
from ._lib import VmiError, LIB_PATH
from .moe import MoELayer, QuantizedProj, fused_moe_slots, fused_moe_staged, workspace_status

__all__ = ["VmiError", "LIB_PATH", "MoELayer", "QuantizedProj", "fused_moe_slots", "fused_moe_staged",
           "workspace_status"]
