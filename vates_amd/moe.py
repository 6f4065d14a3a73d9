"""Host mirror of the reference's fused-MoE operator surface on libvmi.

* ``fused_moe_slots`` keeps the argument list of the reference binding
  ``native_moe_ext.fused_moe_slots`` (native/ext/bindings.cpp:300-320;
  native/ext/compute/fused_moe.h:18-23) and its output contract
  (f32, shape ``x.shape[:-1] + [hidden]``, fused_moe.cpp:653-656).
* ``MoELayer`` is the analogue of ``FileStreamingMoeBlock.__call__``
  (mlx_streaming/core/moe/block.py:245-1013, production branch): router,
  softmax/top-k/renorm, expert->slot table, SwiGLU experts, weighted combine
  and the sigmoid-gated shared expert, in three HIP kernels.

Tensors live on the current HIP device (torch "cuda" device on ROCm).  Every
call is asynchronous on ``torch.cuda.current_stream()`` unless a stream is
given.  Errors raise ``VmiError``; there is no fallback path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import QMat, MoeLayerDesc, VmiError, check, load

_WORKSPACES: dict = {}


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream_handle(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _require(t: torch.Tensor, name: str, elem: int, device: torch.device) -> None:
    if not isinstance(t, torch.Tensor):
        raise VmiError(f"{name} must be a torch.Tensor")
    if t.device != device:
        raise VmiError(f"{name} is on {t.device}, expected {device}")
    if not t.is_contiguous():
        raise VmiError(f"{name} must be contiguous")
    if t.element_size() != elem:
        raise VmiError(f"{name} must have {elem}-byte elements (got {t.dtype})")


def workspace(nbytes: int, device: torch.device, stream_handle: int, tag: str = "moe") -> torch.Tensor:
    """Workspace cached per (device, stream, tag).  It starts zero-filled so
    the device status word and arrival counters read 0; calls on one stream are
    serialised, so reuse across them is safe.  Entry points whose workspaces
    keep state between calls (status word, counters) use distinct tags."""
    key = (device.index, stream_handle, tag)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


@dataclass
class QuantizedProj:
    """One affine-quantised projection stack: weight uint32-bits
    [n, out, in*bits/32], scales/biases bf16-bits [n, out, in/group]."""

    weight: torch.Tensor
    scales: torch.Tensor
    biases: torch.Tensor

    def qmat(self) -> QMat:
        return QMat(self.weight.data_ptr(), self.scales.data_ptr(), self.biases.data_ptr())

    def check(self, name: str, device: torch.device) -> None:
        _require(self.weight, f"{name}.weight", 4, device)
        _require(self.scales, f"{name}.scales", 2, device)
        _require(self.biases, f"{name}.biases", 2, device)


def down_group_major(p: QuantizedProj, group: int = 64, bits: int = 4) -> QuantizedProj:
    """A down-projection stack [n, hidden, inter*bits/32] (the reference's pool
    layout) re-laid group-major for ``MoELayer``: words [n, inter/group, hidden,
    group*bits/32], scales and biases [n, inter/group, hidden].  Quantisation
    group g of row h is then contiguous with group g of rows h+1, h+2, ...:
    the verify kernel projects one group's activations through that strip,
    and the prefill kernel streams the strip of each group in turn."""
    n, rows, words = p.weight.shape
    wpg = group * bits // 32
    G = words // wpg
    if G * wpg != words or tuple(p.scales.shape) != (n, rows, G) or tuple(p.biases.shape) != (n, rows, G):
        raise VmiError(f"down stack shapes {tuple(p.weight.shape)}/{tuple(p.scales.shape)} do not match group={group}")
    w = p.weight.view(n, rows, G, wpg).permute(0, 2, 1, 3).contiguous()
    s = p.scales.permute(0, 2, 1).contiguous()
    b = p.biases.permute(0, 2, 1).contiguous()
    return QuantizedProj(w, s, b)


def gateup_mfma_major(p: QuantizedProj, group: int = 64, bits: int = 4) -> QuantizedProj:
    """A gate or up stack [n, inter, hidden*bits/32] re-laid in the operand
    order of the verify kernel's MFMAs: words [n, inter/64, 4, hidden/128, 64,
    4], where block (c, w, m) holds, for lane l = 16 q + r, the 16 bytes at
    byte 64 m + 16 q of row 64 c + 16 w + r.  One wave's load of a block is
    then 1 KB of contiguous memory, and a 64-row slice of the intermediate
    dimension is one contiguous run.  Scales and biases keep their layout."""
    if bits != 4 or group != 64:
        raise VmiError(f"the MFMA-major layout is built for bits=4 group=64 (got {bits}, {group})")
    n, rows, words = p.weight.shape
    if rows % 64 or words % 16:
        raise VmiError(f"gate/up stack shape {tuple(p.weight.shape)} needs inter % 64 == 0 and hidden % 128 == 0")
    w = p.weight.view(n, rows // 64, 4, 16, words // 16, 4, 4).permute(0, 1, 2, 4, 5, 3, 6).contiguous()
    return QuantizedProj(w.view(n, rows, words), p.scales, p.biases)


def gateup_reference_layout(p: QuantizedProj) -> QuantizedProj:
    """Inverse of ``gateup_mfma_major``: the stack back in the reference's
    [n, inter, hidden*bits/32] row-major pool layout (a new tensor)."""
    n, rows, words = p.weight.shape
    w = p.weight.view(n, rows // 64, 4, words // 16, 4, 16, 4).permute(0, 1, 2, 5, 3, 4, 6).contiguous()
    return QuantizedProj(w.view(n, rows, words), p.scales, p.biases)


def down_reference_layout(p: QuantizedProj, group: int = 64, bits: int = 4) -> QuantizedProj:
    """Inverse of ``down_group_major``: words [n, hidden, inter*bits/32],
    scales and biases [n, hidden, inter/group] (new tensors)."""
    n, G, rows, wpg = p.weight.shape
    if wpg != group * bits // 32:
        raise VmiError(f"group-major down words {tuple(p.weight.shape)} do not match group={group}")
    w = p.weight.permute(0, 2, 1, 3).contiguous().view(n, rows, G * wpg)
    return QuantizedProj(w, p.scales.permute(0, 2, 1).contiguous(), p.biases.permute(0, 2, 1).contiguous())


def _fused_moe_pairs(x: torch.Tensor, local_slots: Optional[torch.Tensor], scores: torch.Tensor, k: int,
                     projs: list, hidden: int, inter: int, group: int, bits: int, stream,
                     out_dtype: torch.dtype) -> torch.Tensor:
    lib = load()
    device = x.device
    if x.shape[-1] != hidden:
        raise VmiError(f"x last dim {x.shape[-1]} != hidden {hidden}")
    T = x.numel() // hidden
    if scores.numel() != T * k or (local_slots is not None and local_slots.numel() != T * k):
        raise VmiError("shape mismatch: local_slots/scores must hold T*k entries")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise VmiError(f"x dtype {x.dtype} not supported (f32 or bf16)")
    _require(x, "x", x.element_size(), device)
    if local_slots is not None:
        _require(local_slots, "local_slots", 4, device)
    if scores.dtype != torch.float32:
        raise VmiError("scores must be float32")
    _require(scores, "scores", 4, device)
    for name, p in zip(("gate", "up", "down"), projs):
        p.check(name, device)
    cap = projs[0].weight.shape[0]
    if local_slots is None and cap < T * k:
        raise VmiError(f"staged stacks hold {cap} matrices, the batch needs T*k = {T * k}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise VmiError("out_dtype must be float32 or bfloat16")
    out = torch.empty(tuple(x.shape[:-1]) + (hidden,), dtype=out_dtype, device=device)
    sh = _stream_handle(stream)
    nbytes = lib.vmi_fused_moe_slots_workspace_bytes(T, k, hidden, inter)
    ws = workspace(nbytes, device, sh)
    xdt = _lib.VMI_BF16 if x.dtype == torch.bfloat16 else _lib.VMI_F32
    odt = _lib.VMI_BF16 if out_dtype == torch.bfloat16 else _lib.VMI_F32
    if local_slots is not None:
        rc = lib.vmi_fused_moe_slots(x.data_ptr(), xdt, local_slots.data_ptr(), scores.data_ptr(),
                                     projs[0].qmat(), projs[1].qmat(), projs[2].qmat(),
                                     T, k, hidden, inter, group, bits, cap, out.data_ptr(), odt,
                                     ws.data_ptr(), ws.numel(), sh)
        check(rc, "vmi_fused_moe_slots")
    else:
        rc = lib.vmi_fused_moe_staged(x.data_ptr(), xdt, scores.data_ptr(),
                                      projs[0].qmat(), projs[1].qmat(), projs[2].qmat(),
                                      T, k, hidden, inter, group, bits, out.data_ptr(), odt,
                                      ws.data_ptr(), ws.numel(), sh)
        check(rc, "vmi_fused_moe_staged")
    return out


def fused_moe_slots(x: torch.Tensor, local_slots: torch.Tensor, scores: torch.Tensor,
                    gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b,
                    hidden: int, inter: int, group: int, bits: int, *, stream=None,
                    out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Fused slot-indexed 4-bit MoE (reference: fused_moe_slots).

    x [..., hidden] f32 or bf16; local_slots [..., k] int32/uint32 (flattened
    token-major, token = pair // k); scores same shape as local_slots, f32;
    pool arrays [cap, out, in*bits/32] / [cap, out, in/group].  Returns
    sum_j scores[..., j] * SwiGLU_expert_{slot}(x) as ``out_dtype``.
    """
    k = local_slots.shape[-1] if local_slots.dim() > 0 else 1
    projs = [QuantizedProj(gate_w, gate_s, gate_b), QuantizedProj(up_w, up_s, up_b),
             QuantizedProj(down_w, down_s, down_b)]
    return _fused_moe_pairs(x, local_slots, scores, k, projs, hidden, inter, group, bits, stream, out_dtype)


def fused_moe_staged(x: torch.Tensor, scores: torch.Tensor,
                     gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b,
                     hidden: int, inter: int, group: int, bits: int, *, stream=None,
                     out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Fused 4-bit MoE over pre-sliced weights (reference: fused_moe_staged,
    fused_moe.cpp:443-504, 605-633): scores [..., k] f32; the stacks hold one
    matrix per (token, rank) pair, pair t*k + j reading matrix t*k + j."""
    k = scores.shape[-1] if scores.dim() > 0 else 1
    projs = [QuantizedProj(gate_w, gate_s, gate_b), QuantizedProj(up_w, up_s, up_b),
             QuantizedProj(down_w, down_s, down_b)]
    return _fused_moe_pairs(x, None, scores, k, projs, hidden, inter, group, bits, stream, out_dtype)


def workspace_status(ws: torch.Tensor, stream=None) -> int:
    """Reads and clears the device status word (synchronises the stream)."""
    flags = ctypes.c_uint32(0)
    check(load().vmi_workspace_status(ws.data_ptr(), _stream_handle(stream), ctypes.byref(flags)),
          "vmi_workspace_status")
    return flags.value


class MoELayer:
    """One routed MoE layer with a sigmoid-gated shared expert on a verify batch.

    Analogue of FileStreamingMoeBlock.__call__ (block.py:245-1013) with every
    expert resident in an HBM pool addressed through ``slot_table``
    (resident_pool.py:549-580): pool stacks hold ``cap`` experts, the table
    maps each of ``num_experts`` router outputs to its slot.  With
    ``norm_weight`` the layer applies the decoder's pre-MoE RMSNorm to its
    input first (the residual passed to ``__call__`` is added unnormalised).

    The stacks are given in the reference's pool layout; the layer keeps its
    own copies in the layouts its kernels read: gate and up in MFMA operand
    order (``gateup_mfma_major``), down group-major (``down_group_major``).
    """

    def __init__(self, router: QuantizedProj, gate: QuantizedProj, up: QuantizedProj, down: QuantizedProj, *,
                 top_k: int, norm_topk_prob: bool = True, group: int = 64, bits: int = 4, router_bits: int = 8,
                 shared_gate: Optional[QuantizedProj] = None, shared_up: Optional[QuantizedProj] = None,
                 shared_down: Optional[QuantizedProj] = None, shared_expert_gate: Optional[QuantizedProj] = None,
                 shared_expert_gate_bits: int = 8, slot_table: Optional[torch.Tensor] = None,
                 router_logit_bias: Optional[torch.Tensor] = None, norm_weight: Optional[torch.Tensor] = None,
                 norm_eps: float = 1e-6):
        device = gate.weight.device
        self.device = device
        self.num_experts = router.weight.shape[-2]
        self.hidden = router.scales.shape[-1] * group
        self.inter = gate.weight.shape[-2]
        self.cap = gate.weight.shape[0]
        for name, p in (("router", router), ("gate", gate), ("up", up), ("down", down)):
            p.check(name, device)
        has_shared = shared_gate is not None
        if has_shared:
            for name, p in (("shared_gate", shared_gate), ("shared_up", shared_up), ("shared_down", shared_down)):
                if p is None:
                    raise VmiError(f"{name} missing")
                p.check(name, device)
        if shared_expert_gate is not None:
            shared_expert_gate.check("shared_expert_gate", device)
        if slot_table is not None:
            if slot_table.dtype != torch.int32 or slot_table.numel() != self.num_experts:
                raise VmiError("slot_table must be int32 [num_experts]")
            _require(slot_table, "slot_table", 4, device)
        if router_logit_bias is not None:
            if router_logit_bias.dtype != torch.float32 or router_logit_bias.numel() != self.num_experts:
                raise VmiError("router_logit_bias must be float32 [num_experts]")
            _require(router_logit_bias, "router_logit_bias", 4, device)
        if norm_weight is not None:
            if norm_weight.dtype != torch.bfloat16 or norm_weight.numel() != self.hidden:
                raise VmiError("norm_weight must be bf16 [hidden]")
            _require(norm_weight, "norm_weight", 2, device)
        gate, up = gateup_mfma_major(gate, group, bits), gateup_mfma_major(up, group, bits)
        down = down_group_major(down, group, bits)
        if has_shared:
            shared_gate = gateup_mfma_major(shared_gate, group, bits)
            shared_up = gateup_mfma_major(shared_up, group, bits)
            shared_down = down_group_major(shared_down, group, bits)
        # keep every tensor alive: the descriptor stores raw pointers
        self._keep = (router, gate, up, down, shared_gate, shared_up, shared_down, shared_expert_gate, slot_table,
                      router_logit_bias, norm_weight)
        self.top_k = top_k
        null = QMat(None, None, None)
        d = MoeLayerDesc()
        d.hidden, d.inter, d.num_experts, d.top_k = self.hidden, self.inter, self.num_experts, top_k
        d.group, d.bits, d.norm_topk_prob, d.router_bits, d.cap = group, bits, int(norm_topk_prob), router_bits, self.cap
        d.router = router.qmat()
        d.router_logit_bias = _ptr(router_logit_bias)
        d.slot_table = _ptr(slot_table)
        d.gate, d.up, d.down = gate.qmat(), up.qmat(), down.qmat()
        d.shared_gate = shared_gate.qmat() if has_shared else null
        d.shared_up = shared_up.qmat() if has_shared else null
        d.shared_down = shared_down.qmat() if has_shared else null
        d.shared_expert_gate = shared_expert_gate.qmat() if shared_expert_gate is not None else null
        d.shared_expert_gate_bits = shared_expert_gate_bits
        d.norm_weight = _ptr(norm_weight)
        d.norm_eps = norm_eps
        self.desc = d
        self.group, self.bits = group, bits
        self._pf_tables: Optional[torch.Tensor] = None

    def prefill_tables(self, stream=None) -> torch.Tensor:
        """The fp16 dequantisation tables of the prefill's expert GEMMs for
        every pool slot (vmi_moe_prefill_tables), built on first use and kept
        with the layer: prefill() then reads them instead of building the
        touched experts' tables on every call.  The first call synchronises
        its stream, so it must not run under graph capture (call this method
        before capturing a prefill)."""
        if self._pf_tables is None:
            if torch.cuda.is_current_stream_capturing():
                raise VmiError("the prefill tables are built outside graph capture: call prefill_tables() first")
            lib = load()
            n = lib.vmi_moe_prefill_tables_bytes(self.hidden, self.inter, self.cap)
            t = torch.empty(n, dtype=torch.uint8, device=self.device)
            sh = _stream_handle(stream)
            check(lib.vmi_moe_prefill_tables(ctypes.byref(self.desc), t.data_ptr(), n, sh), "vmi_moe_prefill_tables")
            (stream if stream is not None else torch.cuda.current_stream()).synchronize()
            self._pf_tables = t
            self.desc.prefill_tables = t.data_ptr()
        return self._pf_tables

    def reference_weights(self) -> dict:
        """The layer's weights in the reference's layouts (new tensors for the
        six expert stacks, the stored tensors for the rest): keys router, gate,
        up, down, shared_gate, shared_up, shared_down, shared_expert_gate,
        slot_table, router_logit_bias, norm_weight."""
        names = ("router", "gate", "up", "down", "shared_gate", "shared_up", "shared_down", "shared_expert_gate",
                 "slot_table", "router_logit_bias", "norm_weight")
        out = dict(zip(names, self._keep))
        for key in ("gate", "up", "shared_gate", "shared_up"):
            if out[key] is not None:
                out[key] = gateup_reference_layout(out[key])
        for key in ("down", "shared_down"):
            if out[key] is not None:
                out[key] = down_reference_layout(out[key], self.group, self.bits)
        return out

    def workspace_bytes(self, T: int) -> int:
        return load().vmi_moe_layer_workspace_bytes(T, self.top_k, self.hidden, self.inter, self.num_experts)

    def prefill_workspace_bytes(self, T: int) -> int:
        return load().vmi_moe_prefill_workspace_bytes(T, self.top_k, self.hidden, self.inter, self.num_experts,
                                                      self.cap, self.desc.router_bits)

    def prefill(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None, *,
                out: Optional[torch.Tensor] = None, ids_out: Optional[torch.Tensor] = None,
                scores_out: Optional[torch.Tensor] = None, stream=None,
                ws: Optional[torch.Tensor] = None, use_tables: bool = True) -> torch.Tensor:
        """The layer on a long prompt, expert-major (block.py:111-243): x bf16 [T, hidden].
        use_tables=False builds the touched experts' dequantisation tables in
        the workspace for this call instead of reading the layer's own."""
        lib = load()
        if x.dtype != torch.bfloat16 or x.shape[-1] != self.hidden:
            raise VmiError("x must be bf16 [..., hidden]")
        _require(x, "x", 2, self.device)
        T = x.numel() // self.hidden
        if residual is not None:
            if residual.shape != x.shape or residual.dtype != torch.bfloat16:
                raise VmiError("residual must match x (bf16)")
            _require(residual, "residual", 2, self.device)
        if out is None:
            out = torch.empty_like(x)
        else:
            _require(out, "out", 2, self.device)
            if out.shape != x.shape or out.dtype != torch.bfloat16:
                raise VmiError("out must match x (bf16)")
        for name, t, dt in (("ids_out", ids_out, torch.int32), ("scores_out", scores_out, torch.float32)):
            if t is not None:
                if t.dtype != dt or t.numel() != T * self.top_k:
                    raise VmiError(f"{name} must be {dt} [T, top_k]")
                _require(t, name, 4, self.device)
        sh = _stream_handle(stream)
        if use_tables:
            self.prefill_tables(stream)
        if ws is None:
            ws = workspace(self.prefill_workspace_bytes(T), self.device, sh, tag="prefill")
        saved = self.desc.prefill_tables
        if not use_tables:
            self.desc.prefill_tables = None
        try:
            rc = lib.vmi_moe_prefill(ctypes.byref(self.desc), x.data_ptr(), T, _ptr(residual), out.data_ptr(),
                                     _ptr(ids_out), _ptr(scores_out), ws.data_ptr(), ws.numel(), sh)
        finally:
            self.desc.prefill_tables = saved
        check(rc, "vmi_moe_prefill")
        return out

    def __call__(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None, *, out: Optional[torch.Tensor] = None,
                 ids_out: Optional[torch.Tensor] = None, scores_out: Optional[torch.Tensor] = None,
                 stream=None, ws: Optional[torch.Tensor] = None) -> torch.Tensor:
        lib = load()
        if x.dtype != torch.bfloat16 or x.shape[-1] != self.hidden:
            raise VmiError("x must be bf16 [..., hidden]")
        _require(x, "x", 2, self.device)
        T = x.numel() // self.hidden
        if residual is not None:
            if residual.shape != x.shape or residual.dtype != torch.bfloat16:
                raise VmiError("residual must match x (bf16)")
            _require(residual, "residual", 2, self.device)
        if out is None:
            out = torch.empty_like(x)
        else:
            _require(out, "out", 2, self.device)
            if out.shape != x.shape or out.dtype != torch.bfloat16:
                raise VmiError("out must match x (bf16)")
        for name, t, dt in (("ids_out", ids_out, torch.int32), ("scores_out", scores_out, torch.float32)):
            if t is not None:
                if t.dtype != dt or t.numel() != T * self.top_k:
                    raise VmiError(f"{name} must be {dt} [T, top_k]")
                _require(t, name, 4, self.device)
        sh = _stream_handle(stream)
        if ws is None:
            ws = workspace(self.workspace_bytes(T), self.device, sh)
        rc = lib.vmi_moe_layer(ctypes.byref(self.desc), x.data_ptr(), T, _ptr(residual), out.data_ptr(),
                               _ptr(ids_out), _ptr(scores_out), ws.data_ptr(), ws.numel(), sh)
        check(rc, "vmi_moe_layer")
        return out
