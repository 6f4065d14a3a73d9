"""Gated DeltaNet (linear attention) block on libvmi.

``GatedDeltaNetLayer`` is the linear-attention half of a Qwen3-Next decoder
layer as the reference runs it at verify time: mlx-lm's
Qwen3NextGatedDeltaNet patched to capture per-token [conv, ssm] checkpoints
(mlx_streaming/mtp/kv_cache.py:34-102, core/linear_attn/
gated_delta_multistate.py:27-143).  ``GdnCache`` replaces the reference's
ArraysCache and its checkpoint list: the conv inputs and the recurrent state
are kept in rings indexed by position, so committing an accepted prefix
(commit_verified_prefix, kv_cache.py:222-251: state = checkpoint[accepted-1])
is setting ``length``.  Errors raise ``VmiError``; there is no fallback path.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from ._lib import QMat, VmiError, check, load
from .moe import QuantizedProj, _require, _stream_handle, workspace

CONV_RING = 32
HEAD_DIM = 128


class GdnDesc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("n_k_heads", ctypes.c_int), ("n_v_heads", ctypes.c_int),
                ("head_k_dim", ctypes.c_int), ("head_v_dim", ctypes.c_int), ("norm_eps", ctypes.c_float),
                ("bits", ctypes.c_int), ("group", ctypes.c_int), ("input_norm", ctypes.c_void_p),
                ("in_proj_qkvz", QMat), ("in_proj_ba", QMat), ("out_proj", QMat), ("conv_weight", ctypes.c_void_p),
                ("A_log", ctypes.c_void_p), ("dt_bias", ctypes.c_void_p), ("norm_weight", ctypes.c_void_p)]


class GdnCache:
    """Conv inputs bf16 [32, conv_dim] (row p % 32 = position p) and recurrent
    states f32 [n_slots, n_v, 128, 128] (slot p % n_slots = state before
    position p); ``length`` = committed positions."""

    def __init__(self, n_k_heads: int, n_v_heads: int, n_slots: int, device):
        self.conv_dim = 2 * n_k_heads * HEAD_DIM + n_v_heads * HEAD_DIM
        self.conv = torch.zeros((CONV_RING, self.conv_dim), dtype=torch.bfloat16, device=device)
        self.state = torch.zeros((n_slots, n_v_heads, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=device)
        self.n_slots = n_slots
        self.length = 0
        self.n_k, self.n_v = n_k_heads, n_v_heads
        # a draft tree's conv inputs and recurrence inputs, per token (16 tokens at most)
        self.tree_conv = torch.zeros((16, self.conv_dim), dtype=torch.bfloat16, device=device)
        self.tree_side = torch.zeros((16, (n_k_heads + n_v_heads) * HEAD_DIM + 2 * n_v_heads), dtype=torch.float32,
                                     device=device)

    def trim(self, n: int) -> None:
        """Drops the last n positions (the rejected drafts of a verify batch)."""
        if n < 0 or n > self.length:
            raise VmiError(f"cannot trim {n} of {self.length} positions")
        self.length -= n

    def state_before(self, pos: int) -> torch.Tensor:
        """The recurrent state before position pos (a view; zeros for pos 0)."""
        if pos == 0:
            return torch.zeros_like(self.state[0])
        return self.state[pos % self.n_slots]

    def conv_rows(self, pos: int) -> torch.Tensor:
        """Conv inputs of positions pos-3..pos-1 [3, conv_dim] (zeros before 0)."""
        rows = torch.zeros((3, self.conv_dim), dtype=torch.bfloat16, device=self.conv.device)
        for j, p in enumerate(range(pos - 3, pos)):
            if p >= 0:
                rows[j] = self.conv[p % CONV_RING]
        return rows


class GatedDeltaNetLayer:
    def __init__(self, in_proj_qkvz: QuantizedProj, in_proj_ba: QuantizedProj, out_proj: QuantizedProj,
                 input_norm: torch.Tensor, conv_weight: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor,
                 norm_weight: torch.Tensor, *, n_k_heads: int = 16, n_v_heads: int = 32, eps: float = 1e-6,
                 bits: int = 4):
        dev = input_norm.device
        self.device = dev
        self.hidden = input_norm.numel()
        self.n_k, self.n_v = n_k_heads, n_v_heads
        for name, p in (("in_proj_qkvz", in_proj_qkvz), ("in_proj_ba", in_proj_ba), ("out_proj", out_proj)):
            p.check(name, dev)
        for name, t in (("input_norm", input_norm), ("conv_weight", conv_weight), ("norm_weight", norm_weight)):
            _require(t, name, 2, dev)
        for name, t in (("A_log", A_log), ("dt_bias", dt_bias)):
            if t.dtype != torch.float32 or t.numel() != n_v_heads:
                raise VmiError(f"{name} must be float32 [{n_v_heads}]")
            _require(t, name, 4, dev)
        conv_dim = 2 * n_k_heads * HEAD_DIM + n_v_heads * HEAD_DIM
        if conv_weight.numel() != conv_dim * 4:
            raise VmiError(f"conv_weight must hold [{conv_dim}, 4] bf16")
        self._keep = (in_proj_qkvz, in_proj_ba, out_proj, input_norm, conv_weight, A_log, dt_bias, norm_weight)
        d = GdnDesc()
        d.hidden, d.n_k_heads, d.n_v_heads, d.head_k_dim, d.head_v_dim = self.hidden, n_k_heads, n_v_heads, 128, 128
        d.norm_eps, d.bits, d.group = eps, bits, 64
        d.input_norm = input_norm.data_ptr()
        d.in_proj_qkvz, d.in_proj_ba, d.out_proj = in_proj_qkvz.qmat(), in_proj_ba.qmat(), out_proj.qmat()
        d.conv_weight, d.A_log, d.dt_bias = conv_weight.data_ptr(), A_log.data_ptr(), dt_bias.data_ptr()
        d.norm_weight = norm_weight.data_ptr()
        self.desc = d

    def new_cache(self, max_batch: int = 8) -> GdnCache:
        """A cache for verify batches of up to max_batch tokens."""
        return GdnCache(self.n_k, self.n_v, max_batch + 1, self.device)

    def __call__(self, x: torch.Tensor, cache: GdnCache, *, pos0: Optional[int] = None,
                 out: Optional[torch.Tensor] = None, stream=None,
                 pos_device: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x bf16 [T, hidden] at positions pos0.. (default: cache.length);
        records the conv inputs and the state after every token, sets
        cache.length = pos0 + T.  With pos_device (int32 [1] on the device) the
        position is read there when the kernels run and cache.length is left
        to the caller."""
        T = x.shape[0]
        pos0 = cache.length if pos0 is None else pos0
        _require(x, "x", 2, self.device)
        if out is None:
            out = torch.empty_like(x)
        sh = _stream_handle(stream)
        lib = load()
        ws = workspace(lib.vmi_gdn_layer_workspace_bytes(T, self.hidden, self.n_k, self.n_v), self.device, sh,
                       tag="gdn")
        rc = lib.vmi_gdn_layer(ctypes.byref(self.desc), x.data_ptr(), T, pos0,
                               None if pos_device is None else pos_device.data_ptr(), cache.conv.data_ptr(),
                               cache.state.data_ptr(), cache.n_slots, out.data_ptr(), ws.data_ptr(), ws.numel(), sh)
        check(rc, "vmi_gdn_layer")
        if pos_device is None:
            cache.length = pos0 + T
        return out

    def tree(self, x: torch.Tensor, cache: GdnCache, paths: int, *, pos0: Optional[int] = None,
             out: Optional[torch.Tensor] = None, stream=None, pos_device: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The block over a draft tree: x bf16 [paths * span, hidden], every
        path from the state before pos0 (default: cache.length).  The rings are
        only read; conv and recurrence inputs go to cache.tree_conv /
        cache.tree_side until vmi_tree_commit applies the winner's."""
        T = x.shape[0]
        if T % paths or T > cache.tree_conv.shape[0]:
            raise VmiError(f"{T} rows do not split into {paths} paths of a tree of at most 16 tokens")
        span = T // paths
        pos0 = cache.length if pos0 is None else pos0
        _require(x, "x", 2, self.device)
        if out is None:
            out = torch.empty_like(x)
        sh = _stream_handle(stream)
        lib = load()
        ws = workspace(lib.vmi_gdn_layer_workspace_bytes(T, self.hidden, self.n_k, self.n_v), self.device, sh,
                       tag="gdn")
        rc = lib.vmi_gdn_tree(ctypes.byref(self.desc), x.data_ptr(), paths, span, pos0,
                              None if pos_device is None else pos_device.data_ptr(), cache.conv.data_ptr(),
                              cache.state.data_ptr(), cache.n_slots, cache.tree_conv.data_ptr(),
                              cache.tree_side.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(), sh)
        check(rc, "vmi_gdn_tree")
        return out

