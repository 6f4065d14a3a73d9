"""Full-attention decoder block and quantised GEMV on libvmi.

``AttentionLayer`` is the attention half of a Qwen3-Next decoder layer as the
MTP layer runs it (mlx_streaming/mtp/qwen3_next_mtp.py:34-57, ``self.layer``)
and as the main model's full-attention layers run it in the verify forward
(mlx_streaming/mtp/generate.py:101-220): out = x + attn(rmsnorm(x)) with the KV
cache updated in place.  ``KVCache`` holds one layer's bf16 keys and values
and the number of committed positions, the analogue of mlx-lm's KVCache with
its trim (mlx_streaming/mtp/kv_cache.py:222-251); its storage is blocks of 32
positions in the attention kernel's operand order (``keys``/``values`` and
``write`` convert from and to [n_kv_heads, positions, 256]).
Errors raise ``VmiError``; there is no fallback path.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from ._lib import QMat, VmiError, check, load
from .moe import QuantizedProj, _require, _stream_handle, workspace


class AttnDesc(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("n_heads", ctypes.c_int), ("n_kv_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("rope_dim", ctypes.c_int), ("rope_theta", ctypes.c_float),
                ("norm_eps", ctypes.c_float), ("bits", ctypes.c_int), ("group", ctypes.c_int),
                ("input_norm", ctypes.c_void_p), ("q_proj", QMat), ("k_proj", QMat), ("v_proj", QMat),
                ("o_proj", QMat), ("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p)]


def qgemv(x: torch.Tensor, w: QuantizedProj, *, bits: int = 4, out: Optional[torch.Tensor] = None,
          residual: Optional[torch.Tensor] = None, out_bf16: Optional[torch.Tensor] = None, stream=None):
    """y = W x for x bf16 [T, K] (T <= 8): f32 [T, N] and/or bf16(y + residual)."""
    T, K = x.shape
    N = w.weight.shape[-2]
    dev = x.device
    _require(x, "x", 2, dev)
    if out is None and out_bf16 is None:
        out = torch.empty((T, N), dtype=torch.float32, device=dev)
    rc = load().vmi_qgemv(x.data_ptr(), T, K, w.qmat(), N, bits, 64, None if out is None else out.data_ptr(),
                          None if residual is None else residual.data_ptr(),
                          None if out_bf16 is None else out_bf16.data_ptr(), _stream_handle(stream))
    check(rc, "vmi_qgemv")
    return out if out is not None else out_bf16


KV_BLOCK = 32          # positions per cache block
_PERM = {}


def _block_perm(kind: str, device) -> torch.Tensor:
    """Storage offset inside a block (8192 bf16) of (position kt, dim d), flattened
    as kt * 256 + d: keys ((a*8 + kk)*64 + q4*16 + nl)*8 + e with
    kt = 8*(nl>>2) + 4*a + (nl&3), d = 32*kk + 8*q4 + e; values
    ((dt*64 + q4*16 + nl)*8 + e) with kt = 8*q4 + e, d = 16*dt + nl."""
    key = (kind, str(device))
    if key not in _PERM:
        kt = torch.arange(KV_BLOCK).view(-1, 1)
        d = torch.arange(256).view(1, -1)
        if kind == "k":
            nl, a = 4 * (kt >> 3) + (kt & 3), (kt >> 2) & 1
            off = (((a * 8 + (d >> 5)) * 64 + ((d >> 3) & 3) * 16 + nl) << 3) + (d & 7)
        else:
            off = ((((d >> 4) * 64 + (kt >> 3) * 16 + (d & 15)) << 3) + (kt & 7))
        _PERM[key] = off.reshape(-1).to(device)
    return _PERM[key]


class KVCache:
    """bf16 keys and values of one attention layer: k, v [n_kv_heads, blocks, 8192]
    (32 positions per block, kernel operand order); capacity rounds up to 32."""

    def __init__(self, n_kv_heads: int, max_len: int, device, head_dim: int = 256):
        if head_dim != 256:
            raise VmiError(f"head_dim={head_dim} (256 only)")
        self.max_len = -(-max_len // KV_BLOCK) * KV_BLOCK
        nb = self.max_len // KV_BLOCK
        self.k = torch.zeros((n_kv_heads, nb, KV_BLOCK * head_dim), dtype=torch.bfloat16, device=device)
        self.v = torch.zeros_like(self.k)
        self.length = 0  # committed positions
        self.n_kv = n_kv_heads
        self.tree_kv = None  # [paths, n_kv, 2, span, 256] bf16: a draft tree's new keys and values
        self._tree_flat = None

    def tree_buffer(self, paths: int, span: int) -> torch.Tensor:
        """The tree forward's keys and values [paths, n_kv, 2, span, 256]: one
        allocation for every tree of at most 16 tokens, so commit tables built
        for different (paths, span) see the same address."""
        if paths * span > 16:
            raise VmiError(f"a tree of {paths} x {span} tokens exceeds 16")
        if self._tree_flat is None:
            self._tree_flat = torch.zeros(16 * self.n_kv * 2 * 256, dtype=torch.bfloat16, device=self.k.device)
        self.tree_kv = self._tree_flat[:paths * self.n_kv * 2 * span * 256].view(paths, self.n_kv, 2, span, 256)
        return self.tree_kv

    def trim(self, n: int) -> None:
        """Drops the last n positions (kv_cache.py:222-251: rejected drafts)."""
        if n < 0 or n > self.length:
            raise VmiError(f"cannot trim {n} of {self.length} positions")
        self.length -= n

    def _read(self, raw: torch.Tensor, kind: str, start: int, stop: int) -> torch.Tensor:
        b0, b1 = start // KV_BLOCK, -(-stop // KV_BLOCK)
        blk = raw[:, b0:b1]
        logical = blk[:, :, _block_perm(kind, raw.device)].reshape(raw.shape[0], (b1 - b0) * KV_BLOCK, 256)
        return logical[:, start - b0 * KV_BLOCK:stop - b0 * KV_BLOCK]

    def keys(self, start: int = 0, stop: Optional[int] = None) -> torch.Tensor:
        """Keys of positions start..stop-1 as [n_kv_heads, positions, 256] (a copy)."""
        return self._read(self.k, "k", start, self.length if stop is None else stop)

    def values(self, start: int = 0, stop: Optional[int] = None) -> torch.Tensor:
        return self._read(self.v, "v", start, self.length if stop is None else stop)

    def write(self, start: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Stores [n_kv_heads, n, 256] keys and values at positions start..start+n-1."""
        n = keys.shape[1]
        if start < 0 or start + n > self.max_len:
            raise VmiError(f"positions {start}..{start + n} outside the capacity {self.max_len}")
        b0, b1 = start // KV_BLOCK, -(-(start + n) // KV_BLOCK)
        for raw, kind, data in ((self.k, "k", keys), (self.v, "v", values)):
            logical = self._read(raw, kind, b0 * KV_BLOCK, b1 * KV_BLOCK).clone()
            logical[:, start - b0 * KV_BLOCK:start - b0 * KV_BLOCK + n] = data
            blk = torch.empty_like(raw[:, b0:b1])
            blk[:, :, _block_perm(kind, raw.device)] = logical.reshape(raw.shape[0], b1 - b0, -1)
            raw[:, b0:b1] = blk


class AttentionLayer:
    def __init__(self, q_proj: QuantizedProj, k_proj: QuantizedProj, v_proj: QuantizedProj, o_proj: QuantizedProj,
                 input_norm: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor, *, n_heads: int = 16,
                 n_kv_heads: int = 2, rope_dim: int = 64, rope_theta: float = 1e7, eps: float = 1e-6,
                 bits: int = 4):
        dev = input_norm.device
        self.device = dev
        self.hidden = input_norm.numel()
        self.n_heads, self.n_kv = n_heads, n_kv_heads
        for name, p in (("q_proj", q_proj), ("k_proj", k_proj), ("v_proj", v_proj), ("o_proj", o_proj)):
            p.check(name, dev)
        for name, t in (("input_norm", input_norm), ("q_norm", q_norm), ("k_norm", k_norm)):
            _require(t, name, 2, dev)
        self._keep = (q_proj, k_proj, v_proj, o_proj, input_norm, q_norm, k_norm)
        d = AttnDesc()
        d.hidden, d.n_heads, d.n_kv_heads, d.head_dim, d.rope_dim = self.hidden, n_heads, n_kv_heads, 256, rope_dim
        d.rope_theta, d.norm_eps, d.bits, d.group = rope_theta, eps, bits, 64
        d.input_norm = input_norm.data_ptr()
        d.q_proj, d.k_proj, d.v_proj, d.o_proj = q_proj.qmat(), k_proj.qmat(), v_proj.qmat(), o_proj.qmat()
        d.q_norm, d.k_norm = q_norm.data_ptr(), k_norm.data_ptr()
        self.desc = d

    def new_cache(self, max_len: int) -> KVCache:
        return KVCache(self.n_kv, max_len, self.device)

    def __call__(self, x: torch.Tensor, cache: KVCache, *, pos0: Optional[int] = None,
                 out: Optional[torch.Tensor] = None, stream=None,
                 pos_device: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x bf16 [T, hidden] at cache positions pos0.. (default: cache.length);
        appends k, v there and sets cache.length = pos0 + T.  With pos_device
        (int32 [1] on the device) the position is read there when the kernels
        run and cache.length is left to the caller."""
        T = x.shape[0]
        pos0 = cache.length if pos0 is None else pos0
        _require(x, "x", 2, self.device)
        if out is None:
            out = torch.empty_like(x)
        sh = _stream_handle(stream)
        lib = load()
        ws = workspace(lib.vmi_attention_layer_workspace_bytes(T, self.hidden, self.n_heads, self.n_kv, cache.max_len),
                       self.device, sh, tag="attention")
        rc = lib.vmi_attention_layer(ctypes.byref(self.desc), x.data_ptr(), T, pos0,
                                     None if pos_device is None else pos_device.data_ptr(), cache.k.data_ptr(),
                                     cache.v.data_ptr(), cache.max_len, out.data_ptr(), ws.data_ptr(), ws.numel(), sh)
        check(rc, "vmi_attention_layer")
        if pos_device is None:
            cache.length = pos0 + T
        return out

    def tree(self, x: torch.Tensor, cache: KVCache, paths: int, *, pos0: Optional[int] = None,
             out: Optional[torch.Tensor] = None, stream=None, pos_device: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The block over a draft tree: x bf16 [paths * span, hidden], path p's
        tokens at rows p*span.. and positions pos0.. (default: cache.length).
        The cache is only read; every path's new keys and values go to
        cache.tree_kv until vmi_tree_commit writes the winner's."""
        T = x.shape[0]
        if T % paths:
            raise VmiError(f"{T} rows do not split into {paths} paths")
        span = T // paths
        pos0 = cache.length if pos0 is None else pos0
        _require(x, "x", 2, self.device)
        if out is None:
            out = torch.empty_like(x)
        tkv = cache.tree_buffer(paths, span)
        sh = _stream_handle(stream)
        lib = load()
        ws = workspace(lib.vmi_attention_tree_workspace_bytes(paths, span, self.hidden, self.n_heads, self.n_kv,
                                                              cache.max_len), self.device, sh, tag="attention")
        rc = lib.vmi_attention_tree(ctypes.byref(self.desc), x.data_ptr(), paths, span, pos0,
                                    None if pos_device is None else pos_device.data_ptr(), cache.k.data_ptr(),
                                    cache.v.data_ptr(), cache.max_len, tkv.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                    ws.numel(), sh)
        check(rc, "vmi_attention_tree")
        return out

