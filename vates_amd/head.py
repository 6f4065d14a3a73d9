"""lm_head over the vocabulary with the argmax fused in (libvmi ``vmi_lm_head``).

The analogue of the verify forward's tail ``logits = model.lm_head(inner.norm(h))``
followed by ``preds = mx.argmax(logits, -1)`` (mlx_streaming/mtp/generate.py:208-217,
:756) and of the draft step's ``int(mx.argmax(lg))`` (mlx_streaming/mtp/drafter.py:20-40).
Errors raise ``VmiError``; there is no fallback path.
"""
from __future__ import annotations

from typing import Optional

import torch

from ._lib import VmiError, check, load
from .moe import _require, _stream_handle, workspace


class TiledHead:
    """A bf16 [vocab, hidden] head re-laid once in tile-major order
    (``vmi_head_tiles``: each 16-row x 128-value chunk is 4 KB of contiguous
    memory), for callers that run the head every decode step; ``lm_head`` on it
    gives the row-major head's results bit for bit, faster."""

    def __init__(self, weight: torch.Tensor, stream=None):
        if weight.dim() != 2 or weight.dtype != torch.bfloat16 or not weight.is_cuda:
            raise VmiError("weight must be a bf16 [vocab, hidden] device tensor")
        weight = weight.contiguous()
        self.vocab, self.hidden = int(weight.shape[0]), int(weight.shape[1])
        lib = load()
        nbytes = int(lib.vmi_head_tiles_bytes(self.vocab, self.hidden))
        if nbytes == 0:
            raise VmiError(f"unsupported head shape {tuple(weight.shape)}")
        self.tiles = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=weight.device)
        check(lib.vmi_head_tiles(weight.data_ptr(), self.vocab, self.hidden, self.tiles.data_ptr(),
                                 _stream_handle(stream)), "vmi_head_tiles")

    @property
    def device(self):
        return self.tiles.device


def lm_head(x: torch.Tensor, weight, norm_weight: Optional[torch.Tensor] = None, *,
            eps: float = 1e-6, want_logits: bool = True, logits: Optional[torch.Tensor] = None,
            argmax: Optional[torch.Tensor] = None, max_logit: Optional[torch.Tensor] = None,
            top_prob: Optional[torch.Tensor] = None, stream=None):
    """Returns (logits f32 [T, V] or None, argmax int32 [T], max logit f32 [T]).

    x bf16 [T, H] (T <= 16), weight bf16 [V, H] or a TiledHead of one,
    norm_weight bf16 [H] or None.
    top_prob (f32 [T], optional) receives the softmax probability of each
    row's argmax (the draft confidence of drafter.py:42-62).
    """
    dev = x.device
    if x.dim() != 2:
        raise VmiError(f"x must be [T, hidden], got {tuple(x.shape)}")
    T, H = x.shape
    tiled = isinstance(weight, TiledHead)
    if tiled:
        if weight.hidden != H:
            raise VmiError(f"tiled head has hidden {weight.hidden}, x has {H}")
        V, wt = weight.vocab, weight.tiles
    else:
        if weight.dim() != 2 or weight.shape[1] != H:
            raise VmiError(f"weight must be [vocab, {H}], got {tuple(weight.shape)}")
        V, wt = weight.shape[0], weight
    _require(x, "x", 2, dev)
    _require(wt, "weight", 2, dev)
    if norm_weight is not None:
        _require(norm_weight, "norm_weight", 2, dev)
        if norm_weight.numel() != H:
            raise VmiError(f"norm_weight must have {H} elements")
    if want_logits and logits is None:
        logits = torch.empty((T, V), dtype=torch.float32, device=dev)
    if argmax is None:
        argmax = torch.empty(T, dtype=torch.int32, device=dev)
    if max_logit is None:
        max_logit = torch.empty(T, dtype=torch.float32, device=dev)
    for t, name, n in ((logits, "logits", T * V), (argmax, "argmax", T), (max_logit, "max_logit", T),
                       (top_prob, "top_prob", T)):
        if t is not None:
            _require(t, name, 4, dev)
            if t.numel() != n:
                raise VmiError(f"{name} must have {n} elements")
    sh = _stream_handle(stream)
    lib = load()
    nbytes = lib.vmi_lm_head_workspace_bytes(T, V)
    ws = workspace(nbytes, dev, sh, tag="lm_head")
    fn = lib.vmi_lm_head_tiled if tiled else lib.vmi_lm_head
    rc = fn(x.data_ptr(), T, H, None if norm_weight is None else norm_weight.data_ptr(), float(eps),
                         wt.data_ptr(), V, None if logits is None else logits.data_ptr(), argmax.data_ptr(),
                         max_logit.data_ptr(), None if top_prob is None else top_prob.data_ptr(), ws.data_ptr(),
                         ws.numel(), sh)
    check(rc, "vmi_lm_head_tiled" if tiled else "vmi_lm_head")
    return logits, argmax, max_logit
