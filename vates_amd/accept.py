"""Acceptance of a speculative verify step on the device (libvmi).

* ``accept_greedy`` mirrors ``accept_prefix`` plus the emission rules of the
  reference's decode loop (mlx_streaming/mtp/generate.py:338-351, :819,
  :850-856) and the tree winner rule (:379-386).
* ``accept_stochastic`` is speculative sampling (Leviathan et al. 2023) on the
  same verify layout; the reference has no stochastic path.
* ``sample_top_p`` draws one token per logit row from the temperature / top-p
  distribution that ``accept_stochastic`` uses.

Results stay on the device: an int32 record [n_emitted, matched, accepted_len,
path, tokens...]; ``decode_result`` turns a host copy into Python values.
Errors raise ``VmiError``; there is no fallback path.
"""
from __future__ import annotations

from typing import Optional

import torch

from ._lib import VMI_ERR_HIP, VMI_STATUS_BAD_LOGITS, VMI_STATUS_WAIT_GAVE_UP, VmiError, check, load
from .moe import _require, _stream_handle, workspace


def decode_result(rec) -> dict:
    r = [int(v) for v in (rec.tolist() if hasattr(rec, "tolist") else rec)]
    n = r[0]
    return {"emitted": r[4:4 + n], "matched": r[1], "accepted_len": r[2], "path": r[3]}


def _result(K: int, dev, out: Optional[torch.Tensor]) -> torch.Tensor:
    if out is None:
        out = torch.zeros(4 + K + 1, dtype=torch.int32, device=dev)
    _require(out, "result", 4, dev)
    if out.numel() < 4 + K + 1:
        raise VmiError(f"result needs {4 + K + 1} entries")
    return out


def accept_greedy(drafts: torch.Tensor, preds: torch.Tensor, *, mode: int = 1, out: Optional[torch.Tensor] = None,
                  stream=None) -> torch.Tensor:
    """drafts int32 [K] or [P, K]; preds int32 [K + mode] or [P, K + mode]."""
    dev = drafts.device
    d2 = drafts.reshape(-1, drafts.shape[-1])
    P, K = d2.shape
    if preds.numel() != P * (K + mode):
        raise VmiError(f"preds must hold {P} x {K + mode} entries")
    _require(d2, "drafts", 4, dev)
    _require(preds, "preds", 4, dev)
    out = _result(K, dev, out)
    rc = load().vmi_accept_greedy(d2.data_ptr(), preds.data_ptr(), P, K, mode, out.data_ptr(),
                                  _stream_handle(stream))
    check(rc, "vmi_accept_greedy")
    return out


def spec_commit(rec: torch.Tensor, hid: torch.Tensor, H: torch.Tensor, x: torch.Tensor, pos: torch.Tensor,
                mtp_len: torch.Tensor, mtp_pos: torch.Tensor, *, rows: Optional[int] = None, paths: int = 1,
                status: Optional[torch.Tensor] = None, stream=None) -> None:
    """Commits one speculative step on the device from accept_greedy's record
    (vmi_spec_commit), with acc = accepted_len and w = the winning path:
    H = hid[w * rows + acc - 1], x = the last emitted token, pos += acc,
    mtp_len += acc, mtp_pos = mtp_len + arange(K).  hid bf16 [paths * rows, H]
    holds the verify rows (rows = K + 1 after a mode-1 record, the step's
    verify length after a mode-0 one; default: all of hid's rows).  A record
    outside [1, rows] changes nothing and sets VMI_STATUS_BAD_RECORD in status
    (int32 [1] on the device, or None)."""
    dev = rec.device
    K = mtp_pos.numel()
    if hid.dim() != 2 or hid.dtype != torch.bfloat16 or H.dtype != torch.bfloat16:
        raise VmiError("hid must be bf16 [rows, hidden] and H bf16")
    if hid.shape[0] % paths:
        raise VmiError(f"hid's {hid.shape[0]} rows do not split into {paths} paths")
    rows = hid.shape[0] // paths if rows is None else rows
    if rows <= 0 or rows * paths > hid.shape[0]:
        raise VmiError(f"hid holds {hid.shape[0]} rows, fewer than {paths} x {rows}")
    hidden = hid.shape[1]
    if H.numel() != hidden:
        raise VmiError(f"H must hold {hidden} values")
    if rec.dtype != torch.int32 or rec.numel() < 4 + rows:
        raise VmiError(f"the record must be int32 with at least {4 + rows} entries")
    for t, name in ((x, "x"), (pos, "pos"), (mtp_len, "mtp_len")):
        if t.dtype != torch.int32 or t.numel() != 1:
            raise VmiError(f"{name} must be int32 [1]")
    if mtp_pos.dtype != torch.int32:
        raise VmiError("mtp_pos must be int32")
    for t, name, elem in ((rec, "result", 4), (hid, "hid", 2), (H, "H", 2), (x, "x", 4), (pos, "pos", 4),
                          (mtp_len, "mtp_len", 4), (mtp_pos, "mtp_pos", 4)):
        _require(t, name, elem, dev)
    if status is not None:
        _require(status, "status", 4, dev)
    rc = load().vmi_spec_commit(rec.data_ptr(), hid.data_ptr(), rows, paths, hidden, K, H.data_ptr(), x.data_ptr(),
                                pos.data_ptr(), mtp_len.data_ptr(), mtp_pos.data_ptr(),
                                None if status is None else status.data_ptr(), _stream_handle(stream))
    check(rc, "vmi_spec_commit")


def _status_word(status: Optional[torch.Tensor], dev) -> torch.Tensor:
    if status is None:
        return torch.zeros(1, dtype=torch.int32, device=dev)
    _require(status, "status", 4, dev)
    return status


def _offset_device(offset_device: Optional[torch.Tensor], dev):
    if offset_device is None:
        return None
    if offset_device.dtype != torch.int64 or offset_device.numel() != 1:
        raise VmiError("offset_device must be int64 [1] on the device")
    _require(offset_device, "offset_device", 8, dev)
    return offset_device.data_ptr()


def raise_sampling_status(bits: int, what: str) -> None:
    """Raises VmiError for the status bits a sampling or stochastic
    acceptance call sets (a wait that gave up, a row without a finite logit)."""
    if bits & VMI_STATUS_WAIT_GAVE_UP:
        raise VmiError(f"{what}: a co-residency wait gave up (the device was busy with other work); "
                       "the result is the failure record", VMI_ERR_HIP)
    if bits & VMI_STATUS_BAD_LOGITS:
        raise VmiError(f"{what}: a logit row had no finite value")


def accept_stochastic(target_logits: torch.Tensor, draft_logits: Optional[torch.Tensor], drafts: torch.Tensor, *,
                      temperature: float, top_p: float, seed: int, offset: int, out: Optional[torch.Tensor] = None,
                      offset_device: Optional[torch.Tensor] = None, status: Optional[torch.Tensor] = None,
                      stream=None) -> torch.Tensor:
    """target_logits f32 [K+1, V]; draft_logits f32 [K, V] or None; drafts int32 [K].

    offset_device (int64 [1] on the device): added to offset when the kernel
    runs.  status (int32 [1] on the device): the caller's status word, which
    receives VMI_STATUS_WAIT_GAVE_UP / VMI_STATUS_BAD_LOGITS and is read by
    the caller (graph-safe).  Without it the call waits for its result and
    raises VmiError when either bit is set (the record is then [0, 0, 0, -1])."""
    dev = target_logits.device
    K1, V = target_logits.shape
    K = K1 - 1
    _require(target_logits, "target_logits", 4, dev)
    _require(drafts, "drafts", 4, dev)
    if drafts.numel() != K:
        raise VmiError(f"drafts must hold {K} entries")
    if draft_logits is not None:
        _require(draft_logits, "draft_logits", 4, dev)
        if tuple(draft_logits.shape) != (K, V):
            raise VmiError(f"draft_logits must be [{K}, {V}]")
    out = _result(K, dev, out)
    st = _status_word(status, dev)
    od = _offset_device(offset_device, dev)
    sh = _stream_handle(stream)
    lib = load()
    nbytes = lib.vmi_accept_stochastic_workspace_bytes(K, V, int(draft_logits is not None))
    ws = workspace(nbytes, dev, sh, tag="accept")
    rc = lib.vmi_accept_stochastic(target_logits.data_ptr(), None if draft_logits is None else draft_logits.data_ptr(),
                                   drafts.data_ptr(), K, V, float(temperature), float(top_p), int(seed) & (2**64 - 1),
                                   int(offset) & (2**64 - 1), od, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                   st.data_ptr(), sh)
    check(rc, "vmi_accept_stochastic")
    if status is None:
        raise_sampling_status(int(st.item()), "vmi_accept_stochastic")
    return out


def sample_top_p(logits: torch.Tensor, *, temperature: float, top_p: float, seed: int, offset: int,
                 out: Optional[torch.Tensor] = None, offset_device: Optional[torch.Tensor] = None,
                 status: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """logits f32 [rows, V] -> int32 [rows].  offset_device and status as for
    ``accept_stochastic`` (without status the call raises on a failed row)."""
    dev = logits.device
    rows, V = logits.shape
    _require(logits, "logits", 4, dev)
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=dev)
    _require(out, "out", 4, dev)
    st = _status_word(status, dev)
    od = _offset_device(offset_device, dev)
    sh = _stream_handle(stream)
    lib = load()
    ws = workspace(lib.vmi_sample_top_p_workspace_bytes(rows, V), dev, sh, tag="sample")
    rc = lib.vmi_sample_top_p(logits.data_ptr(), rows, V, float(temperature), float(top_p), int(seed) & (2**64 - 1),
                              int(offset) & (2**64 - 1), od, out.data_ptr(), ws.data_ptr(), ws.numel(),
                              st.data_ptr(), sh)
    check(rc, "vmi_sample_top_p")
    if status is None:
        raise_sampling_status(int(st.item()), "vmi_sample_top_p")
    return out


def set_wait_limit(polls: int) -> int:
    """Bound of the sampling kernels' co-residency waits (vmi_set_wait_limit);
    polls <= 0 restores the default.  Returns the previous bound."""
    return int(load().vmi_set_wait_limit(int(polls)))
