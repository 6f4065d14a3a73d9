"""K-draft MTP speculative decoding on libvmi: the analogue of ``mtp_generate``.

* ``SpecModel.forward`` is ``forward_with_hidden`` (mlx_streaming/mtp/
  generate.py:101-220): embedding, decoder layers (full attention or the
  Gated DeltaNet block, then the routed MoE with its shared expert), the final norm
  and the head; returns the argmax of every position and the pre-norm hidden
  states the MTP drafter consumes (generate.py:209-216).
* ``speculative_decode`` is the decode loop of ``mtp_generate`` in the verify
  layout [x, d1..dK] (generate.py:540-906, T = K + 1): draft K tokens with the
  MTP layer, verify them in one batch, accept the longest matching prefix plus
  the model's next token (``vmi_accept_greedy``), commit by trimming the
  attention caches to the accepted length (kv_cache.py:222-251) and re-advance
  the MTP cache with the accepted positions (drafter.py:178-188).
* ``greedy_decode`` is the non-speculative reference the speculative loop must
  reproduce token for token (test_mtp_generate.py:421-489).

Each decoder layer runs full attention or the Gated DeltaNet block (or
neither), then the MoE block.
Errors raise ``VmiError``; there is no fallback path.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import List, Optional

import torch

from ._lib import VmiError
from .accept import accept_greedy
from .attention import AttentionLayer, KVCache
from .gdn import GatedDeltaNetLayer, GdnCache
from .head import lm_head
from .moe import MoELayer
from .mtp import MTPDrafter, MTPLayer, rmsnorm


@dataclass
class DecoderLayer:
    moe: MoELayer                        # norm_weight = the post-attention norm
    attn: Optional[AttentionLayer] = None
    gdn: Optional[GatedDeltaNetLayer] = None


@dataclass
class DecodeStats:
    tokens: List[int] = field(default_factory=list)
    steps: int = 0
    accept_hist: List[int] = field(default_factory=list)   # matched drafts per step
    seconds: float = 0.0

    @property
    def avg_accept_len(self) -> float:
        return (sum(self.accept_hist) / len(self.accept_hist) + 1.0) if self.accept_hist else 0.0


class SpecModel:
    def __init__(self, embed: torch.Tensor, layers: List[DecoderLayer], final_norm: torch.Tensor,
                 head: torch.Tensor, mtp: Optional[MTPLayer] = None, eps: float = 1e-6):
        self.embed, self.layers, self.final_norm, self.head, self.mtp, self.eps = embed, layers, final_norm, head, mtp, eps
        self.hidden = embed.shape[1]

    def new_caches(self, max_len: int, max_batch: int = 8) -> list:
        """Per layer: a KVCache (full attention), a GdnCache (linear attention,
        verify batches up to max_batch tokens) or None."""
        return [l.attn.new_cache(max_len) if l.attn is not None else
                l.gdn.new_cache(max_batch) if l.gdn is not None else None for l in self.layers]

    def forward(self, ids: torch.Tensor, caches: list, pos0: int, *, want_logits: bool = False):
        """ids int32 [T] on the device at positions pos0..; returns (argmax int32 [T],
        pre-norm hidden bf16 [T, H], logits f32 [T, V] or None)."""
        x = rmsnorm(self.embed, None, ids=ids)
        for layer, cache in zip(self.layers, caches):
            if layer.attn is not None:
                x = layer.attn(x, cache, pos0=pos0)
            elif layer.gdn is not None:
                x = layer.gdn(x, cache, pos0=pos0)
            x = layer.moe(x, residual=x)
        logits, am, _ = lm_head(x, self.head, self.final_norm, eps=self.eps, want_logits=want_logits)
        return am, x, logits

    def commit(self, caches: list, length: int) -> None:
        """Keeps positions < length in every cache (commit_verified_prefix,
        kv_cache.py:222-251): attention caches drop the rejected keys, linear
        attention continues from the state captured after position length - 1."""
        for c in caches:
            if c is not None:
                c.length = length


def prefill(model: SpecModel, prompt: torch.Tensor, caches, drafter: Optional[MTPDrafter] = None, chunk: int = 8):
    """Runs the prompt (int32 [P] on the device) through the model in chunks of
    at most `chunk` tokens and, with a drafter, advances its cache over the
    prompt's (hidden, next token) pairs; returns (next token [1], hidden of the
    last position [1, H])."""
    P = prompt.numel()
    hs = []
    am = None
    for s in range(0, P, chunk):
        am, h, _ = model.forward(prompt[s:s + chunk], caches, s)
        hs.append(h)
    hid = torch.cat(hs)
    if drafter is not None and P > 1:
        drafter.cache.length = 0
        for s in range(0, P - 1, chunk):
            e = min(P - 1, s + chunk)
            drafter.mtp.advance(hid[s:e].contiguous(), prompt[s + 1:e + 1].contiguous(), drafter.cache)
    return am[-1:].clone(), hid[-1:].clone()


def greedy_decode(model: SpecModel, caches, x: torch.Tensor, pos: int, n_tokens: int) -> DecodeStats:
    """One token per forward (the non-speculative loop)."""
    st = DecodeStats()
    t0 = time.perf_counter()
    for _ in range(n_tokens):
        am, _, _ = model.forward(x, caches, pos)
        st.tokens.append(int(am[0].item()))
        x = am[:1].clone()
        pos += 1
        st.steps += 1
    st.seconds = time.perf_counter() - t0
    return st


def speculative_decode(model: SpecModel, drafter: MTPDrafter, caches, x: torch.Tensor, H_last: torch.Tensor,
                       pos: int, n_tokens: int, K: int = 3) -> DecodeStats:
    """K-draft MTP decoding with greedy acceptance in the [x, d1..dK] layout.

    x: the last emitted token [1] (not yet run through the model) at position
    `pos`; H_last: the model's pre-norm hidden at pos - 1 [1, H]; the MTP cache
    holds every committed position before pos.
    """
    if model.mtp is None:
        raise VmiError("the model has no MTP layer")
    st = DecodeStats()
    dev = x.device
    verify = torch.empty(K + 1, dtype=torch.int32, device=dev)
    t0 = time.perf_counter()
    while len(st.tokens) < n_tokens:
        mtp_start = drafter.cache.length
        drafts = drafter.draft(H_last, x, K)
        verify[0:1].copy_(x)
        verify[1:].copy_(drafts)
        preds, hid, _ = model.forward(verify, caches, pos)
        rec = accept_greedy(drafts, preds, mode=1)
        r = rec.cpu().tolist()  # the step's one host synchronisation
        n, m, acc = r[0], r[1], r[2]
        emitted = r[4:4 + n]
        model.commit(caches, pos + acc)
        # MTP cache: (main hidden at pos-1 .. pos+m-1, tokens x, d1..dm)
        h_seq = torch.cat([H_last, hid[:m]]) if m else H_last
        drafter.sync(mtp_start, h_seq.contiguous(), verify[:m + 1].contiguous())
        st.tokens.extend(emitted)
        st.accept_hist.append(m)
        st.steps += 1
        pos += acc
        x = torch.tensor([emitted[-1]], dtype=torch.int32, device=dev)
        H_last = hid[m:m + 1].clone()
    st.seconds = time.perf_counter() - t0
    st.tokens = st.tokens[:n_tokens]
    return st
