"""MTP drafter on libvmi: the analogue of Qwen3NextMTP / mtp_step / MTPDrafter.

* ``MTPLayer.step`` is ``mtp_step`` (mlx_streaming/mtp/qwen3_next_mtp.py:60-63)
  over ``Qwen3NextMTP.__call__`` (:34-57): emb = norm_e(embed(token)),
  hid = norm_h(hidden), x = fc([emb | hid]), x = layer(x) (full attention then
  the routed MoE with its shared expert), H = norm(x), logits = lm_head(H).
* ``MTPLayer.advance`` is ``mtp_advance`` (:66-73): the same without lm_head,
  used to commit accepted positions to the MTP cache.
* ``MTPDrafter`` mirrors ``MTPDrafter.draft`` / ``draft_adaptive`` /
  ``draft_paths`` / ``sync`` (mlx_streaming/mtp/drafter.py:20-62, 150-188).  Draft tokens stay on the
  device: each step's argmax feeds the next step's embedding gather directly,
  so drafting needs no host synchronisation (the reference synchronises once
  per draft token, drafter.py:21-23).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

from ._lib import VmiError, check, load
from .attention import AttentionLayer, KVCache, qgemv
from .head import TiledHead, lm_head
from .moe import MoELayer, QuantizedProj, _require, _stream_handle


def rmsnorm(x: torch.Tensor, weight: Optional[torch.Tensor], *, eps: float = 1e-6, ids: Optional[torch.Tensor] = None,
            out: Optional[torch.Tensor] = None, out_stride: Optional[int] = None, stream=None) -> torch.Tensor:
    """bf16 RMSNorm per row (weight None: plain copy); with ids, rows are
    gathered from the table x first (embedding lookup)."""
    H = x.shape[-1]
    T = ids.numel() if ids is not None else x.numel() // H
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=x.device)
    rc = load().vmi_rmsnorm(x.data_ptr(), None if ids is None else ids.data_ptr(),
                            x.shape[0] if ids is not None else 0, T, H,
                            None if weight is None else weight.data_ptr(), float(eps), out.data_ptr(),
                            out_stride or H, None, _stream_handle(stream))
    check(rc, "vmi_rmsnorm")
    return out


@dataclass
class MTPWeights:
    embed: torch.Tensor           # [V, H] bf16 (shared with the main model)
    norm_emb: torch.Tensor        # [H] pre_fc_norm_embedding
    norm_hid: torch.Tensor        # [H] pre_fc_norm_hidden
    fc: QuantizedProj             # [1, H, 2H]
    attn: AttentionLayer
    moe: MoELayer                 # norm_weight = the layer's post-attention norm
    norm: torch.Tensor            # [H] final MTP norm
    lm_head: torch.Tensor         # [V, H] bf16 (the main model's head)
    eps: float = 1e-6


class MTPLayer:
    def __init__(self, w: MTPWeights):
        self.w = w
        self.hidden = w.embed.shape[1]
        self.vocab = w.embed.shape[0]
        self._head_tiles: Optional[TiledHead] = None

    @property
    def head_tiles(self) -> TiledHead:
        """The head in tile-major order (made on first use unless the model
        that shares this head has set its own)."""
        if self._head_tiles is None:
            self._head_tiles = TiledHead(self.w.lm_head)
        return self._head_tiles

    @head_tiles.setter
    def head_tiles(self, t: TiledHead) -> None:
        self._head_tiles = t

    def _trunk(self, hidden: torch.Tensor, tokens: torch.Tensor, cache: KVCache, stream=None,
               pos_device: Optional[torch.Tensor] = None) -> torch.Tensor:
        T, H = hidden.shape
        cat = torch.empty((T, 2 * H), dtype=torch.bfloat16, device=hidden.device)
        rmsnorm(self.w.embed, self.w.norm_emb, eps=self.w.eps, ids=tokens, out=cat, out_stride=2 * H, stream=stream)
        rmsnorm(hidden, self.w.norm_hid, eps=self.w.eps, out=cat[:, H:], out_stride=2 * H, stream=stream)
        x = torch.empty((T, H), dtype=torch.bfloat16, device=hidden.device)
        qgemv(cat, self.w.fc, out_bf16=x, stream=stream)
        x = self.w.attn(x, cache, stream=stream, pos_device=pos_device)
        x = self.w.moe(x, residual=x, stream=stream)
        return rmsnorm(x, self.w.norm, eps=self.w.eps, stream=stream)

    def step(self, hidden: torch.Tensor, tokens: torch.Tensor, cache: KVCache, *, want_logits: bool = False,
             stream=None, pos_device: Optional[torch.Tensor] = None, argmax_out: Optional[torch.Tensor] = None,
             prob_out: Optional[torch.Tensor] = None, logits_out: Optional[torch.Tensor] = None):
        """(argmax int32 [T], MTP hidden H bf16 [T, H], logits f32 [T, V] or None).
        With pos_device the cache position is read on the device; with
        argmax_out (int32 [T]) the argmax is written there; with prob_out
        (f32 [T]) the softmax probability of the argmax; with logits_out
        (f32 [T, V]) the logits are written there (want_logits implied)."""
        Hn = self._trunk(hidden, tokens, cache, stream, pos_device)
        logits, am, _ = lm_head(Hn, self.head_tiles, None, want_logits=want_logits or logits_out is not None,
                                logits=logits_out, argmax=argmax_out, top_prob=prob_out, stream=stream)
        return am, Hn, logits

    def advance(self, hidden: torch.Tensor, tokens: torch.Tensor, cache: KVCache, stream=None,
                pos_device: Optional[torch.Tensor] = None) -> torch.Tensor:
        return self._trunk(hidden, tokens, cache, stream, pos_device)


class MTPDrafter:
    def __init__(self, mtp: MTPLayer, max_len: int):
        self.mtp = mtp
        self.cache = mtp.w.attn.new_cache(max_len)

    def draft(self, H_last: torch.Tensor, x_tok: torch.Tensor, K: int) -> torch.Tensor:
        """K greedy drafts (int32 [K] on the device) from the main model's last
        hidden [1, H] and the last emitted token [1]."""
        drafts = torch.empty(K, dtype=torch.int32, device=H_last.device)
        h, tok = H_last, x_tok
        for i in range(K):
            am, h, _ = self.mtp.step(h, tok, self.cache)
            drafts[i:i + 1].copy_(am)
            tok = drafts[i:i + 1]
        return drafts

    def draft_sampled(self, H_last: torch.Tensor, x_tok: torch.Tensor, K: int, *, temperature: float,
                      top_p: float, seed: int, offset: int, offset_device: Optional[torch.Tensor] = None,
                      logits_out: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                      status: Optional[torch.Tensor] = None) -> torch.Tensor:
        """K drafts sampled from the MTP layer's own temperature / top-p
        distributions (the stochastic counterpart of ``draft``, whose argmax is
        the reference's drafter.py:20-40): draft i is vmi_sample_top_p of the
        step's logits with counter offset `offset + i` (plus *offset_device).
        logits_out (f32 [K, V]) keeps every step's logits, the draft
        distributions q that stochastic acceptance needs; out (int32 [K])
        receives the drafts; status as for ``sample_top_p``."""
        from .accept import sample_top_p
        dev = H_last.device
        if logits_out is None:
            logits_out = torch.empty((K, self.mtp.vocab), dtype=torch.float32, device=dev)
        if out is None:
            out = torch.empty(K, dtype=torch.int32, device=dev)
        h, tok = H_last, x_tok
        for i in range(K):
            _, h, _ = self.mtp.step(h, tok, self.cache, logits_out=logits_out[i:i + 1])
            sample_top_p(logits_out[i:i + 1], temperature=temperature, top_p=top_p, seed=seed, offset=offset + i,
                         offset_device=offset_device, out=out[i:i + 1], status=status)
            tok = out[i:i + 1]
        return out

    def draft_adaptive(self, H_last: torch.Tensor, x_tok: torch.Tensor, depth_max: int, tau: float,
                       logits_out: Optional[list] = None) -> torch.Tensor:
        """Confidence-gated drafts (draft_adaptive, drafter.py:42-62): greedy
        drafts while the running product of their softmax probabilities stays
        at or above tau, at least one and at most depth_max; the last position
        is not gated.  The product is taken in fp32 on the host, which reads
        each step's probability (the reference reads it the same way).
        Returns int32 [depth] on the device.  logits_out (a list) receives each
        step's f32 logits [1, V] (tests)."""
        dev = H_last.device
        drafts = torch.empty(depth_max, dtype=torch.int32, device=dev)
        probs = torch.empty(depth_max, dtype=torch.float32, device=dev)
        h, tok = H_last, x_tok
        conf = np.float32(1.0)
        for i in range(depth_max):
            _, h, lg = self.mtp.step(h, tok, self.cache, want_logits=logits_out is not None,
                                     argmax_out=drafts[i:i + 1], prob_out=probs[i:i + 1])
            if logits_out is not None:
                logits_out.append(lg)
            tok = drafts[i:i + 1]
            if i + 1 < depth_max:
                conf = np.float32(conf * np.float32(probs[i].item()))
                if conf < tau:
                    return drafts[:i + 1]
        return drafts

    def draft_paths(self, H_last: torch.Tensor, x_tok: torch.Tensor, K: int, P: int) -> torch.Tensor:
        """P paths [P, K]: the top-P first tokens (drafter.py:150-160), each
        continued greedily from the shared position-1 state."""
        paths = torch.empty((P, K), dtype=torch.int32, device=H_last.device)
        am, h1, logits = self.mtp.step(H_last, x_tok, self.cache, want_logits=True)
        firsts = torch.empty((1, P), dtype=torch.int32, device=H_last.device)
        check(load().vmi_topk_rows(logits.data_ptr(), 1, logits.shape[1], P, firsts.data_ptr(), None,
                                   _stream_handle(None)), "vmi_topk_rows")
        base = self.cache.length
        for p in range(P):
            self.cache.length = base  # every path forks from the position-1 state
            paths[p, 0:1].copy_(firsts[0, p:p + 1])
            h, tok = h1, paths[p, 0:1]
            for i in range(1, K):
                am, h, _ = self.mtp.step(h, tok, self.cache)
                paths[p, i:i + 1].copy_(am)
                tok = paths[p, i:i + 1]
        return paths

    def _top2(self, logits: torch.Tensor) -> torch.Tensor:
        """The two largest logits' token ids of a [1, V] row, int32 [2]
        (descending, ties to the lower id)."""
        out = torch.empty((1, 2), dtype=torch.int32, device=logits.device)
        check(load().vmi_topk_rows(logits.data_ptr(), 1, logits.shape[1], 2, out.data_ptr(), None,
                                   _stream_handle(None)), "vmi_topk_rows")
        return out[0]

    def _continue(self, h: torch.Tensor, first: torch.Tensor, n: int, out: torch.Tensor) -> None:
        """out[0] = first; then n greedy drafts from MTP hidden h (drafter.py's
        _continue helpers)."""
        out[0:1].copy_(first)
        tok = out[0:1]
        for i in range(1, n + 1):
            am, h, _ = self.mtp.step(h, tok, self.cache)
            out[i:i + 1].copy_(am)
            tok = out[i:i + 1]

    def draft_tree(self, H_last: torch.Tensor, x_tok: torch.Tensor, K: int, pos1: bool = True) -> torch.Tensor:
        """The minimal tree (draft_tree, drafter.py:102-148): rows [A, B, C] of
        K drafts each.  A is all top-1; B takes the second-best first token
        (the position-0 rescue); C (pos1, K >= 2) keeps A's first token and
        takes the second-best second token (the position-1 rescue).  Every
        branch continues greedily from the MTP state at its fork: the cache
        length is set back to the fork (drafter.py's _restore).  Verified
        together (``tree_speculative_decode``), the longest matched prefix with
        ties to the lower row picks the path the reference's sequential rescue
        (generate.py:764-801) ends on."""
        if K < 1:
            raise VmiError("K must be at least 1")
        dev = H_last.device
        P = 3 if pos1 and K >= 2 else 2
        paths = torch.empty((P, K), dtype=torch.int32, device=dev)
        _, h1, lg1 = self.mtp.step(H_last, x_tok, self.cache, want_logits=True)
        t1 = self._top2(lg1)                       # [d1a, d1b]
        base = self.cache.length                   # the state after x
        if P == 3:
            _, h2, lg2 = self.mtp.step(h1, t1[0:1], self.cache, want_logits=True)
            t2 = self._top2(lg2)                   # [d2a, d2c]
            base2 = self.cache.length              # the state after d1a
            paths[0, 0:1].copy_(t1[0:1])
            paths[2, 0:1].copy_(t1[0:1])
            self._continue(h2, t2[0:1], K - 2, paths[0, 1:])
            self.cache.length = base2
            self._continue(h2, t2[1:2], K - 2, paths[2, 1:])
        else:
            self._continue(h1, t1[0:1], K - 1, paths[0])
        self.cache.length = base
        self._continue(h1, t1[1:2], K - 1, paths[1])
        return paths

    def draft_adaptive_tree(self, H_last: torch.Tensor, x_tok: torch.Tensor, depth_max: int, tau: float):
        """Confidence-gated depth with the position-0 branch
        (draft_adaptive_tree, drafter.py:64-100): (chainA int32 [n], chainB
        int32 [n] or None).  chainA is greedy while the running product of its
        drafts' softmax probabilities stays at or above tau (1 <= n <=
        depth_max, the product in fp32 on the host as ``draft_adaptive``);
        chainB, only when n >= 2, takes the second-best first token and
        continues greedily to the same length from the state after x."""
        if depth_max < 1:
            raise VmiError("depth_max must be at least 1")
        dev = H_last.device
        a = torch.empty(depth_max, dtype=torch.int32, device=dev)
        probs = torch.empty(depth_max, dtype=torch.float32, device=dev)
        _, h1, lg1 = self.mtp.step(H_last, x_tok, self.cache, want_logits=True, argmax_out=a[0:1],
                                   prob_out=probs[0:1])
        t1 = self._top2(lg1)
        base = self.cache.length
        conf = np.float32(probs[0].item())
        n, h = 1, h1
        while n < depth_max and conf >= tau:
            _, h, _ = self.mtp.step(h, a[n - 1:n], self.cache, argmax_out=a[n:n + 1], prob_out=probs[n:n + 1])
            conf = np.float32(conf * np.float32(probs[n].item()))
            n += 1
        chain_b = None
        if n >= 2:
            self.cache.length = base
            chain_b = torch.empty(n, dtype=torch.int32, device=dev)
            self._continue(h1, t1[1:2], n - 1, chain_b)
        return a[:n], chain_b

    def sync(self, start: int, h_seq: torch.Tensor, tokens: torch.Tensor) -> None:
        """Replaces the draft-time cache entries from `start` by the accepted
        positions' (main hidden, token) pairs (drafter.py:178-188)."""
        self.cache.length = start
        self.mtp.advance(h_seq, tokens, self.cache)
