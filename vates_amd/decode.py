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
* With a ``Sampling`` the same loop decodes stochastically (speculative
  sampling; the reference has only the greedy loop): drafts sampled from the
  MTP layer's temperature / top-p distributions, accepted or replaced by
  ``vmi_accept_stochastic`` against the verify rows' distributions.

Each decoder layer runs full attention or the Gated DeltaNet block (or
neither), then the MoE block.
Errors raise ``VmiError``; there is no fallback path.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch

from ._lib import VmiError, check, load
from .accept import accept_greedy, accept_stochastic, raise_sampling_status, sample_top_p, spec_commit
from .attention import AttentionLayer, KVCache
from .gdn import GatedDeltaNetLayer, GdnCache
from .head import TiledHead, lm_head
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
    depths: List[int] = field(default_factory=list)        # drafts verified per step (adaptive depth)
    rescues: List[int] = field(default_factory=list)       # tree decoding: the winning path per step
    drafts: List[List[int]] = field(default_factory=list)  # the drafts of each step (with trace=True)
    samples: List[dict] = field(default_factory=list)      # stochastic steps with trace=True: logits, drafts, record
    seconds: float = 0.0

    @property
    def avg_accept_len(self) -> float:
        return (sum(self.accept_hist) / len(self.accept_hist) + 1.0) if self.accept_hist else 0.0


@dataclass(frozen=True)
class Sampling:
    """Stochastic speculative decoding (speculative sampling, Leviathan et al.
    2023; no counterpart in the reference, whose loop is greedy): the K drafts
    are sampled from the MTP layer's temperature / top-p distributions
    (vmi_sample_top_p), the verify rows' distributions accept or replace them
    (vmi_accept_stochastic), and vmi_spec_commit commits the record as in the
    greedy loop.  Step s of a run draws with Philox key `seed` and counter
    offsets 64 (first_step + s) + i for draft i and 64 (first_step + s) + 63
    for the acceptance, so every draw of a run has its own counter."""
    temperature: float
    top_p: float = 1.0
    seed: int = 0
    first_step: int = 0

    ACCEPT_OFFSET = 63

    def step_base(self, step: int) -> int:
        return 64 * (self.first_step + step)


class SpecModel:
    def __init__(self, embed: torch.Tensor, layers: List[DecoderLayer], final_norm: torch.Tensor,
                 head: torch.Tensor, mtp: Optional[MTPLayer] = None, eps: float = 1e-6):
        self.embed, self.layers, self.final_norm, self.head, self.mtp, self.eps = embed, layers, final_norm, head, mtp, eps
        self.hidden = embed.shape[1]
        # the head as the decode loop reads it every step (tile-major copy,
        # shared with an MTP layer whose head is this one)
        self.head_tiles = TiledHead(head)
        if mtp is not None and mtp.w.lm_head is head:
            mtp.head_tiles = self.head_tiles

    def new_caches(self, max_len: int, max_batch: int = 8) -> list:
        """Per layer: a KVCache (full attention), a GdnCache (linear attention,
        verify batches up to max_batch tokens) or None."""
        return [l.attn.new_cache(max_len) if l.attn is not None else
                l.gdn.new_cache(max_batch) if l.gdn is not None else None for l in self.layers]

    def forward(self, ids: torch.Tensor, caches: list, pos0: int, *, want_logits: bool = False,
                pos_device: Optional[torch.Tensor] = None, hidden_out: Optional[torch.Tensor] = None,
                logits_out: Optional[torch.Tensor] = None):
        """ids int32 [T] on the device at positions pos0.. (or at the position
        held by pos_device, int32 [1] on the device); returns (argmax int32 [T],
        pre-norm hidden bf16 [T, H], logits f32 [T, V] or None).  hidden_out
        (bf16 [T, H], optional): where the last layer writes the hidden;
        logits_out (f32 [T, V], optional): where the head writes the logits."""
        x = rmsnorm(self.embed, None, ids=ids)
        last = len(self.layers) - 1
        for i, (layer, cache) in enumerate(zip(self.layers, caches)):
            if layer.attn is not None:
                x = layer.attn(x, cache, pos0=pos0, pos_device=pos_device)
            elif layer.gdn is not None:
                x = layer.gdn(x, cache, pos0=pos0, pos_device=pos_device)
            x = layer.moe(x, residual=x, out=hidden_out if i == last else None)
        logits, am, _ = lm_head(x, self.head_tiles, self.final_norm, eps=self.eps,
                                want_logits=want_logits or logits_out is not None, logits=logits_out)
        return am, x, logits

    def forward_tree(self, ids: torch.Tensor, caches: list, pos0: int, paths: int, *, want_logits: bool = False,
                     pos_device: Optional[torch.Tensor] = None):
        """One forward over a draft tree (tree_verify_step's batched forward,
        generate.py:355-376): ids int32 [paths * span], path p's tokens at rows
        p*span.. and positions pos0..; every path sees the committed caches and
        its own earlier tokens, and the caches are left untouched (the new
        entries wait in the caches' tree buffers for ``TreeCommit``).  Returns
        (argmax int32 [paths * span], pre-norm hidden bf16 [paths * span, H],
        logits or None); a path's rows equal ``forward`` of its tokens alone."""
        x = rmsnorm(self.embed, None, ids=ids)
        for layer, cache in zip(self.layers, caches):
            if layer.attn is not None:
                x = layer.attn.tree(x, cache, paths, pos0=pos0, pos_device=pos_device)
            elif layer.gdn is not None:
                x = layer.gdn.tree(x, cache, paths, pos0=pos0, pos_device=pos_device)
            x = layer.moe(x, residual=x)
        logits, am, _ = lm_head(x, self.head_tiles, self.final_norm, eps=self.eps, want_logits=want_logits)
        return am, x, logits

    def commit(self, caches: list, length: int) -> None:
        """Keeps positions < length in every cache (commit_verified_prefix,
        kv_cache.py:222-251): attention caches drop the rejected keys, linear
        attention continues from the state captured after position length - 1."""
        for c in caches:
            if c is not None:
                c.length = length


class TreeCommit:
    """Commits the winning path of a tree forward into every cache in one
    launch (vmi_tree_commit; commit_tree_row, kv_cache.py:283-316): for the
    acceptance record's path w and accepted length acc, the attention layers'
    keys and values of positions pos0 .. pos0 + acc - 1, the linear-attention
    layers' conv inputs of those positions and their state before pos0 + acc.
    The layer table lives in device memory."""

    def __init__(self, caches: list, paths: int, span: int):
        from ._lib import VMI_TREE_ATTENTION, VMI_TREE_GDN, TreeLayer
        rows = []
        heads = 1
        for c in caches:
            if c is None:
                continue
            e = TreeLayer()
            if isinstance(c, KVCache):
                tkv = c.tree_buffer(paths, span)
                e.kind, e.n_kv_heads, e.max_len = VMI_TREE_ATTENTION, c.n_kv, c.max_len
                e.k_cache, e.v_cache, e.tree_kv = c.k.data_ptr(), c.v.data_ptr(), tkv.data_ptr()
                heads = max(heads, c.n_kv)
            elif isinstance(c, GdnCache):
                e.kind, e.n_k_heads, e.n_v_heads, e.n_slots = VMI_TREE_GDN, c.n_k, c.n_v, c.n_slots
                e.conv_ring, e.state_ring = c.conv.data_ptr(), c.state.data_ptr()
                e.tree_conv, e.tree_side = c.tree_conv.data_ptr(), c.tree_side.data_ptr()
                heads = max(heads, c.n_v)
            else:
                raise VmiError(f"cannot commit a tree into {type(c).__name__}")
            rows.append(bytes(e))
        self.n, self.heads, self.paths, self.span = len(rows), heads, paths, span
        self.caches = caches
        dev = next(c.k.device if isinstance(c, KVCache) else c.conv.device for c in caches if c is not None)
        self.table = torch.frombuffer(bytearray(b"".join(rows)), dtype=torch.uint8).to(dev)

    def __call__(self, rec: torch.Tensor, *, pos0: int = 0, pos_device: Optional[torch.Tensor] = None,
                 stream=None) -> None:
        from .moe import _stream_handle
        rc = load().vmi_tree_commit(rec.data_ptr(), self.table.data_ptr(), self.n, self.heads, self.paths, self.span, pos0,
                                    None if pos_device is None else pos_device.data_ptr(), _stream_handle(stream))
        check(rc, "vmi_tree_commit")


def commit_verified_prefix(caches: list, verified_len: int, accepted_len: int) -> bool:
    """Commits the accepted prefix of a verify batch of verified_len positions
    (kv_cache.py:222-251): every cache drops the rejected verified_len -
    accepted_len positions.  Attention caches keep their keys below the new
    length; linear-attention caches continue from the state captured after the
    last accepted token (the reference's checkpoint[accepted_len - 1]), which
    the position-indexed rings already hold.  Returns True (the rings always
    hold every token's state, so the commit cannot fall back to a replay)."""
    rejected = verified_len - accepted_len
    if rejected < 0 or accepted_len < 0:
        raise VmiError("accepted_len cannot exceed verified_len")
    for c in caches:
        if c is not None:
            c.trim(rejected)
    return True


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


LAYOUTS = ("k+1", "k")


def _check_layout(layout: str, tau: Optional[float]) -> None:
    if layout not in LAYOUTS:
        raise VmiError(f"layout {layout!r} is not one of {LAYOUTS}")
    if tau is not None and layout != "k":
        raise VmiError("adaptive depth verifies in the T = K layout (layout='k')")


def speculative_decode(model: SpecModel, drafter: MTPDrafter, caches, x: torch.Tensor, H_last: torch.Tensor,
                       pos: int, n_tokens: int, K: int = 3, *, layout: str = "k+1",
                       tau: Optional[float] = None, trace: bool = False,
                       sampling: Optional[Sampling] = None) -> DecodeStats:
    """K-draft MTP decoding with greedy acceptance (or, with `sampling`,
    stochastic: see ``Sampling``; layout "k+1" at a fixed depth).

    layout "k+1": the verify batch is [x, d1..dK] (T = K + 1): every draft is
    checked and the model's token after the last accepted one is emitted, so
    a step emits up to K + 1 tokens (accept mode 1).
    layout "k": the reference's batch [x, d1..d_{K-1}] (T = K,
    generate.py:604): dK is checked against the model's last prediction,
    accepted_len = min(matched + 1, K) and a step emits up to K tokens; when
    every draft matches, the next input is dK itself (generate.py:819,
    850-856; accept mode 0).
    tau: adaptive depth (draft_adaptive, drafter.py:42-62, layout "k"): each
    step drafts 1..K tokens while the product of their softmax probabilities
    stays at or above tau and verifies [x, d1..d_{depth-1}].

    x: the last emitted token [1] (not yet run through the model) at position
    `pos`; H_last: the model's pre-norm hidden at pos - 1 [1, H]; the MTP cache
    holds every committed position before pos.  trace: record each step's
    drafts (one more host read per step; stochastic steps also keep their
    target and draft logits and record in ``samples``).  A stochastic step
    whose acceptance fails (record [0, 0, 0, -1]: a wait of the sampling
    kernels gave up, or a logit row had no finite value) raises VmiError.
    """
    if model.mtp is None:
        raise VmiError("the model has no MTP layer")
    _check_layout(layout, tau)
    if sampling is not None and (layout != "k+1" or tau is not None):
        raise VmiError("stochastic decoding verifies [x, d1..dK] (layout 'k+1') at a fixed depth")
    st = DecodeStats()
    dev = x.device
    verify = torch.empty(K + 1, dtype=torch.int32, device=dev)
    if sampling is not None:
        V = model.head.shape[0]
        dlog = torch.empty((K, V), dtype=torch.float32, device=dev)
        tlog = torch.empty((K + 1, V), dtype=torch.float32, device=dev)
        status = torch.zeros(1, dtype=torch.int32, device=dev)
    t0 = time.perf_counter()
    while len(st.tokens) < n_tokens:
        mtp_start = drafter.cache.length
        if sampling is not None:
            base = sampling.step_base(st.steps)
            drafts = drafter.draft_sampled(H_last, x, K, temperature=sampling.temperature, top_p=sampling.top_p,
                                           seed=sampling.seed, offset=base, logits_out=dlog, status=status)
        elif tau is not None:
            drafts = drafter.draft_adaptive(H_last, x, K, tau)
        else:
            drafts = drafter.draft(H_last, x, K)
        d = drafts.numel()
        T = d + 1 if layout == "k+1" else d
        verify[0:1].copy_(x)
        verify[1:T].copy_(drafts[:T - 1])
        preds, hid, _ = model.forward(verify[:T], caches, pos, logits_out=tlog if sampling is not None else None)
        if sampling is not None:
            rec = accept_stochastic(tlog, dlog, drafts, temperature=sampling.temperature, top_p=sampling.top_p,
                                    seed=sampling.seed, offset=base + Sampling.ACCEPT_OFFSET, status=status)
        else:
            rec = accept_greedy(drafts, preds, mode=1 if layout == "k+1" else 0)
        r = rec.cpu().tolist()  # the step's one host synchronisation
        if sampling is not None:
            bits = int(status.item())
            raise_sampling_status(bits, f"stochastic decode step {st.steps}")
            if r[3] < 0:
                raise VmiError(f"stochastic decode step {st.steps}: acceptance failed (record {r[:4]})")
            if trace:
                st.samples.append({"offset": base, "target": tlog.cpu().numpy(), "draft": dlog.cpu().numpy(),
                                   "drafts": drafts.cpu().tolist(), "record": r})
        n, m, acc = r[0], r[1], r[2]
        emitted = r[4:4 + n]
        commit_verified_prefix(caches, T, acc)
        # MTP cache: (main hidden at pos-1 .. pos+acc-2, tokens of the acc accepted positions)
        h_seq = torch.cat([H_last, hid[:acc - 1]]) if acc > 1 else H_last
        drafter.sync(mtp_start, h_seq.contiguous(), verify[:acc].contiguous())
        st.tokens.extend(emitted)
        st.accept_hist.append(m)
        st.depths.append(d)
        if trace:
            st.drafts.append(drafts.cpu().tolist())
        st.steps += 1
        pos += acc
        x = torch.tensor([emitted[-1]], dtype=torch.int32, device=dev)
        H_last = hid[acc - 1:acc].clone()
    st.seconds = time.perf_counter() - t0
    st.tokens = st.tokens[:n_tokens]
    return st


def tree_speculative_decode(model: SpecModel, drafter: MTPDrafter, caches, x: torch.Tensor, H_last: torch.Tensor,
                            pos: int, n_tokens: int, K: int = 3, P: int = 3, plant=None, *, mode: str = "paths",
                            pos1: bool = True, tau: Optional[float] = None) -> DecodeStats:
    """Tree verification (tree_verify_step, generate.py:355-420): the MTP
    drafter's paths, each [x, d1..d_{K-1}] (the T = K layout), verified in
    one forward over the paths' tokens (``SpecModel.forward_tree``); the winner
    is the longest matched prefix, ties to the lower path (vmi_accept_greedy,
    generate.py:383); emission and accepted length as accept_prefix's T = K
    rules (generate.py:338-351, 819); the winner's entries are committed into
    every cache in one launch (``TreeCommit``, commit_tree_row,
    kv_cache.py:283-316).  Drafting (mode):
      "paths"          P paths: top-P first tokens, greedy continuations
                       (draft_paths, drafter.py:150-177);
      "tree"           the minimal tree A, B (position-0 rescue) and, with
                       pos1, C (position-1 rescue) (draft_tree,
                       drafter.py:102-148; generate.py:587-588, 764-801);
      "adaptive_tree"  a confidence-gated chain of depth n <= K with tau and,
                       when n >= 2, its position-0 branch (draft_adaptive_tree,
                       drafter.py:64-100; generate.py:592-599, 764-784): the
                       step verifies depth n.
    Verified together, the lowest-index longest match picks the same path as
    the reference's sequential rescue: a branch wins only where the chain
    before it rejected exactly at its fork and the branch's token there is the
    model's.  plant(step, pos) -> rows x K draft tokens replaces the drafts of
    "paths" and "tree" (tests)."""
    if model.mtp is None:
        raise VmiError("the model has no MTP layer")
    if mode not in ("paths", "tree", "adaptive_tree"):
        raise VmiError(f"unknown tree mode {mode!r}")
    if mode == "adaptive_tree" and tau is None:
        raise VmiError("adaptive_tree needs tau")
    width = P if mode == "paths" else (3 if mode == "tree" and pos1 and K >= 2 else 2)
    if width * K > 16:
        raise VmiError(f"a tree of {width} x {K} tokens exceeds 16")
    st = DecodeStats()
    dev = x.device
    commits = {}
    t0 = time.perf_counter()
    while len(st.tokens) < n_tokens:
        mtp_start = drafter.cache.length
        if mode == "paths":
            paths = drafter.draft_paths(H_last, x, K, P)       # [P, K]
            if plant is not None:
                paths.copy_(torch.tensor(plant(st.steps, pos), dtype=torch.int32))
        elif mode == "tree":
            paths = drafter.draft_tree(H_last, x, K, pos1)      # [2 or 3, K]
            if plant is not None:
                paths.copy_(torch.tensor(plant(st.steps, pos), dtype=torch.int32))
        else:
            chain_a, chain_b = drafter.draft_adaptive_tree(H_last, x, K, tau)
            paths = (chain_a.view(1, -1) if chain_b is None else torch.stack([chain_a, chain_b])).contiguous()
        pw, span = paths.shape
        commit = commits.get((pw, span))
        if commit is None:
            commit = commits[(pw, span)] = TreeCommit(caches, pw, span)
        verify = torch.cat([x.view(1, 1).expand(pw, 1), paths[:, :span - 1]], dim=1).contiguous()  # [pw, span]
        preds, hid, _ = model.forward_tree(verify.view(-1), caches, pos, pw)
        rec = accept_greedy(paths, preds, mode=0)
        commit(rec, pos0=pos)
        r = rec.cpu().tolist()  # the step's one host synchronisation
        n, m, acc, best = r[0], r[1], r[2], r[3]
        emitted = r[4:4 + n]
        model.commit(caches, pos + acc)
        w0 = best * span
        h_seq = torch.cat([H_last, hid[w0:w0 + acc - 1]]) if acc > 1 else H_last
        drafter.sync(mtp_start, h_seq.contiguous(), verify[best, :acc].contiguous())
        st.tokens.extend(emitted)
        st.accept_hist.append(m)
        st.depths.append(span)
        st.rescues.append(best)
        st.steps += 1
        pos += acc
        x = torch.tensor([emitted[-1]], dtype=torch.int32, device=dev)
        H_last = hid[w0 + acc - 1:w0 + acc].clone()
    st.seconds = time.perf_counter() - t0
    st.tokens = st.tokens[:n_tokens]
    return st


class GraphSpecDecoder:
    """The speculative decode step of ``speculative_decode`` captured as HIP
    graphs and replayed per step, with every position on the device.

    A step runs: the draft steps of the MTP layer at MTP positions
    mtp_len + i; the verify forward at pos; greedy acceptance
    (``vmi_accept_greedy``); the MTP cache update over all verify rows (main
    hidden at pos-1.., tokens x, d1..) at mtp_len, whose rows past the
    accepted ones lie beyond the committed length and are written over by the
    next step; and the commit (``vmi_spec_commit``): pos += accepted_len,
    mtp_len += accepted_len, x = the last emitted token, H_last = the hidden of
    the last accepted position.  Layouts as ``speculative_decode``:
    "k+1" verifies [x, d1..dK], "k" verifies [x, d1..d_{K-1}].  With a fixed
    depth the whole step is one graph and the host reads the acceptance
    record once per step.  With tau (adaptive depth, layout "k") each draft
    step is its own graph and the verify of each depth 1..K another; the host
    reads each draft's probability to choose the depth, as the reference's
    draft_adaptive does (drafter.py:42-62).  Results equal
    ``speculative_decode`` token for token (the kernels' results do not depend
    on batch composition).  With `sampling` (``Sampling``; layout "k+1", fixed
    depth) each draft step samples its token (vmi_sample_top_p into the verify
    row, the step's logits kept as the draft distribution), the verify
    computes the target logits and vmi_accept_stochastic the record; the
    counter offsets come from a device word that the step advances by 64, so
    replays draw what ``speculative_decode`` with the same Sampling draws.  A
    failed acceptance (record [0, 0, 0, -1]) raises VmiError when the host
    reads that step's record.
    """

    def __init__(self, model: SpecModel, drafter: MTPDrafter, caches: list, K: int = 3, planted: bool = False,
                 layout: str = "k+1", tau: Optional[float] = None, sampling: Optional[Sampling] = None):
        """planted: the verify batch takes its drafts from ``self.planted``
        (int32 [K], written by the host before each replay) instead of the MTP
        layer's, which still runs and keeps its cache; for drafts from another
        source and for tests that force acceptance lengths."""
        if model.mtp is None:
            raise VmiError("the model has no MTP layer")
        _check_layout(layout, tau)
        if sampling is not None and (layout != "k+1" or tau is not None or planted):
            raise VmiError("stochastic decoding verifies [x, d1..dK] (layout 'k+1') at a fixed depth, unplanted")
        self.sampling = sampling
        self.model, self.drafter, self.caches, self.K = model, drafter, caches, K
        self.layout, self.tau = layout, tau
        dev = model.embed.device
        self.dev = dev
        self.state = torch.zeros(2, dtype=torch.int32, device=dev)     # [pos, mtp_len]
        self.pos, self.mtp_len = self.state[0:1], self.state[1:2]
        self.mtp_pos = torch.zeros(K, dtype=torch.int32, device=dev)
        self.steps_ar = torch.arange(K, dtype=torch.int32, device=dev)
        # verify rows [x, d1..dK] hold the step's input token and the drafts the
        # MTP layer writes; row 0 of the MTP update holds H_last
        self.verify = torch.zeros(K + 1, dtype=torch.int32, device=dev)
        self.x, self.drafts = self.verify[0:1], self.verify[1:]
        self.probs = torch.zeros(K, dtype=torch.float32, device=dev)
        # hidden rows of the MTP update: row 0 H_last, rows 1.. the verify
        # forward's hidden, which it writes there itself (one row beyond the
        # update's K + 1 takes the last verify row)
        hext = torch.zeros((K + 2, model.hidden), dtype=torch.bfloat16, device=dev)
        self.hseq, self.hrows = hext[0:K + 1], hext[1:K + 2]
        self.H = self.hseq[0:1]
        self.rec_buf = torch.zeros(4 + K + 1, dtype=torch.int32, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.use_planted = planted
        self.planted = torch.zeros(K, dtype=torch.int32, device=dev)
        if sampling is not None:
            V = model.head.shape[0]
            self.dlog = torch.zeros((K, V), dtype=torch.float32, device=dev)      # draft distributions
            self.tlog = torch.zeros((K + 1, V), dtype=torch.float32, device=dev)  # verify distributions
            self.rng = torch.full((1,), sampling.step_base(0), dtype=torch.int64, device=dev)
        self.stream = torch.cuda.Stream(device=dev)
        self.graph = None        # fixed depth: the whole step
        self.draft_graphs = []   # adaptive: one per draft step
        self.verify_graphs = {}  # adaptive: depth -> verify + accept + commit
        self._keep = []

    def _draft(self, i: int, h: torch.Tensor) -> torch.Tensor:
        tok = self.x if i == 0 else self.drafts[i - 1:i]
        sp = self.sampling
        if sp is not None:
            _, hn, _ = self.model.mtp.step(h, tok, self.drafter.cache, pos_device=self.mtp_pos[i:i + 1],
                                           logits_out=self.dlog[i:i + 1])
            sample_top_p(self.dlog[i:i + 1], temperature=sp.temperature, top_p=sp.top_p, seed=sp.seed, offset=i,
                         offset_device=self.rng, out=self.drafts[i:i + 1], status=self.status)
            return hn
        _, hn, _ = self.model.mtp.step(h, tok, self.drafter.cache, pos_device=self.mtp_pos[i:i + 1],
                                       argmax_out=self.drafts[i:i + 1], prob_out=self.probs[i:i + 1])
        return hn

    def _verify(self, d: int) -> torch.Tensor:
        """Verify, accept and commit after d drafts."""
        T = d + 1 if self.layout == "k+1" else d
        mtp = self.model.mtp
        if self.use_planted:
            self.drafts[:d].copy_(self.planted[:d])
        sp = self.sampling
        preds, hid, _ = self.model.forward(self.verify[:T], self.caches, 0, pos_device=self.pos,
                                           hidden_out=self.hrows[:T], logits_out=self.tlog[:T] if sp else None)
        if sp is not None:
            rec = accept_stochastic(self.tlog[:T], self.dlog[:d], self.drafts[:d], temperature=sp.temperature,
                                    top_p=sp.top_p, seed=sp.seed, offset=Sampling.ACCEPT_OFFSET,
                                    offset_device=self.rng, out=self.rec_buf, status=self.status)
        else:
            rec = accept_greedy(self.drafts[:d], preds, mode=1 if self.layout == "k+1" else 0, out=self.rec_buf)
        mtp.advance(self.hseq[:T], self.verify[:T], self.drafter.cache, pos_device=self.mtp_len)
        spec_commit(rec, hid, self.H, self.x, self.pos, self.mtp_len, self.mtp_pos, rows=T, status=self.status)
        if sp is not None:
            self.rng.add_(64)
        return rec

    def _step(self) -> torch.Tensor:
        h = self.H
        for i in range(self.K):
            h = self._draft(i, h)
        return self._verify(self.K)

    def start(self, x: torch.Tensor, H_last: torch.Tensor, pos: int) -> None:
        """Sets the state: x (int32 [1]) at position pos, H_last [1, H] the
        hidden of pos - 1; the MTP cache length is the drafter's."""
        self.x.copy_(x)
        self.H.copy_(H_last)
        self.state.copy_(torch.tensor([pos, self.drafter.cache.length], dtype=torch.int32))
        torch.add(self.steps_ar, self.mtp_len, out=self.mtp_pos)
        self.pos_host = pos

    def _capture(self, fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            out = fn()
        self._keep.append(out)
        return g, out

    def capture(self) -> None:
        """Warms the workspaces up on the capture stream (every shape the
        graphs use), restores the state, and captures."""
        live = (self.state, self.x, self.H, self.mtp_pos, self.status) + \
            ((self.rng,) if self.sampling is not None else ())
        saved = [t.clone() for t in live]
        self.stream.wait_stream(torch.cuda.current_stream(self.dev))
        # each warm-up starts from the saved state, so none writes a ring slot
        # the real steps read (linear-attention rings hold K + 2 or more states)
        warmups = [self._step] + ([lambda d=d: self._verify(d) for d in range(1, self.K)] if self.tau is not None else [])
        for fn in warmups:
            with torch.cuda.stream(self.stream):
                fn()
                for t, v in zip(live, saved):
                    t.copy_(v)
            self.stream.synchronize()
        torch.cuda.synchronize(self.dev)
        if self.tau is None:
            self.graph, self.rec = self._capture(self._step)
        else:
            h = self.H
            for i in range(self.K):
                g, h = self._capture(lambda i=i, h=h: self._draft(i, h))
                self.draft_graphs.append(g)
            for d in range(1, self.K + 1):
                self.verify_graphs[d], self.rec = self._capture(lambda d=d: self._verify(d))
        torch.cuda.synchronize(self.dev)

    def _replay_step(self) -> None:
        if self.tau is None:
            self.graph.replay()
            self._depth = self.K
            return
        conf = np.float32(1.0)
        d = 0
        for i in range(self.K):
            self.draft_graphs[i].replay()
            d = i + 1
            if i + 1 < self.K:
                conf = np.float32(conf * np.float32(self.probs[i].item()))
                if conf < self.tau:
                    break
        self.verify_graphs[d].replay()
        self._depth = d

    def run(self, n_tokens: int, plant=None, trace: bool = False) -> DecodeStats:
        """Decodes n_tokens tokens by graph replays.  plant(step, pos) -> K
        draft tokens for a decoder made with planted=True; trace records each
        step's drafts (one more host read per step)."""
        if self.graph is None and not self.draft_graphs:
            self.capture()
        K = self.K
        need = self.pos_host + n_tokens + 2 * K + 2  # the last step overshoots by < K + 1 and writes K + 1 rows
        for c in list(self.caches) + [self.drafter.cache]:
            if isinstance(c, KVCache) and need > c.max_len:
                raise VmiError(f"cache capacity {c.max_len} < {need} positions needed")
        st = DecodeStats()
        t0 = time.perf_counter()
        pos = self.pos_host

        def take(r):
            nonlocal pos
            if r[3] < 0:
                bits = int(self.status.item())
                raise_sampling_status(bits, f"graph decode step {st.steps}")
                raise VmiError(f"graph decode step {st.steps}: acceptance failed (record {r[:4]}, status {bits:#x})")
            n, m = r[0], r[1]
            pos += r[2]
            st.tokens.extend(r[4:4 + n])
            st.accept_hist.append(m)
            st.depths.append(self._depth)
            st.steps += 1

        if plant is None and self.tau is None and not trace:
            # one step ahead: each step's record goes to pinned memory in stream
            # order and is read while the next step runs; a step is enqueued
            # ahead only while the pending ones cannot finish the run even if
            # they accept everything, so the run stops where the synchronous
            # loop would
            bufs = [torch.empty(self.rec_buf.shape, dtype=self.rec_buf.dtype).pin_memory() for _ in range(2)]
            evs = [torch.cuda.Event() for _ in range(2)]
            pending = []

            def enqueue():
                i = (pending[-1] + 1) % 2 if pending else 0
                self._replay_step()
                bufs[i].copy_(self.rec_buf, non_blocking=True)
                evs[i].record()
                pending.append(i)

            while len(st.tokens) < n_tokens:
                if not pending:
                    enqueue()
                if len(pending) == 1 and len(st.tokens) + (K + 1) < n_tokens:
                    enqueue()
                i = pending.pop(0)
                evs[i].synchronize()  # the step's one host synchronisation, under the next step
                take(bufs[i].tolist())
        else:
            while len(st.tokens) < n_tokens:
                if plant is not None:
                    self.planted.copy_(torch.tensor(plant(st.steps, pos), dtype=torch.int32), non_blocking=False)
                self._replay_step()
                take(self.rec_buf.cpu().tolist())  # the step's one host synchronisation
                if trace:
                    st.drafts.append(self.drafts[:self._depth].cpu().tolist())
        st.seconds = time.perf_counter() - t0
        st.tokens = st.tokens[:n_tokens]
        pos, mtp_len = self.state.cpu().tolist()
        bits = int(self.status.item())
        if bits:
            raise_sampling_status(bits, "graph decode")
            raise VmiError(f"device status {bits:#x}: an acceptance record was out of range")
        self.pos_host = pos
        for c in self.caches:
            if c is not None:
                c.length = pos
        self.drafter.cache.length = mtp_len
        return st


class GraphGreedyDecoder:
    """Non-speculative greedy decoding (one token per forward) captured as a
    HIP graph: one replay runs the forward of the last token at the position
    held on the device, writes its argmax as the next input and into the
    token log at the step index, and advances the position and the index.
    Replays need no host synchronisation; the host reads the log at the end.
    The like-for-like baseline of ``GraphSpecDecoder``."""

    def __init__(self, model: SpecModel, caches: list, max_tokens: int):
        self.model, self.caches = model, caches
        dev = model.embed.device
        self.dev = dev
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.x = torch.zeros(1, dtype=torch.int32, device=dev)
        self.idx = torch.zeros(1, dtype=torch.int64, device=dev)
        self.log = torch.zeros(max_tokens, dtype=torch.int32, device=dev)
        self.one_i32 = torch.ones(1, dtype=torch.int32, device=dev)
        self.one_i64 = torch.ones(1, dtype=torch.int64, device=dev)
        self.stream = torch.cuda.Stream(device=dev)
        self.graph = None

    def _step(self) -> None:
        am, _, _ = self.model.forward(self.x, self.caches, 0, pos_device=self.pos)
        self.x.copy_(am)
        self.log.index_copy_(0, self.idx, am)
        self.pos.add_(self.one_i32)
        self.idx.add_(self.one_i64)

    def start(self, x: torch.Tensor, pos: int) -> None:
        self.x.copy_(x)
        self.pos.fill_(pos)
        self.idx.zero_()
        self.pos_host = pos

    def capture(self) -> None:
        live = (self.x, self.pos, self.idx)
        saved = [t.clone() for t in live]
        self.stream.wait_stream(torch.cuda.current_stream(self.dev))
        with torch.cuda.stream(self.stream):
            self._step()
            for t, v in zip(live, saved):
                t.copy_(v)
        self.stream.synchronize()
        torch.cuda.synchronize(self.dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self._step()
        torch.cuda.synchronize(self.dev)

    def run(self, n_tokens: int) -> DecodeStats:
        if self.graph is None:
            self.capture()
        if n_tokens > self.log.numel():
            raise VmiError(f"the token log holds {self.log.numel()} tokens")
        for c in self.caches:
            if isinstance(c, KVCache) and self.pos_host + n_tokens > c.max_len:
                raise VmiError(f"cache capacity {c.max_len} < {self.pos_host + n_tokens} positions needed")
        st = DecodeStats()
        torch.cuda.synchronize(self.dev)
        t0 = time.perf_counter()
        for _ in range(n_tokens):
            self.graph.replay()
        torch.cuda.synchronize(self.dev)
        st.seconds = time.perf_counter() - t0
        st.tokens = self.log[:n_tokens].cpu().tolist()
        st.steps = n_tokens
        self.pos_host += n_tokens
        for c in self.caches:
            if c is not None:
                c.length = self.pos_host
        return st
