"""GPU parity of the lm_head GEMV with fused argmax (vmi_lm_head) against the
CPU oracle.

Bars (written here):
  normalised operand and synthetic tensors: bit-exact (shared recipe);
  logits: |gpu - ref| <= 1e-4 * sum|x w| per element against the float64
  oracle (fp32 accumulation of bf16 products), relative L2 <= 1e-6;
  argmax / max logit: bit-exact against the oracle's first-maximum rule applied
  to the GPU's own logits, and equal to the oracle's argmax wherever the
  oracle's top-two margin exceeds the error bound;
  top_prob (softmax probability of the argmax): relative error <= 1e-5
  against 1 / sum exp(l - max l) in float64 over the GPU's own logits (fp32
  exponentials and sums over up to 151,936 terms).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ABS_BOUND = 1e-4


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


from oracle.torch_bridge import u16  # noqa: E402


def _check_head(orc, x, nw, W, logits, am, mx, eps=1e-6):
    xn = u16(x)
    ref, absdot = orc.lm_head(xn, None if nw is None else u16(nw), eps, u16(W))
    got = logits.cpu().numpy().astype(np.float64) if logits is not None else None
    if got is not None:
        err = np.abs(got - ref)
        assert (err <= ABS_BOUND * absdot + 1e-30).all(), f"logit error {err.max():.3g} beyond bound"
        rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
        assert rel <= 1e-6, f"relative L2 {rel:.3g}"
        want = orc.argmax_rows(logits.cpu().numpy())
        assert np.array_equal(am.cpu().numpy(), want), "argmax differs from the first maximum of the GPU logits"
        assert np.array_equal(mx.cpu().numpy().view(np.uint32),
                              logits.cpu().numpy()[np.arange(len(want)), want].view(np.uint32))
    # against the exact logits where the decision is unambiguous
    srt = np.sort(ref, axis=1)
    margin = srt[:, -1] - srt[:, -2]
    bound = 2 * ABS_BOUND * absdot.max(axis=1)
    ref_am = np.argmax(ref, axis=1)
    clear = margin > bound
    assert np.array_equal(am.cpu().numpy()[clear], ref_am[clear])
    return clear.sum()


@pytest.mark.parametrize("T,H,V,norm", [(1, 512, 1000, True), (3, 512, 4099, False), (4, 1024, 2048, True),
                                        (4, 2048, 3001, True), (7, 512, 777, True), (16, 2048, 1601, True),
                                        (16, 512, 16, False)])
def test_lm_head_small(gpu, orc, T, H, V, norm):
    log(f"case: lm_head T={T} H={H} V={V} norm={norm}")
    import torch
    from vates_amd.head import lm_head
    from vates_amd.synth import synth_bf16
    x = synth_bf16(31, 1, (T, H), device=gpu)
    W = synth_bf16(31, 2, (V, H), std=0.02, device=gpu)
    nw = synth_bf16(31, 3, (H,), std=0.1, device=gpu) + 1.0 if norm else None
    logits, am, mx = lm_head(x, W, nw)
    torch.cuda.synchronize()
    _check_head(orc, x, nw, W, logits, am, mx)
    # argmax-only call (no logits written) gives the same answer, twice in a row
    for _ in range(2):
        _, am2, mx2 = lm_head(x, W, nw, want_logits=False)
        torch.cuda.synchronize()
        assert torch.equal(am2, am) and torch.equal(mx2.view(torch.int32), mx.view(torch.int32))


def test_lm_head_ties_nan_and_zero(gpu, orc):
    log("case: lm_head ties / NaN / all-zero rows")
    import torch
    from vates_amd.head import lm_head
    from vates_amd.synth import synth_bf16
    T, H, V = 4, 512, 2000
    x = synth_bf16(32, 1, (T, H), device=gpu)
    W = torch.zeros((V, H), dtype=torch.bfloat16, device=gpu)
    _, am, mx = lm_head(x, W, None)
    torch.cuda.synchronize()
    assert am.tolist() == [0] * T and mx.tolist() == [0.0] * T
    # identical best rows at 1500, 37 and 1999 -> the lowest index wins; a NaN row never wins
    best = x[0].float() / x[0].float().norm()
    for r in (1500, 37, 1999):
        W[r] = best.to(torch.bfloat16)
    W[5] = float("nan")
    logits, am, mx = lm_head(x, W, None)
    torch.cuda.synchronize()
    assert am[0].item() == 37
    lg = logits.cpu().numpy()
    assert np.isnan(lg[:, 5]).all()
    assert np.array_equal(am.cpu().numpy(), orc.argmax_rows(lg))


def test_lm_head_vocab_151936(gpu, orc):
    log("case: lm_head full vocabulary V=151936 H=2048 T=4")
    import torch
    from vates_amd.head import lm_head
    from vates_amd.synth import synth_bf16
    T, H, V = 4, 2048, 151936
    x = synth_bf16(33, 1, (T, H), device=gpu)
    W = synth_bf16(33, 2, (V, H), std=0.02, device=gpu)
    nw = synth_bf16(33, 3, (H,), std=0.1, device=gpu) + 1.0
    logits, am, mx = lm_head(x, W, nw)
    torch.cuda.synchronize()
    clear = _check_head(orc, x, nw, W, logits, am, mx)
    assert clear == T
    # the draft step's shape: one token
    _, am1, _ = lm_head(x[1:2].contiguous(), W, nw, want_logits=False)
    torch.cuda.synchronize()
    assert am1.item() == am[1].item()


@pytest.mark.parametrize("T,V,scale", [(1, 151936, 0.02), (4, 151936, 1.0), (3, 4099, 3.0), (16, 1601, 0.5)])
def test_lm_head_top_prob(gpu, orc, T, V, scale):
    """The fused top-1 probability (draft_adaptive's confidence,
    mlx_streaming/mtp/drafter.py:42-62) against float64 softmax of the GPU's
    logits; the argmax and logits are unchanged by asking for it."""
    log(f"case: lm_head top_prob T={T} V={V} weight std {scale}")
    import torch
    from vates_amd.head import lm_head
    from vates_amd.synth import synth_bf16
    H = 2048
    W = synth_bf16(61, 1, (V, H), std=scale, device=gpu)
    x = synth_bf16(61, 2, (T, H), device=gpu)
    nw = synth_bf16(61, 3, (H,), std=0.1, device=gpu) + 1.0
    p = torch.empty(T, dtype=torch.float32, device=gpu)
    logits, am, mx = lm_head(x, W, nw, top_prob=p)
    logits2, am2, _ = lm_head(x, W, nw)
    torch.cuda.synchronize()
    assert torch.equal(logits, logits2) and torch.equal(am, am2)
    lg = logits.cpu().numpy().astype(np.float64)
    ref = 1.0 / np.exp(lg - lg.max(axis=1, keepdims=True)).sum(axis=1)
    got = p.cpu().numpy().astype(np.float64)
    log(f"  top_prob {got} ref {ref}")
    assert np.all(np.abs(got - ref) <= 1e-5 * ref), (got, ref)



@pytest.mark.gpu
@pytest.mark.parametrize("T,V,norm", [(4, 151936, True), (1, 151936, False), (5, 1000, True), (16, 1003, False)])
def test_lm_head_tiled_equals_row_major(gpu, T, V, norm):
    """vmi_lm_head_tiled on the vmi_head_tiles copy gives vmi_lm_head's logits,
    argmax, maximum and top-1 probability bit for bit, including vocabularies
    that are not a multiple of 16 (the copy's zero padding rows)."""
    import torch
    from vates_amd.head import TiledHead, lm_head
    from vates_amd.synth import synth_bf16
    H = 2048
    log(f"case: tiled head T={T} V={V} norm={norm}")
    W = synth_bf16(31, 0x7100 + V, (V, H), std=0.02, device=gpu)
    x = synth_bf16(31, 0x7200 + T, (T, H), device=gpu)
    nw = synth_bf16(31, 0x7300, (H,), std=0.1, device=gpu) + 1.0 if norm else None
    Wt = TiledHead(W)
    assert Wt.tiles.numel() == ((V + 15) // 16) * 16 * H
    outs = []
    for head in (W, Wt):
        prob = torch.empty(T, dtype=torch.float32, device=gpu)
        lg, am, mx = lm_head(x, head, nw, top_prob=prob)
        torch.cuda.synchronize()
        outs.append((lg.cpu(), am.cpu(), mx.cpu(), prob.cpu()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    # the copy itself: element (v, h) at ((v/16)(H/128) + h/128) 2048 + (v%16) 128 + h%128
    v = torch.arange(V, device=gpu)[:, None]
    h = torch.arange(H, device=gpu)[None, :]
    idx = ((v // 16) * (H // 128) + h // 128) * 2048 + (v % 16) * 128 + h % 128
    assert torch.equal(Wt.tiles[idx.reshape(-1)].reshape(V, H), W)
    Vp = ((V + 15) // 16) * 16
    if Vp > V:  # the padding rows are zeros
        vp = torch.arange(V, Vp, device=gpu)[:, None]
        pidx = ((vp // 16) * (H // 128) + h // 128) * 2048 + (vp % 16) * 128 + h % 128
        assert not Wt.tiles[pidx.reshape(-1)].float().any()
