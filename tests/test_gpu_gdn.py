"""GPU parity of the Gated DeltaNet block (vmi_gdn_layer) against the CPU oracle.

Bars (written here): block outputs relative L2 <= 1e-2, cosine >= 0.9999 and
max |err| <= 1e-2 max |ref| per token against the float64 oracle (bf16 conv
inputs, fp32 recurrence); captured states relative L2 <= 1e-2 per v-head;
conv rows within one bf16 ulp of the oracle's exact values plus the GEMV's
fp32 error (1e-5 of the row maximum); a T-token call equals T
one-token calls bit for bit (outputs, conv rows, every captured state: the
reference's multistate invariant, tests/test_gated_delta_multistate.py:29-57);
continuing after a commit of m < T positions equals a run that only ever saw
the committed positions, bit for bit.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
REL, COS = 1e-2, 0.9999


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


from oracle.torch_bridge import u16, u32  # noqa: E402


def assert_close(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    for t in range(ref.shape[0]):
        g, r = got[t].ravel(), ref[t].ravel()
        rel = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
        cos = float(g @ r / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-30))
        mx = np.abs(g - r).max() / max(np.abs(r).max(), 1e-30)
        assert rel <= REL and cos >= COS and mx <= REL, f"{what} row {t}: rel={rel:.3g} cos={cos:.7f} max={mx:.3g}"


def make_gdn(gpu, seed, H=2048, n_k=16, n_v=32):
    from vates_amd.workload import synth_gdn
    layer = synth_gdn(seed, 3, hidden=H, n_k_heads=n_k, n_v_heads=n_v, device=gpu)
    qkvz, ba, out, inn, conv, A_log, dt_bias, nw = layer._keep
    G = {"H": H, "n_k": n_k, "n_v": n_v, "dk": 128, "dv": 128, "eps": 1e-6, "bits": 4, "in_norm": u16(inn),
         "conv_w": u16(conv).reshape(-1, 4), "A_log": A_log.cpu().numpy(), "dt_bias": dt_bias.cpu().numpy(),
         "norm_w": u16(nw)}
    for name, p in (("qkvz", qkvz), ("ba", ba), ("out", out)):
        G[name + "_w"], G[name + "_s"], G[name + "_b"] = u32(p.weight), u16(p.scales), u16(p.biases)
    return layer, G


def _state_np(cache, pos):
    return cache.state_before(pos).double().cpu().numpy()


def _conv_np(orc, cache, pos):
    return orc.bf16_to_f32(u16(cache.conv_rows(pos))).astype(np.float64)


@pytest.mark.parametrize("T,prefix", [(1, 0), (4, 0), (8, 0), (4, 5), (1, 13), (4, 35)])
def test_gdn_layer_parity(gpu, orc, T, prefix):
    log(f"case: gdn layer H=2048 16/32 heads T={T} after {prefix} positions")
    import torch
    from vates_amd.synth import synth_bf16
    layer, G = make_gdn(gpu, 91)
    cache = layer.new_cache(8)
    for s in range(0, prefix, 8):
        n = min(8, prefix - s)
        layer(synth_bf16(91, 100 + s, (n, 2048), device=gpu), cache)
    torch.cuda.synchronize()
    assert cache.length == prefix
    conv_in, state_in = _conv_np(orc, cache, prefix), _state_np(cache, prefix)
    x = synth_bf16(91, 7 + T, (T, 2048), device=gpu)
    out = layer(x, cache)
    torch.cuda.synchronize()
    ref, rows, states = orc.gdn_layer(u16(x), G, conv_in=conv_in, state_in=state_in if prefix else None)
    assert_close(orc.bf16_to_f32(u16(out).reshape(T, -1)), ref, f"gdn out T={T}")
    for t in range(T):
        got = _state_np(cache, prefix + t + 1)
        assert_close(got, states[t], f"state after token {t}")
    got_rows = orc.bf16_to_f32(u16(cache.conv_rows(prefix + T))).astype(np.float64)
    want = rows[-3:] if T >= 3 else np.concatenate([conv_in[T:], rows])
    # the GPU rounds its fp32 GEMV result to bf16: one bf16 ulp (2^-7 relative) from the exact value,
    # plus the GEMV's fp32 accumulation error, bounded per row (1e-5 of the row's largest value)
    bound = 2.0 ** -7 * np.abs(want) + 1e-5 * np.abs(want).max(axis=1, keepdims=True)
    assert np.all(np.abs(got_rows - want) <= bound)


def test_gdn_batch_equals_steps(gpu):
    log("case: gdn T=4 batch vs four single-token steps, bit for bit")
    import torch
    from vates_amd.synth import synth_bf16
    layer, _ = make_gdn(gpu, 92)
    c1, c2 = layer.new_cache(8), layer.new_cache(8)
    pre = synth_bf16(92, 1, (6, 2048), device=gpu)
    layer(pre, c1)
    layer(pre, c2)
    x = synth_bf16(92, 2, (4, 2048), device=gpu)
    batch = layer(x, c1)
    steps = torch.cat([layer(x[t:t + 1].contiguous(), c2) for t in range(4)])
    torch.cuda.synchronize()
    assert torch.equal(batch.view(torch.int16), steps.view(torch.int16))
    for p in range(7, 11):
        assert torch.equal(c1.state_before(p), c2.state_before(p)), p
    assert torch.equal(c1.conv_rows(10).view(torch.int16), c2.conv_rows(10).view(torch.int16))


def test_gdn_commit_prefix(gpu):
    log("case: gdn verify 4, commit 2, continue == a run over the committed positions")
    import torch
    from vates_amd.synth import synth_bf16
    layer, _ = make_gdn(gpu, 93)
    a, b = layer.new_cache(8), layer.new_cache(8)
    pre = synth_bf16(93, 1, (5, 2048), device=gpu)
    x = synth_bf16(93, 2, (4, 2048), device=gpu)
    nxt = synth_bf16(93, 3, (4, 2048), device=gpu)
    layer(pre, a)
    layer(x, a)          # verify 4 positions
    a.length = 5 + 2     # accept 2 of them
    ya = layer(nxt, a)
    layer(pre, b)
    layer(x[:2].contiguous(), b)
    yb = layer(nxt, b)
    torch.cuda.synchronize()
    assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))
    assert torch.equal(a.state_before(11), b.state_before(11))


def test_gdn_rejects_bad_arguments(gpu):
    from vates_amd._lib import VmiError
    from vates_amd.synth import synth_bf16
    layer, _ = make_gdn(gpu, 94)
    cache = layer.new_cache(2)   # 3 slots: at most 2 tokens per call
    with pytest.raises(VmiError, match="n_slots"):
        layer(synth_bf16(94, 1, (4, 2048), device=gpu), cache)
    with pytest.raises(VmiError, match="T="):
        layer(synth_bf16(94, 1, (9, 2048), device=gpu), layer.new_cache(16))


def test_gdn_position_on_device(gpu):
    """pos_device gives the result and rings of the host position, bit for bit."""
    import torch
    from vates_amd.synth import synth_bf16
    layer, _ = make_gdn(gpu, 95)
    c1, c2 = layer.new_cache(8), layer.new_cache(8)
    pre = synth_bf16(95, 1, (7, 2048), device=gpu)
    layer(pre, c1)
    layer(pre, c2)
    x = synth_bf16(95, 2, (4, 2048), device=gpu)
    a = layer(x, c1)
    b = layer(x, c2, pos_device=torch.tensor([7], dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(c1.state, c2.state)
    assert torch.equal(c1.conv.view(torch.int16), c2.conv.view(torch.int16))
