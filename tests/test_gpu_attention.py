"""GPU parity of the quantised GEMV and the full-attention block against the
CPU oracle (float64).

Bars (written here): GEMV outputs relative L2 <= 1e-5 per token (fp32
accumulation of exact dequantised weights times bf16 inputs); attention block
outputs relative L2 <= 1e-2, cosine >= 0.9999 and max |err| <= 1e-2 max |ref|
per token (bf16 q, k, v, p operands, fp32 accumulation); appended cache
entries within bf16 rounding (|err| <= 2^-7 max |value| per head vector); a T=4 verify batch
equals four one-token steps bit for bit (outputs and caches).
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
        g, r = got[t], ref[t]
        rel = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
        cos = float(g @ r / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-30))
        mx = np.abs(g - r).max() / max(np.abs(r).max(), 1e-30)
        assert rel <= REL and cos >= COS and mx <= REL, f"{what} token {t}: rel={rel:.3g} cos={cos:.7f} max={mx:.3g}"


@pytest.mark.parametrize("bits", [4, 8])
def test_qgemv_parity(gpu, orc, bits):
    import torch
    from vates_amd.attention import qgemv
    from vates_amd.synth import synth_bf16, synth_proj
    # K in {512, 1024, 2048, 4096} at 4 bits takes the MFMA kernel, K = 1536 the per-row one
    for T, K, N in ((1, 2048, 1000), (4, 2048, 9216), (8, 4096, 256), (3, 512, 64), (2, 1536, 100), (5, 1024, 48)):
        log(f"case: qgemv bits={bits} T={T} K={K} N={N}")
        w = synth_proj(71, 1, 1, N, K, bits=bits, device=gpu)
        x = synth_bf16(71, 2, (T, K), device=gpu)
        y = qgemv(x, w, bits=bits)
        res = synth_bf16(71, 3, (T, N), device=gpu)
        yb = torch.empty((T, N), dtype=torch.bfloat16, device=gpu)
        qgemv(x, w, bits=bits, residual=res, out_bf16=yb)
        torch.cuda.synchronize()
        ref = orc.qgemv_f64(u32(w.weight).reshape(N, -1), u16(w.scales).reshape(N, -1),
                            u16(w.biases).reshape(N, -1), N, K, orc.bf16_to_f32(u16(x)), bits=bits)
        got = y.cpu().numpy().astype(np.float64)
        for t in range(T):
            assert np.linalg.norm(got[t] - ref[t]) <= 1e-5 * np.linalg.norm(ref[t])
        want_b = orc.bf16_to_f32(u16(res).reshape(T, N)).astype(np.float64) + got
        assert np.abs(orc.bf16_to_f32(u16(yb).reshape(T, N)) - want_b).max() <= 2 ** -7 * np.abs(want_b).max()


def test_qgemv_batch_invariant(gpu):
    """A token's result does not depend on the other tokens of its batch (bit for bit)."""
    import torch
    from vates_amd.attention import qgemv
    from vates_amd.synth import synth_bf16, synth_proj
    for K, N in ((2048, 12352), (4096, 2048)):
        log(f"case: qgemv batch invariance K={K} N={N}")
        w = synth_proj(72, 1, 1, N, K, device=gpu)
        x = synth_bf16(72, 2, (4, K), device=gpu)
        x[2] *= 1000.0   # a token with a different range factor must not move the others
        y = qgemv(x, w)
        ys = torch.cat([qgemv(x[t:t + 1].contiguous(), w) for t in range(4)])
        torch.cuda.synchronize()
        assert torch.equal(y, ys)


def make_attention(gpu, seed, H=2048, n_heads=16, n_kv=2):
    import torch
    from vates_amd.attention import AttentionLayer
    from vates_amd.synth import synth_bf16, synth_proj
    q = synth_proj(seed, 1, 1, n_heads * 512, H, device=gpu)
    k = synth_proj(seed, 2, 1, n_kv * 256, H, device=gpu)
    v = synth_proj(seed, 3, 1, n_kv * 256, H, device=gpu)
    o = synth_proj(seed, 4, 1, H, n_heads * 256, device=gpu)
    inn = (synth_bf16(seed, 5, (H,), std=0.1, device=gpu).float() + 1.0).to(torch.bfloat16)
    qn = (synth_bf16(seed, 6, (256,), std=0.1, device=gpu).float() + 1.0).to(torch.bfloat16)
    kn = (synth_bf16(seed, 7, (256,), std=0.1, device=gpu).float() + 1.0).to(torch.bfloat16)
    layer = AttentionLayer(q, k, v, o, inn, qn, kn, n_heads=n_heads, n_kv_heads=n_kv)
    A = {"H": H, "n_heads": n_heads, "n_kv": n_kv, "rope_dim": 64, "theta": 1e7, "eps": 1e-6, "bits": 4,
         "in_norm": u16(inn), "q_norm": u16(qn), "k_norm": u16(kn)}
    for name, p in (("q", q), ("k", k), ("v", v), ("o", o)):
        A[name + "_w"], A[name + "_s"], A[name + "_b"] = u32(p.weight), u16(p.scales), u16(p.biases)
    return layer, A


# Capacities up to 32,768 positions split the keys into 256-key chunks; 33,376 into 288-key chunks
# (9 blocks: 2 x 116 chunks fit 256 CUs) and 40,960 into 320-key chunks (10 blocks), where the
# batch's keys land in a chunk's extra blocks (positions 288c + 256.., 320c + 256..) or straddle a
# chunk boundary (33,120 = 115 x 288).
@pytest.mark.parametrize("T,pos0,max_len", [(1, 0, 256), (4, 0, 256), (1, 63, 256), (4, 200, 512), (4, 1000, 2048),
                                            (1, 4095, 4096), (4, 30000, 32768), (4, 33090, 33376),
                                            (4, 33118, 33376), (1, 39000, 40960), (4, 39006, 40960)])
def test_attention_layer_parity(gpu, orc, T, pos0, max_len):
    log(f"case: attention layer H=2048 16/2 heads T={T} pos0={pos0} max_len={max_len}")
    import torch
    from vates_amd.synth import synth_bf16
    layer, A = make_attention(gpu, 81)
    cache = layer.new_cache(max_len)
    if pos0:
        cache.write(0, synth_bf16(81, 20, (2, pos0, 256), device=gpu), synth_bf16(81, 21, (2, pos0, 256), device=gpu))
    x = synth_bf16(81, 22 + T, (T, 2048), device=gpu)
    kc0, vc0 = u16(cache.keys(0, pos0 + T)).copy(), u16(cache.values(0, pos0 + T)).copy()
    raw_k0 = cache.k.clone()
    out = layer(x, cache, pos0=pos0)
    torch.cuda.synchronize()
    assert cache.length == pos0 + T
    ref, kn, vn = orc.attention_layer(u16(x), A, pos0, kc0, vc0)
    assert_close(orc.bf16_to_f32(u16(out).reshape(T, -1)), ref, f"attention T={T} pos0={pos0}")
    kg = orc.bf16_to_f32(u16(cache.keys(pos0, pos0 + T)).reshape(2, T, 256)).transpose(1, 0, 2)
    vg = orc.bf16_to_f32(u16(cache.values(pos0, pos0 + T)).reshape(2, T, 256)).transpose(1, 0, 2)
    # bf16 cache entries: the key is rounded after the norm and again after the rotation, so a
    # small rotated value carries the rounding of its larger partner: bound per head vector
    for got_c, ref_c in ((kg, kn), (vg, vn)):
        err = np.abs(got_c - ref_c).max(axis=2)
        assert np.all(err <= 2 ** -7 * np.abs(ref_c).max(axis=2)), err
    # untouched cache entries stay: only the storage of positions pos0..pos0+T-1 changed
    assert np.array_equal(u16(cache.keys(0, pos0)), kc0[:, :pos0])
    changed = (cache.k.view(torch.int16) != raw_k0.view(torch.int16)).any(dim=2).cpu().numpy()  # [n_kv, blocks]
    touched = np.zeros_like(changed)
    touched[:, pos0 // 32:(pos0 + T - 1) // 32 + 1] = True
    assert not changed[~touched].any()


@pytest.mark.parametrize("pos0,max_len", [(500, 1024), (33117, 33376), (39005, 40960)])
def test_attention_batch_equals_steps(gpu, orc, pos0, max_len):
    log(f"case: attention T=4 batch vs four single-token steps pos0={pos0} max_len={max_len}")
    import torch
    from vates_amd.synth import synth_bf16
    layer, A = make_attention(gpu, 82)
    c1, c2 = layer.new_cache(max_len), layer.new_cache(max_len)
    pre_k = synth_bf16(82, 20, (2, pos0, 256), device=gpu)
    pre_v = synth_bf16(82, 21, (2, pos0, 256), device=gpu)
    for c in (c1, c2):
        c.write(0, pre_k, pre_v)
        c.length = pos0
    x = synth_bf16(82, 30, (4, 2048), device=gpu)
    batch = layer(x, c1)
    steps = torch.cat([layer(x[t:t + 1].contiguous(), c2) for t in range(4)])
    torch.cuda.synchronize()
    assert torch.equal(c1.k.view(torch.int16), c2.k.view(torch.int16))
    assert torch.equal(c1.v.view(torch.int16), c2.v.view(torch.int16))
    # keys in chunks at fixed positions and per-row MFMA results: bit-identical
    assert torch.equal(batch.view(torch.int16), steps.view(torch.int16)), "batch result differs from single steps"


@pytest.mark.parametrize("pos0,max_len", [(700, 1024), (33100, 33376)])
def test_attention_position_on_device(gpu, pos0, max_len):
    """pos_device gives the result and cache of the host position, bit for bit
    (every chunk of the capacity launched, those past the cache exiting)."""
    log(f"case: attention position on the device pos0={pos0} max_len={max_len}")
    import torch
    from vates_amd.synth import synth_bf16
    layer, _ = make_attention(gpu, 83)
    c1, c2 = layer.new_cache(max_len), layer.new_cache(max_len)
    pk, pv = synth_bf16(83, 20, (2, pos0, 256), device=gpu), synth_bf16(83, 21, (2, pos0, 256), device=gpu)
    c1.write(0, pk, pv)
    c2.write(0, pk, pv)
    x = synth_bf16(83, 30, (4, 2048), device=gpu)
    a = layer(x, c1, pos0=pos0)
    b = layer(x, c2, pos0=0, pos_device=torch.tensor([pos0], dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(c1.k.view(torch.int16), c2.k.view(torch.int16))
    assert torch.equal(c1.v.view(torch.int16), c2.v.view(torch.int16))


@pytest.mark.parametrize("pos0,max_len", [(1000, 2048), (33090, 33376), (39005, 40960)])
def test_attention_tree_equals_paths(gpu, pos0, max_len):
    """The block over a tree of 3 paths x 3 tokens equals each path run alone
    on a copy of the cache, bit for bit: outputs, and the path's new keys and
    values against the entries the single-path call wrote (256-, 288- and
    320-key chunks)."""
    log(f"case: attention tree 3 x 3 vs paths pos0={pos0} max_len={max_len}")
    import torch
    from vates_amd.synth import synth_bf16
    layer, _ = make_attention(gpu, 84)
    P, S = 3, 3
    base = layer.new_cache(max_len)
    base.write(0, synth_bf16(84, 20, (2, pos0, 256), device=gpu), synth_bf16(84, 21, (2, pos0, 256), device=gpu))
    base.length = pos0
    x = synth_bf16(84, 30, (P * S, 2048), device=gpu)
    out_t = layer.tree(x, base, P, pos0=pos0)
    tkv = base.tree_kv.clone()
    torch.cuda.synchronize()
    for p in range(P):
        c = layer.new_cache(max_len)
        c.k.copy_(base.k)
        c.v.copy_(base.v)
        c.length = pos0
        o = layer(x[p * S:(p + 1) * S].contiguous(), c, pos0=pos0)
        torch.cuda.synchronize()
        assert torch.equal(out_t[p * S:(p + 1) * S].view(torch.int16), o.view(torch.int16)), f"path {p}: output"
        assert torch.equal(tkv[p, :, 0].view(torch.int16), c.keys(pos0, pos0 + S).view(torch.int16)), f"path {p}: keys"
        assert torch.equal(tkv[p, :, 1].view(torch.int16), c.values(pos0, pos0 + S).view(torch.int16)), f"path {p}: values"
