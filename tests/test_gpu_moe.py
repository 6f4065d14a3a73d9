"""GPU parity of the fused 4-bit MoE (libvmi) against the CPU oracle.

Bars (written here, checked per token):
  integer work (synthetic tensors, dequant, routed ids, slots): bit-exact;
  MoE outputs: relative L2 error <= 1e-2, cosine >= 0.9999 and
  max |err| <= 1e-2 * max |ref| against the oracle's float64 result
  (bf16 activations, fp32 accumulation on the GPU);
  fused_moe_slots / fused_moe_staged with f32 x (the reference operator's
  fp32 arithmetic): relative L2 error and max |err| / max |ref| <= 1e-5.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REL, COS = 1e-2, 0.9999
REL32 = 1e-5


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


from oracle.torch_bridge import layer_np, pool_np, u16, u32  # noqa: E402


def assert_moe_close(got, ref, what, rel_bar=REL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    for t in range(ref.shape[0]):
        g, r = got[t], ref[t]
        rel = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
        cos = float(g @ r / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-30))
        mx = np.abs(g - r).max() / max(np.abs(r).max(), 1e-30)
        assert rel <= rel_bar and cos >= COS and mx <= rel_bar, \
            f"{what} token {t}: rel={rel:.3g} cos={cos:.7f} max={mx:.3g}"


@pytest.fixture(scope="module")
def torch_mod(gpu):
    import torch
    return torch


def test_synth_bit_identical_to_oracle(gpu, orc, torch_mod):
    log("case: synth 4/8-bit and bf16 vs oracle")
    from vates_amd.synth import synth_bf16, synth_proj
    for bits in (4, 8):
        p = synth_proj(21, 5, 3, 40, 512, bits=bits, device=gpu)
        wq, s, b = orc.synth_quantized(21, 5, 120, 512, 64, bits, 0.02)
        assert np.array_equal(u32(p.weight).reshape(wq.shape), wq)
        assert np.array_equal(u16(p.scales).reshape(s.shape), s)
        assert np.array_equal(u16(p.biases).reshape(b.shape), b)
    x = synth_bf16(21, 6, (3, 1001), device=gpu)
    assert np.array_equal(u16(x).reshape(-1), orc.synth_bf16(21, 6, (3003,), 1.0))


def test_dequant_bit_exact(gpu, orc, torch_mod):
    log("case: dequant 4/8-bit vs oracle")
    import ctypes
    torch = torch_mod
    from vates_amd._lib import QMat, check, load
    from vates_amd.synth import synth_proj
    for bits in (4, 8):
        p = synth_proj(22, 1, 1, 96, 2048, bits=bits, device=gpu)
        out = torch.empty((96, 2048), dtype=torch.float32, device=gpu)
        q = QMat(p.weight.data_ptr(), p.scales.data_ptr(), p.biases.data_ptr())
        check(load().vmi_dequant_affine(q, 96, 2048, 64, bits, out.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream), "dequant")
        ref = orc.dequant(u32(p.weight).reshape(96, -1), u16(p.scales).reshape(96, -1),
                          u16(p.biases).reshape(96, -1), 96, 2048, 64, bits)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("H,I", [(2048, 512), (1024, 256), (512, 128), (2048, 128)])
@pytest.mark.parametrize("xdt", ["f32", "bf16"])
def test_fused_moe_slots_parity(gpu, orc, torch_mod, H, I, xdt):
    torch = torch_mod
    from vates_amd import fused_moe_slots
    from vates_amd.synth import synth_proj
    cap, k = 24, 10
    gate = synth_proj(31, 1, cap, I, H, device=gpu)
    up = synth_proj(31, 2, cap, I, H, device=gpu)
    down = synth_proj(31, 3, cap, H, I, device=gpu)
    P = pool_np(gate, up, down)
    rng = np.random.default_rng(H + I)
    for T in (1, 2, 4):
        log(f"case: fused_moe_slots H={H} I={I} x={xdt} T={T}")
        slots = np.stack([rng.choice(cap, size=k, replace=False) for _ in range(T)]).astype(np.int32)
        slots[0, k - 1] = slots[0, 0]  # one slot twice within a token (legal in the reference)
        if T > 1:
            slots[1, :3] = slots[0, :3]  # experts shared across tokens
        scores = rng.random((T, k)).astype(np.float32)
        scores /= scores.sum(1, keepdims=True)
        x32 = rng.normal(size=(T, H)).astype(np.float32)
        if xdt == "bf16":
            xb = orc.f32_to_bf16(x32)
            x_t = torch.from_numpy(xb.view(np.int16)).to(gpu).view(torch.bfloat16)
            x_ref = orc.bf16_to_f32(xb)
        else:
            x_t = torch.from_numpy(x32).to(gpu)
            x_ref = x32
        out = fused_moe_slots(x_t, torch.from_numpy(slots).to(gpu), torch.from_numpy(scores).to(gpu),
                              gate.weight, gate.scales, gate.biases, up.weight, up.scales, up.biases,
                              down.weight, down.scales, down.biases, H, I, 64, 4)
        torch.cuda.synchronize()
        ref = orc.fused_moe_slots(x_ref, slots, scores, P, T, k, H, I, cap)
        assert out.dtype == torch.float32 and tuple(out.shape) == (T, H)
        assert_moe_close(out.cpu().numpy(), ref, f"slots H={H} I={I} {xdt} T={T}",
                         REL32 if xdt == "f32" else REL)


@pytest.mark.parametrize("H,I,T", [(2048, 512, 4), (512, 128, 3)])
def test_fused_moe_staged_equals_identity_slots(gpu, orc, torch_mod, H, I, T):
    """fused_moe_staged (fused_moe.cpp:443-504, 605-633): pair t*k + j reads
    matrix t*k + j of the pre-sliced stacks.  Bit-identical to
    fused_moe_slots with local_slots = 0..T*k-1 on the same stacks, and within
    the MoE bar of the oracle."""
    torch = torch_mod
    from vates_amd import fused_moe_slots, fused_moe_staged
    from vates_amd.synth import synth_proj
    k = 10
    n = T * k
    log(f"case: fused_moe_staged H={H} I={I} T={T}")
    gate = synth_proj(41, 1, n, I, H, device=gpu)
    up = synth_proj(41, 2, n, I, H, device=gpu)
    down = synth_proj(41, 3, n, H, I, device=gpu)
    rng = np.random.default_rng(H + T)
    scores = rng.random((T, k)).astype(np.float32)
    scores /= scores.sum(1, keepdims=True)
    x = rng.normal(size=(T, H)).astype(np.float32)
    xt, st = torch.from_numpy(x).to(gpu), torch.from_numpy(scores).to(gpu)
    w = (gate.weight, gate.scales, gate.biases, up.weight, up.scales, up.biases, down.weight, down.scales,
         down.biases)
    staged = fused_moe_staged(xt, st, *w, H, I, 64, 4)
    ident = torch.arange(n, dtype=torch.int32, device=gpu).view(T, k)
    slots = fused_moe_slots(xt, ident, st, *w, H, I, 64, 4)
    torch.cuda.synchronize()
    assert torch.equal(staged.view(torch.int32), slots.view(torch.int32))
    ref = orc.fused_moe_slots(x, np.arange(n, dtype=np.int32).reshape(T, k), scores, pool_np(gate, up, down), T, k,
                              H, I, n)
    assert_moe_close(staged.cpu().numpy(), ref, f"staged H={H} I={I} T={T}", REL32)


@pytest.mark.parametrize("H,I", [(2048, 512), (1024, 192), (512, 64)])
def test_fused_moe_slots_f32_duplicates(gpu, orc, torch_mod, H, I):
    """f32 x at the reference operator's fp32 precision with repeated slots:
    a slot twice and three times within one token, every one of 16 tokens on
    slot 0 (more tokens on one slot than one LDS chunk holds), and both output
    dtypes (bf16 out = the fp32 result rounded to nearest even)."""
    torch = torch_mod
    from vates_amd import fused_moe_slots
    from vates_amd.synth import synth_proj
    cap, k, T = 12, 10, 16
    gate = synth_proj(35, 1, cap, I, H, device=gpu)
    up = synth_proj(35, 2, cap, I, H, device=gpu)
    down = synth_proj(35, 3, cap, H, I, device=gpu)
    P = pool_np(gate, up, down)
    rng = np.random.default_rng(7 * H + I)
    slots = np.stack([rng.choice(np.arange(1, cap), size=k, replace=False) for _ in range(T)]).astype(np.int32)
    slots[:, 4] = 0
    slots[0, 7] = slots[0, 1]
    slots[3, 2] = slots[3, 8] = slots[3, 9]
    slots[5, :] = slots[5, 0]
    scores = rng.random((T, k)).astype(np.float32)
    scores /= scores.sum(1, keepdims=True)
    x = rng.normal(size=(T, H)).astype(np.float32)
    log(f"case: fused_moe_slots f32 duplicates H={H} I={I} T={T}")
    args = (torch.from_numpy(x).to(gpu), torch.from_numpy(slots).to(gpu), torch.from_numpy(scores).to(gpu),
            gate.weight, gate.scales, gate.biases, up.weight, up.scales, up.biases, down.weight, down.scales,
            down.biases, H, I, 64, 4)
    out = fused_moe_slots(*args)
    outb = fused_moe_slots(*args, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    ref = orc.fused_moe_slots(x, slots, scores, P, T, k, H, I, cap)
    assert_moe_close(out.cpu().numpy(), ref, f"f32 duplicates H={H} I={I}", REL32)
    assert np.array_equal(u16(outb).reshape(T, H), orc.f32_to_bf16(out.cpu().numpy()))


def test_fused_moe_slots_slot_pool_fixture(gpu, orc, torch_mod):
    """The reference's slot-pool known answer (test_native_moe_ext.py:50-72):
    a 4-slot pool acquiring experts [1, 2, 1] gives local slots [0, 1, 0], then
    [2, 1] gives [1, 0].  With those pool slots holding experts 1 and 2, the
    operator on the local slots equals the oracle on the expert ids of the full
    stack (the call repeats expert 1 within one token)."""
    import json
    from pathlib import Path
    torch = torch_mod
    from vates_amd import fused_moe_slots
    from vates_amd.synth import synth_proj
    fx = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())["slot_pool"]
    H, I, E = 512, 128, 8
    gate = synth_proj(33, 1, E, I, H, device=gpu)
    up = synth_proj(33, 2, E, I, H, device=gpu)
    down = synth_proj(33, 3, E, H, I, device=gpu)
    full = pool_np(gate, up, down)
    cap = fx["cap"]
    held = {}  # slot -> expert, as the fixture's acquisitions fill the pool
    for ids, local in zip(fx["calls"], fx["local"]):
        for e, s in zip(ids, local):
            assert held.setdefault(s, e) == e
    order = [held.get(s, 0) for s in range(cap)]
    pool = [t[order].contiguous() for t in (gate.weight, gate.scales, gate.biases, up.weight, up.scales,
                                            up.biases, down.weight, down.scales, down.biases)]
    rng = np.random.default_rng(9)
    for ids, local in zip(fx["calls"], fx["local"]):
        log(f"case: slot pool fixture experts {ids} -> slots {local}")
        k = len(ids)
        x = rng.normal(size=(1, H)).astype(np.float32)
        scores = rng.random((1, k)).astype(np.float32)
        out = fused_moe_slots(torch.from_numpy(x).to(gpu), torch.tensor([local], dtype=torch.int32, device=gpu),
                              torch.from_numpy(scores).to(gpu), *pool, H, I, 64, 4)
        torch.cuda.synchronize()
        ref = orc.fused_moe_slots(x, np.array([ids], np.int32), scores, full, 1, k, H, I, E)
        assert_moe_close(out.cpu().numpy(), ref, f"slot pool {ids}", REL32)


def test_fused_moe_slots_bad_slot_flags_and_skips(gpu, orc, torch_mod):
    log("case: fused_moe_slots with an out-of-range slot")
    torch = torch_mod
    from vates_amd import fused_moe_slots
    from vates_amd.moe import workspace, workspace_status
    from vates_amd.synth import synth_proj
    H, I, cap, k, T = 512, 128, 8, 4, 2
    gate = synth_proj(32, 1, cap, I, H, device=gpu)
    up = synth_proj(32, 2, cap, I, H, device=gpu)
    down = synth_proj(32, 3, cap, H, I, device=gpu)
    P = pool_np(gate, up, down)
    slots = np.array([[0, 1, 2, 3], [4, cap, 6, -1]], np.int32)
    scores = np.full((T, k), 0.25, np.float32)
    x = np.random.default_rng(3).normal(size=(T, H)).astype(np.float32)
    out = fused_moe_slots(torch.from_numpy(x).to(gpu), torch.from_numpy(slots).to(gpu),
                          torch.from_numpy(scores).to(gpu), gate.weight, gate.scales, gate.biases, up.weight,
                          up.scales, up.biases, down.weight, down.scales, down.biases, H, I, 64, 4)
    from vates_amd._lib import VMI_STATUS_BAD_SLOT, load
    ws = workspace(load().vmi_fused_moe_slots_workspace_bytes(T, k, H, I), gpu,
                   torch.cuda.current_stream().cuda_stream)
    assert workspace_status(ws) & VMI_STATUS_BAD_SLOT
    ok = slots.copy()
    sc = scores.copy()
    sc[slots < 0] = 0.0
    sc[slots >= cap] = 0.0
    ok[(slots < 0) | (slots >= cap)] = 0
    ref = orc.fused_moe_slots(x, ok, sc, P, T, k, H, I, cap)
    assert_moe_close(out.cpu().numpy(), ref, "bad slot", REL32)
    assert workspace_status(ws) == 0


def _layer_case(gpu, orc, torch, T, *, zipf_alpha=1.0, router_bits=8, norm=True, residual=True, H=2048, I=512,
                E=512, k=10, seed=41, layer=0, with_norm=True):
    from vates_amd.synth import synth_bf16
    from vates_amd.workload import make_layer, synth_layer
    w = synth_layer(seed, layer, hidden=H, inter=I, num_experts=E, router_bits=router_bits, zipf_alpha=zipf_alpha,
                    with_norm=with_norm, device=gpu)
    moe = make_layer(w, top_k=k, norm_topk_prob=norm)
    x = synth_bf16(seed, 1000 + T, (T, H), device=gpu)
    ids = torch.empty((T, k), dtype=torch.int32, device=gpu)
    sc = torch.empty((T, k), dtype=torch.float32, device=gpu)
    out = moe(x, residual=x if residual else None, ids_out=ids, scores_out=sc)
    torch.cuda.synchronize()
    L = layer_np(w, k, norm)
    ref_f32, ref_bf16, rid, rsc, rsl = orc.moe_layer(u16(x), L, residual=residual)
    return moe, x, out, ids, sc, ref_f32, rid, rsc


@pytest.mark.parametrize("T", [1, 4, 6, 9, 16])
def test_moe_layer_parity(gpu, orc, torch_mod, T):
    torch = torch_mod
    for residual in (False, True):
        log(f"case: moe_layer full size T={T} residual={residual}")
        moe, x, out, ids, sc, ref, rid, rsc = _layer_case(gpu, orc, torch, T, residual=residual)
        assert np.array_equal(ids.cpu().numpy(), rid), "routed expert ids differ from the oracle"
        np.testing.assert_allclose(sc.cpu().numpy(), rsc, rtol=2e-6, atol=1e-7)
        got = orc.bf16_to_f32(u16(out).reshape(T, -1))
        # without the residual the output is the MoE term itself (bf16-rounded)
        assert_moe_close(got, ref, f"layer T={T} residual={residual}")


def test_moe_layer_variants(gpu, orc, torch_mod):
    torch = torch_mod
    for kw in (dict(zipf_alpha=0.0, router_bits=4, norm=False, residual=False, with_norm=False),
               dict(zipf_alpha=2.0, residual=False, H=1024, I=256, E=128, k=8),
               dict(zipf_alpha=0.5, residual=True, H=512, I=192, E=64, k=6, with_norm=False)):
        log(f"case: moe_layer variant {kw}")
        moe, x, out, ids, sc, ref, rid, rsc = _layer_case(gpu, orc, torch, 4, **kw)
        assert np.array_equal(ids.cpu().numpy(), rid)
        np.testing.assert_allclose(sc.cpu().numpy(), rsc, rtol=2e-6, atol=1e-7)
        got = orc.bf16_to_f32(u16(out).reshape(4, -1))
        assert_moe_close(got, ref, f"variant {kw}")


def test_moe_layer_repeatable_bitwise(gpu, orc, torch_mod):
    log("case: moe_layer repeat determinism")
    torch = torch_mod
    moe, x, out, ids, sc, ref, rid, rsc = _layer_case(gpu, orc, torch, 4)
    outs = [moe(x, residual=x).clone() for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o.view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("T", [4, 6, 9, 16])
def test_moe_layer_batch_invariant(gpu, orc, torch_mod, T):
    """Every token's output equals its output in a batch of one, bit for bit:
    each token adds its experts in its own rank order (speculative decoding
    emits tokens from verify rows 1..K and must reproduce one-token decoding)."""
    log(f"case: moe_layer batch invariance T={T}")
    torch = torch_mod
    for kw in (dict(), dict(zipf_alpha=2.0, H=1024, I=256, E=128, k=8)):
        moe, x, out, ids, sc, ref, rid, rsc = _layer_case(gpu, orc, torch, T, **kw)
        singles = torch.cat([moe(x[t:t + 1].contiguous(), residual=x[t:t + 1].contiguous()) for t in range(T)])
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), singles.view(torch.int16)), kw


def test_moe_layer_router_ties(gpu, orc, torch_mod):
    """All router logits equal: the top-k is experts 0..k-1, lower index first
    on ties (the oracle's rule, generate.py:383's convention), in every token."""
    log("case: moe_layer with tied router logits")
    torch = torch_mod
    from vates_amd.synth import synth_bf16
    from vates_amd.workload import make_layer, synth_layer
    k, T = 10, 4
    w = synth_layer(44, 0, device=gpu)
    w.router.weight.zero_()
    w.router.scales.zero_()
    w.router.biases.zero_()
    moe = make_layer(w, top_k=k)
    x = synth_bf16(44, 1, (T, 2048), device=gpu)
    ids = torch.empty((T, k), dtype=torch.int32, device=gpu)
    sc = torch.empty((T, k), dtype=torch.float32, device=gpu)
    out = moe(x, residual=x, ids_out=ids, scores_out=sc)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), np.tile(np.arange(k), (T, 1)))
    np.testing.assert_allclose(sc.cpu().numpy(), 1.0 / k, rtol=1e-6)
    L = layer_np(w, k, True)
    ref, _, rid, _, _ = orc.moe_layer(u16(x), L, residual=True)
    assert np.array_equal(rid, ids.cpu().numpy())
    assert_moe_close(orc.bf16_to_f32(u16(out).reshape(T, -1)), ref, "tied router")
