#!/usr/bin/env python3
"""Verify-batch fused 4-bit MoE benchmark on one MI355X.

Workload (one "step"): a 48-layer MoE-only stack in verify mode, T=4 tokens
(the K=3 speculative verify batch), every layer a Qwen3-Next MoE block
(hidden 2048, 512 routed SwiGLU experts of intermediate 512, softmax top-10
with renormalised scores, 8-bit router, 4-bit MLX-affine g64 experts
addressed through a 512-slot pool table, sigmoid-gated 4-bit shared expert)
with a residual connection x <- x + MoE(x).  Router logits carry a Zipf(1.1)
per-layer expert-popularity bias (alpha 0.5) so that about 30 distinct experts
are touched per layer per step.  All ~43.7 GB of weights are resident in HBM.
Every step feeds fresh synthetic N(0,1) bf16 activations.

Prints one JSON line.  value = algorithmic HBM bytes of all timed steps /
timed seconds (GB/s); bytes per layer = U*1,769,472 (distinct routed experts)
+ 1,769,472 (shared expert) + 1,114,112 (8-bit router) + 2,176 (8-bit shared
gate) + 3*T*hidden*2 (x, residual, out).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "K=3 MTP decode tokens/s; fused 4-bit MoE verify HBM GB/s vs peak"
PEAK_HBM_GBS = 8000.0
EXPERT_BYTES = 3 * (512 * 2048 // 2 + 2 * 512 * 32 * 2)  # 1,769,472
ROUTER8_BYTES = 512 * 2048 + 2 * 512 * 32 * 2  # 1,114,112
SGATE8_BYTES = 2048 + 2 * 32 * 2  # 2,176
SEED = 1234
ZIPF_S, ZIPF_ALPHA = 1.1, 0.5
# HBM bytes a layer call of the MoE stack moves per algorithmic byte, measured
# by rocprofv3 counter passes (profiles/moe_layer_48x_T4_traffic.md) over
# `--layers 8 --steps 3 --warmup 1 --no-graph --no-decode --no-ceiling`:
# FETCH_SIZE summed over the layer's kernels, scaled by what the counter reads
# for a plain copy of known size (bench.py --path copy), plus WRITE_SIZE
# likewise, divided by those calls' algorithmic bytes.  The line reports
# roofline.traffic = this ratio x this run's algorithmic bytes per call.
MOE_TRAFFIC_RATIO = 1.0585
MOE_TRAFFIC_SOURCE = ("profiles/moe_layer_48x_T4_traffic.md: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE over 34 layer "
                      "calls, scaled by a 512 MiB copy (x2.000 / x1.000): 61,948,825 B against 58,525,824 "
                      "algorithmic B (expert weights x1.003; 2.9 MB of bf16 split-K partial rows written and re-read)")


def eprint(*a):
    print(*a, file=sys.stderr, flush=True)


def layer_bytes(U: np.ndarray, T: int, H: int) -> np.ndarray:
    return U.astype(np.float64) * EXPERT_BYTES + EXPERT_BYTES + ROUTER8_BYTES + SGATE8_BYTES + 3 * T * H * 2


def _threads_label(threads: int) -> int:
    avail = len(os.sched_getaffinity(0))
    return min(threads, avail) if threads > 0 else min(int(os.environ.get("OMP_NUM_THREADS", "0")) or avail, avail)


def cpu_baseline(layers_w, x_bank, args, budget_s: float, threads: int = 0):
    """Times the CPU oracle (OpenMP, float64 accumulation) on a bounded sample of
    the same workload: the first layers' weights copied to host, fed with the
    first steps' activations, until `budget_s` seconds of CPU work.  threads:
    OpenMP threads (0: all the process may use)."""
    from oracle import oracle as orc
    from oracle.torch_bridge import layer_np

    n_layers = min(2, len(layers_w))
    Ls = [layer_np(layers_w[i], args.top_k) for i in range(n_layers)]
    prev = orc.set_threads(threads if threads > 0 else len(os.sched_getaffinity(0)))
    done_bytes, done = 0.0, 0
    t0 = time.perf_counter()
    s = 0
    try:
        while time.perf_counter() - t0 < budget_s:
            x = x_bank[s % x_bank.shape[0]].view(np.uint16)
            for L in Ls:
                out_f32, out_bf16, ids, sc, sl = orc.moe_layer(x, L, residual=True)
                U = len(np.unique(ids))
                done_bytes += float(layer_bytes(np.array([U]), args.T, args.hidden)[0])
                done += 1
                x = out_bf16
            s += 1
    finally:
        orc.set_threads(prev)
    el = time.perf_counter() - t0
    return {"value": round(done_bytes / el / 1e9, 4), "unit": "GB/s", "cores": _threads_label(threads),
            "kind": "port",
            "sample": f"{done} layer calls ({n_layers} layers x {s} steps, T={args.T}) of the same stack, "
                      f"{el:.1f} s, float64 oracle with OpenMP"}


def moe_parity(layers, layers_w, x, args) -> dict:
    """The first two layers of the stack on one verify batch against the oracle:
    routed ids, and each layer's output from the GPU's own input (relative L2,
    cosine, worst token)."""
    import torch
    from oracle import oracle as orc
    from oracle.torch_bridge import layer_np, u16

    T, k = x.shape[0], args.top_k
    cur = x
    worst_rel, worst_cos, ids_equal = 0.0, 1.0, True
    for l in range(2):
        ids = torch.empty((T, k), dtype=torch.int32, device=x.device)
        out = layers[l](cur, residual=cur, ids_out=ids)
        torch.cuda.synchronize()
        ref32, _, rid, _, _ = orc.moe_layer(u16(cur), layer_np(layers_w[l], k), residual=True)
        ids_equal &= bool(np.array_equal(ids.cpu().numpy(), rid))
        got = orc.bf16_to_f32(u16(out).reshape(T, -1)).astype(np.float64)
        for t in range(T):
            g, r = got[t], ref32[t]
            worst_rel = max(worst_rel, float(np.linalg.norm(g - r) / np.linalg.norm(r)))
            worst_cos = min(worst_cos, float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r))))
        cur = out
    ok = ids_equal and worst_rel <= 1e-2 and worst_cos >= 0.9999
    return {"layers": 2, "tokens": T, "routed_ids_equal": ids_equal, "max_rel_l2": round(worst_rel, 6),
            "min_cosine": round(worst_cos, 8), "bar": "ids exact, rel L2 <= 1e-2, cos >= 0.9999", "ok": ok}


def bench_copy(args) -> int:
    """Calibration workload for the HBM byte counters: one elementwise pass
    that reads and writes args.copy_mib MiB (fp32 y = x * 1), repeated
    args.steps times.  A counter pass over it gives the counter's reading per
    known byte."""
    import torch

    dev = torch.device("cuda:0")
    n = args.copy_mib * (1 << 20) // 4
    x = torch.ones(n, dtype=torch.float32, device=dev)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        torch.mul(x, 1.0, out=y)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    nbytes = 2 * 4 * n
    print(json.dumps({"path": "copy", "bytes_read": 4 * n, "bytes_written": 4 * n, "launches": args.steps,
                      "us_per_launch": round(ms * 1e3 / args.steps, 3),
                      "GBps": round(nbytes * args.steps / (ms / 1e3) / 1e9, 1)}), flush=True)
    return 0


def measure_stream_peak(mib: int = 4096, reps: int = 10) -> dict:
    """Read ceiling of this GPU's HBM, measured with libvmi's read-only stream
    kernel (vmi_stream_read) over a `mib` MiB buffer: best GB/s over a sweep
    of workgroup counts, nontemporal and cached loads, each the mean of `reps`
    launches timed with HIP events.  The XOR of the buffer is checked against
    torch's, so a launch that skipped bytes would not count."""
    import torch
    from vates_amd._lib import check, load
    lib = load()
    dev = torch.device("cuda:0")
    n = mib * (1 << 20) // 4
    if n & (n - 1):
        raise ValueError(f"stream buffer of {mib} MiB: a power of two is needed")
    buf = torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device=dev)
    fold = buf  # XOR of all words by halving on the device (n is a power of two)
    while fold.numel() > 1:
        h = fold.numel() // 2
        fold = torch.bitwise_xor(fold[:h], fold[h:])
    want = int(fold.cpu().numpy().view(np.uint32)[0])
    del fold
    stream = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.zeros(cus * 16, dtype=torch.int32, device=dev)
    results = {}
    for nt in (1, 0):
        for per_cu in (1, 2, 4, 8, 16):
            wgs = cus * per_cu
            check(lib.vmi_stream_read(buf.data_ptr(), buf.numel() * 4, nt, wgs, sink.data_ptr(), stream),
                  "vmi_stream_read")
            torch.cuda.synchronize()
            if int(np.bitwise_xor.reduce(sink[:wgs].cpu().numpy().view(np.uint32))) != want:
                raise RuntimeError(f"vmi_stream_read checksum mismatch (nt={nt}, workgroups={wgs})")
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(reps):
                lib.vmi_stream_read(buf.data_ptr(), buf.numel() * 4, nt, wgs, sink.data_ptr(), stream)
            end.record()
            torch.cuda.synchronize()
            gbs = buf.numel() * 4 * reps / (start.elapsed_time(end) / 1e3) / 1e9
            results[(nt, wgs)] = gbs
    del buf
    torch.cuda.empty_cache()
    best_nt = max((v, k) for k, v in results.items() if k[0] == 1)
    best_c = max((v, k) for k, v in results.items() if k[0] == 0)
    return {"gbs": round(max(best_nt[0], best_c[0]), 1), "nontemporal_gbs": round(best_nt[0], 1),
            "nontemporal_workgroups": best_nt[1][1], "cached_gbs": round(best_c[0], 1),
            "cached_workgroups": best_c[1][1], "buffer_mib": mib, "launches_each": reps,
            "kernel": "vmi_stream_read (libvmi): 16-byte buffer loads, 8 in flight per lane, XOR-checked"}


def measure_mfma_peak(iters: int = 20000) -> dict:
    """Dense fp16 MFMA ceiling of this GPU, measured with libvmi's
    vmi_mfma_peak (four independent v_mfma_f32_16x16x32_f16 chains per wave,
    the instruction of the prefill GEMMs): best TFLOP/s over a sweep of
    workgroup counts, each the mean of 3 launches timed with HIP events."""
    import torch
    from vates_amd._lib import check, load
    lib = load()
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream().cuda_stream
    best = (0.0, 0)
    for per_cu in (2, 4, 8, 16):
        wgs = cus * per_cu
        sink = torch.zeros(wgs, dtype=torch.float32, device=dev)
        check(lib.vmi_mfma_peak(wgs, 64, sink.data_ptr(), stream), "vmi_mfma_peak")
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(3):
            lib.vmi_mfma_peak(wgs, iters, sink.data_ptr(), stream)
        end.record()
        torch.cuda.synchronize()
        tfs = 3 * wgs * 16.0 * iters * 16384 / (start.elapsed_time(end) / 1e3) / 1e12
        if not bool(torch.isfinite(sink).all()):
            raise RuntimeError("vmi_mfma_peak produced a non-finite checksum")
        best = max(best, (tfs, wgs))
    return {"tflops": round(best[0], 1), "workgroups": best[1], "iters": iters,
            "kernel": "vmi_mfma_peak (libvmi): v_mfma_f32_16x16x32_f16, 4 independent chains per wave"}


def bench_stream(args) -> int:
    """The device's measured ceilings on their own: HBM read (vmi_stream_read)
    and dense fp16 MFMA (vmi_mfma_peak)."""
    import torch
    torch.cuda.set_device(0)
    st = measure_stream_peak(args.stream_mib)
    mf = measure_mfma_peak()
    eprint(f"[bench] stream read {st['gbs']} GB/s (nt {st['nontemporal_gbs']}, cached {st['cached_gbs']}); "
           f"MFMA {mf['tflops']} TFLOP/s")
    print(json.dumps({"path": "stream", "metric": "measured HBM read ceiling", "value": st["gbs"], "unit": "GB/s",
                      "frac_of_published": round(st["gbs"] / PEAK_HBM_GBS, 4), "stream": st,
                      "mfma": mf, "mfma_frac_of_published": round(mf["tflops"] / PEAK_MFMA_TFLOPS, 4)}),
          flush=True)
    return 0


def layer_latency(one_step, layers_n: int, xa, x_bank, steps: int) -> dict:
    """Per-layer-call latency distribution of the MoE stack.  Each step's
    layer calls are launched eagerly with a HIP event between consecutive
    calls; a bounded device-side sleep (torch.cuda._sleep) ahead of every step
    lets the host queue the whole step before the GPU reaches it, so the event
    gaps hold device time, not host latency.  Event markers add to each call,
    so the same steps are also run without them (one event pair per step) and
    the difference is reported as the markers' cost.  (ROCm does not record
    events inside a captured graph.)"""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    torch.cuda._sleep(2_000_000)
    e1.record()
    torch.cuda.synchronize()
    cyc_per_us = 2_000_000 / max(e0.elapsed_time(e1) * 1e3, 1.0)
    head_start = int(cyc_per_us * layers_n * 80)  # 80 us of host time per layer call
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(layers_n + 1)]
    samples, plain = [], []
    for st in range(steps):
        xa.copy_(x_bank[st])
        torch.cuda._sleep(head_start)
        one_step(ev)
        torch.cuda.synchronize()
        samples += [ev[l].elapsed_time(ev[l + 1]) * 1e3 for l in range(layers_n)]
        xa.copy_(x_bank[st])
        torch.cuda._sleep(head_start)
        e0.record()
        one_step(None)
        e1.record()
        torch.cuda.synchronize()
        plain.append(e0.elapsed_time(e1) * 1e3 / layers_n)
    a = np.array(samples)
    return {"p50_us": round(float(np.percentile(a, 50)), 3), "p99_us": round(float(np.percentile(a, 99)), 3),
            "mean_us": round(float(a.mean()), 3), "max_us": round(float(a.max()), 3), "samples": int(a.size),
            "mean_us_without_markers": round(float(np.mean(plain)), 3),
            "marker_cost_us": round(float(a.mean() - np.mean(plain)), 3),
            "method": f"{steps} steps x {layers_n} layer calls launched eagerly behind a device-side sleep, "
                      "HIP events between calls"}


def bench_lm_head(args) -> int:
    """lm_head GEMV + fused argmax over the full vocabulary: bf16 [V, 2048] head
    (622 MB at V=151936), T tokens RMS-normalised in the kernel, f32 logits out.
    Algorithmic bytes per launch = V*H*2 (head) + T*H*2 (x) + H*2 (norm weight)
    + T*V*4 (logits)."""
    import torch
    from vates_amd.head import TiledHead, lm_head
    from vates_amd.synth import synth_bf16

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T, H, V = args.T, args.hidden, args.vocab
    W = synth_bf16(SEED, 0x4EAD, (V, H), std=0.02, device=dev)
    # the decode loop's form: the head re-laid once, tile-major (vmi_head_tiles)
    Wt = TiledHead(W)
    nw = synth_bf16(SEED, 0x4EAE, (H,), std=0.1, device=dev) + 1.0
    xs = synth_bf16(SEED, 0x4EAF, (args.steps + args.warmup, T, H), device=dev)
    logits = torch.empty((T, V), dtype=torch.float32, device=dev)
    am = torch.empty(T, dtype=torch.int32, device=dev)
    mx = torch.empty(T, dtype=torch.float32, device=dev)
    def timed(head):
        for s in range(args.warmup):
            lm_head(xs[args.steps + s], head, nw, logits=logits, argmax=am, max_logit=mx)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for s in range(args.steps):
            lm_head(xs[s], head, nw, logits=logits, argmax=am, max_logit=mx)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end)

    ms_rows = timed(W)  # the row-major head (vmi_lm_head), for comparison
    ms = timed(Wt)
    us = ms * 1e3 / args.steps
    nbytes = V * H * 2 + T * H * 2 + H * 2 + T * V * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    eprint(f"[bench] lm_head T={T} V={V}: {us:.2f} us per launch, {gbs:.1f} GB/s")

    cpu = None
    if args.cpu_baseline_s > 0:
        from oracle import oracle as orc
        from oracle.torch_bridge import u16
        rows = 8192
        Wn, xn, nwn = u16(W[:rows]), u16(xs[0]), u16(nw)
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_baseline_s:
            orc.lm_head(xn, nwn, 1e-6, Wn)
            done += 1
        el = time.perf_counter() - t0
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
        threads = min(threads, len(os.sched_getaffinity(0)))
        cpu = {"value": round(done * (rows * H * 2 + T * rows * 4) / el / 1e9, 4), "unit": "GB/s", "cores": threads,
               "kind": "port", "sample": f"{done} oracle calls over the first {rows} head rows, T={T}, {el:.1f} s, "
                                         f"float64 accumulation with OpenMP"}
    line = {
        "metric": "lm_head GEMV + argmax HBM GB/s", "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 x bf16 MFMA, f32 accumulate", "data": "synthetic",
        "config": {"workload": f"lm_head over vocab {V}, hidden {H}, T={T}, RMSNorm fused, f32 logits + argmax",
                   "T": T, "vocab": V, "hidden": H},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None, "unit_of_work": "one lm_head call",
                     "bytes_per_launch": nbytes, "us_per_launch": round(us, 3),
                     "kernel": "vmi_lm_head_tiled (tile-major head copy)",
                     "row_major_us_per_launch": round(ms_rows * 1e3 / args.steps, 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def _proj_bytes(p) -> int:
    return p.weight.numel() * 4 + p.scales.numel() * 2 + p.biases.numel() * 2


def _moe_fixed_bytes(moe) -> int:
    """Router, shared expert and its gate of one MoE layer (bytes read per call)."""
    k = moe._keep
    return sum(_proj_bytes(q) for q in (k[0], k[4], k[5], k[6], k[7]) if q is not None)


def _trace_moe_calls(fn):
    """Runs fn() with every MoE layer call recording its routed ids; returns
    {layer object id: [distinct experts per call]}."""
    import torch
    from vates_amd.moe import MoELayer
    seen = {}
    orig = MoELayer.__call__

    def traced(self, x, residual=None, *, out=None, ids_out=None, scores_out=None, stream=None, ws=None):
        T = x.numel() // self.hidden
        ids = ids_out if ids_out is not None else torch.empty((T, self.top_k), dtype=torch.int32, device=x.device)
        y = orig(self, x, residual, out=out, ids_out=ids, scores_out=scores_out, stream=stream, ws=ws)
        seen.setdefault(id(self), []).append(ids)
        return y

    MoELayer.__call__ = traced
    try:
        fn()
    finally:
        MoELayer.__call__ = orig
    torch.cuda.synchronize()
    return {k: [int(np.unique(i.cpu().numpy()).size) for i in v] for k, v in seen.items()}


def decode_step_bytes(model, K: int, L: int, U: dict) -> dict:
    """Algorithmic HBM bytes of one speculative step in the [x, d1..dK] layout
    at context L: the verify forward (T = K + 1), K MTP draft steps (T = 1)
    and the MTP update (T = K + 1).  Weights are read once per call, caches
    as the kernels read them; U: distinct experts per MoE call, traced."""
    T = K + 1
    H = model.hidden
    V = model.head.shape[0]
    head = V * H * 2
    items = {"verify_attention": 0, "verify_gdn": 0, "verify_moe": 0, "verify_head": head, "mtp_drafts": 0,
             "mtp_update": 0}
    for layer in model.layers:
        if layer.attn is not None:
            a = layer.attn
            kv_read = 2 * a.n_kv * L * 256 * 2
            items["verify_attention"] += sum(_proj_bytes(q) for q in a._keep[:4]) + kv_read + 2 * a.n_kv * T * 512
        elif layer.gdn is not None:
            g = layer.gdn
            state = g.n_v * 128 * 128 * 4
            conv = g._keep[4].numel() * 2
            items["verify_gdn"] += sum(_proj_bytes(q) for q in g._keep[:3]) + conv + state + T * state
        u = U[id(layer.moe)][0]
        items["verify_moe"] += u * EXPERT_BYTES + _moe_fixed_bytes(layer.moe)
    w = model.mtp.w
    att = sum(_proj_bytes(q) for q in w.attn._keep[:4])
    kv = 2 * w.attn.n_kv * L * 256 * 2
    mtp_u = U[id(w.moe)]  # K draft calls (T = 1), then the update (T = K + 1)
    for i in range(K):
        items["mtp_drafts"] += _proj_bytes(w.fc) + att + kv + mtp_u[i] * EXPERT_BYTES + _moe_fixed_bytes(w.moe) + head
    items["mtp_update"] = _proj_bytes(w.fc) + att + kv + mtp_u[K] * EXPERT_BYTES + _moe_fixed_bytes(w.moe)
    items["total"] = sum(items.values())
    return items


def decode_cpu_baseline(model, ctx: int, budget_s: float, threads: int) -> dict:
    """Greedy decoding cost per token of the oracle (float64, OpenMP) on the
    host: one full-attention block at a ctx-token context, one Gated DeltaNet
    block, one MoE layer and the head, each at T = 1, timed and weighted by the
    model's layer counts.  Weights of those blocks copied to the host; the
    context's keys and values are synthetic (their values do not change the
    cost)."""
    import torch
    from oracle import oracle as orc
    from oracle.torch_bridge import u16
    sys.path.insert(0, str(ROOT / "tests"))
    from model_oracle import attn_dict, gdn_dict, moe_dict

    la = next(l for l in model.layers if l.attn is not None)
    lg = next(l for l in model.layers if l.gdn is not None)
    A, G, L = attn_dict(la.attn), gdn_dict(lg.gdn), moe_dict(la.moe)
    W, nw = u16(model.head), u16(model.final_norm)
    rng = np.random.default_rng(0)
    x = orc.f32_to_bf16(rng.standard_normal((1, model.hidden)).astype(np.float32))
    kc = orc.f32_to_bf16(rng.standard_normal((la.attn.n_kv, ctx + 32, 256)).astype(np.float32))
    cd = 2 * G["n_k"] * 128 + G["n_v"] * 128
    conv_in = rng.standard_normal((3, cd)) * 0.1
    state_in = rng.standard_normal((G["n_v"], 128, 128)) * 0.01
    calls = {"attention": lambda: orc.attention_layer(x, A, ctx, kc, kc),
             "gdn": lambda: orc.gdn_layer(x, G, conv_in=conv_in, state_in=state_in),
             "moe": lambda: orc.moe_layer(x, L, residual=True),
             "head": lambda: orc.lm_head(x, nw, 1e-6, W)}
    prev = orc.set_threads(threads if threads > 0 else len(os.sched_getaffinity(0)))
    per = {}
    t_all = time.perf_counter()
    try:
        for name, fn in calls.items():
            n, t0 = 0, time.perf_counter()
            while n == 0 or time.perf_counter() - t0 < budget_s / len(calls):
                fn()
                n += 1
            per[name] = (time.perf_counter() - t0) / n
    finally:
        orc.set_threads(prev)
    n_att = sum(l.attn is not None for l in model.layers)
    n_gdn = sum(l.gdn is not None for l in model.layers)
    sec = n_att * per["attention"] + n_gdn * per["gdn"] + len(model.layers) * per["moe"] + per["head"]
    return {"value": round(1.0 / sec, 4), "unit": "tokens/s", "cores": _threads_label(threads), "kind": "port",
            "sample": f"oracle greedy decode cost per token at T=1, context {ctx}: attention "
                      f"{per['attention'] * 1e3:.1f} ms x {n_att}, Gated DeltaNet {per['gdn'] * 1e3:.1f} ms x {n_gdn}, "
                      f"MoE {per['moe'] * 1e3:.1f} ms x {len(model.layers)}, head {per['head'] * 1e3:.1f} ms "
                      f"({time.perf_counter() - t_all:.1f} s timed), float64 with OpenMP"}


def decode_record(args) -> dict:
    """K-draft MTP speculative decoding of a random-init Qwen3-Next-shaped model:
    `layers` decoder layers (full attention on every attn_every-th, Gated
    DeltaNet linear attention on the others, the 512-expert top-10 4-bit MoE
    with the shared expert on all), the MTP layer, bf16 embedding and head over
    151,936 tokens.  A `context`-token synthetic prompt (random token ids) is
    run through the model first, 8 tokens per forward, filling the attention
    caches, the linear-attention states and the MTP cache.  Timed: `new_tokens`
    decoded tokens by graph replays, wall clock, including drafting,
    verification, acceptance, commit and the MTP cache update.  The same start
    state is then decoded greedily (one token per graph replay, the
    like-for-like baseline) and the two token streams are compared.  A
    random-init MTP layer's argmax drafts almost never match the main model's,
    so the greedy speculative run measures the cost of speculation with no
    gain; drafts planted at a fixed agreement rate show the
    acceptance-dependent speed, and a sampled run (temperature 0.7, top-p 0.9,
    speculative sampling) the stochastic loop."""
    import torch
    from vates_amd.decode import GraphGreedyDecoder, GraphSpecDecoder, Sampling, speculative_decode
    from vates_amd.gdn import GdnCache
    from vates_amd.mtp import MTPDrafter
    from vates_amd.workload import synth_spec_model

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t0 = time.time()
    model = synth_spec_model(SEED, n_layers=args.layers, attn_every=args.attn_every, hidden=args.hidden,
                             inter=args.inter, num_experts=args.experts, top_k=args.top_k, vocab=args.vocab,
                             device=dev)
    ctx, N, K = args.context, args.new_tokens, args.K
    max_len = ctx + 2 * N + 4 * (K + 1) + 8
    caches = model.new_caches(max_len)
    drafter = MTPDrafter(model.mtp, max_len)
    torch.cuda.synchronize()
    eprint(f"[bench] decode model resident: {torch.cuda.memory_allocated() / 2**30:.1f} GiB in {time.time() - t0:.1f} s")
    prompt = torch.from_numpy(np.random.default_rng(SEED).integers(0, args.vocab, ctx).astype(np.int32)).to(dev)
    t1 = time.time()
    if args.synthetic_cache:
        # profiling runs: random keys and values in the caches instead of the
        # prompt's (a decode step's cost does not depend on the contents)
        from vates_amd.attention import KVCache
        from vates_amd.synth import synth_bf16
        for i, c in enumerate(caches + [drafter.cache]):
            if isinstance(c, KVCache):
                c.write(0, synth_bf16(SEED, 0xCA000 + 2 * i, (c.k.shape[0], ctx, 256), device=dev),
                        synth_bf16(SEED, 0xCA001 + 2 * i, (c.v.shape[0], ctx, 256), device=dev))
            elif c is not None:
                c.length = ctx
        drafter.cache.length = ctx - 1
        x0 = prompt[-1:].clone()
        h0 = synth_bf16(SEED, 0xCA0FF, (1, args.hidden), device=dev)
        eprint("[bench] synthetic cache contents (profiling run): the prompt was not run")
    else:
        # the prompt through the model 8 tokens per forward (as decode.prefill),
        # then the MTP cache over its (hidden, next token) pairs; a line every
        # 4,096 tokens
        hs, am = [], None
        for s0 in range(0, ctx, 8):
            am, h, _ = model.forward(prompt[s0:s0 + 8], caches, s0)
            hs.append(h)
            if (s0 + 8) % 4096 == 0 or s0 + 8 >= ctx:
                torch.cuda.synchronize()
                eprint(f"[bench] prompt prefill: {min(ctx, s0 + 8)} of {ctx} tokens, {time.time() - t1:.1f} s")
        hid = torch.cat(hs)
        drafter.cache.length = 0
        for s0 in range(0, ctx - 1, 8):
            e = min(ctx - 1, s0 + 8)
            drafter.mtp.advance(hid[s0:e].contiguous(), prompt[s0 + 1:e + 1].contiguous(), drafter.cache)
            if (s0 + 8) % 8192 == 0:
                torch.cuda.synchronize()
                eprint(f"[bench] MTP cache: {e} of {ctx - 1} positions, {time.time() - t1:.1f} s")
        x0, h0 = am[-1:].clone(), hid[-1:].clone()
        del hs, hid
        torch.cuda.synchronize()
        eprint(f"[bench] prompt of {ctx} tokens run through the model and the MTP layer in {time.time() - t1:.1f} s")
    saved = [(c.conv.clone(), c.state.clone()) if isinstance(c, GdnCache) else None for c in caches]

    def reset():
        for c, sv in zip(caches, saved):
            if c is not None:
                c.length = ctx
            if sv is not None:  # the linear-attention rings as the prompt left them
                c.conv.copy_(sv[0])
                c.state.copy_(sv[1])
        drafter.cache.length = ctx - 1

    # distinct experts of every MoE call of one step, traced on an eager step
    reset()
    U = _trace_moe_calls(lambda: speculative_decode(model, drafter, caches, x0, h0, ctx, 1, K=K))
    step_bytes = decode_step_bytes(model, K, ctx + K + 1, U)

    def graph_spec(planted=None, **kw):
        reset()
        dec = GraphSpecDecoder(model, drafter, caches, K=K, planted=planted is not None, **kw)
        dec.start(x0, h0, ctx)
        dec.capture()
        if args.warmup:
            dec.run(args.warmup * (K + 1), plant=planted)
            reset()
            dec.start(x0, h0, ctx)
        torch.cuda.synchronize()
        return dec.run(N, plant=planted)

    st = graph_spec()
    tps = N / st.seconds
    ms_step = st.seconds * 1e3 / st.steps
    eprint(f"[bench] decode (graph, MTP drafts): {N} tokens in {st.seconds:.3f} s = {tps:.1f} tokens/s, "
           f"{st.steps} steps, {ms_step:.3f} ms per step, avg accept len {st.avg_accept_len:.2f}")
    reset()
    gd = GraphGreedyDecoder(model, caches, N + 4 * (K + 1))
    gd.start(x0, ctx)
    gd.capture()
    if args.warmup:
        gd.run(args.warmup)
        reset()
        gd.start(x0, ctx)
    gr = gd.run(N + 2 * (K + 1))
    truth = gr.tokens
    gr_tps = len(truth) / gr.seconds
    same = truth[:N] == st.tokens
    first_diff = next((i for i, (a, b) in enumerate(zip(truth, st.tokens)) if a != b), None)
    eprint(f"[bench] greedy (graph, one token per replay): {gr_tps:.1f} tokens/s; speculative == greedy: {same}")
    rng = np.random.default_rng(SEED)

    def plant(step, pos):
        base = pos - ctx
        return [truth[base + i] if rng.random() < args.plant_rate else (truth[base + i] + 1) % args.vocab
                for i in range(K)]

    sp = graph_spec(plant)
    sp_tps = N / sp.seconds
    sp_same = sp.tokens == truth[:N]
    eprint(f"[bench] decode (graph, drafts planted at agreement {args.plant_rate}): {sp_tps:.1f} tokens/s, "
           f"avg accept len {sp.avg_accept_len:.2f}, equals greedy: {sp_same}")
    ad = graph_spec(layout="k", tau=args.tau)
    ad_tps = N / ad.seconds
    ad_same = ad.tokens == truth[:N]
    eprint(f"[bench] decode (graph, adaptive depth tau={args.tau}, T=K layout): {ad_tps:.1f} tokens/s, "
           f"depths {[ad.depths.count(d) for d in range(1, K + 1)]}, equals greedy: {ad_same}")
    smp = graph_spec(sampling=Sampling(0.7, 0.9, SEED))
    smp_tps = N / smp.seconds
    smp_hist = [smp.accept_hist.count(m) for m in range(K + 1)]
    eprint(f"[bench] decode (graph, sampled: temperature 0.7, top-p 0.9): {smp_tps:.1f} tokens/s, "
           f"{smp.steps} steps, {smp.seconds * 1e3 / smp.steps:.3f} ms per step, avg accept len "
           f"{smp.avg_accept_len:.2f}, matched histogram {smp_hist}")
    hist = [st.accept_hist.count(m) for m in range(K + 1)]
    achieved = step_bytes["total"] / (ms_step * 1e-3) / 1e9
    cpu = cpu1 = None
    if args.cpu_baseline_s > 0:
        cpu = decode_cpu_baseline(model, ctx, args.cpu_baseline_s * 0.6, 0)
        cpu1 = decode_cpu_baseline(model, ctx, 1.0, 1)
        eprint(f"[bench] decode oracle on the host: {cpu['value']} tokens/s ({cpu['cores']} cores), "
               f"{cpu1['value']} tokens/s (1 core)")
    del model, caches, drafter
    torch.cuda.empty_cache()
    return {
        "metric": f"K=3 MTP decode tokens/s (greedy, random-init MTP drafts: avg accept len "
                  f"{st.avg_accept_len:.2f}, {tps / gr_tps:.3f}x greedy decoding)",
        "value": round(tps, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": st.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u4 experts/projections, bf16 head and KV, f32 accumulate", "data": "synthetic",
        "config": {"workload": f"{args.layers}-layer random-init Qwen3-Next-shaped model ({args.layers // args.attn_every}"
                               f" full-attention and {args.layers - args.layers // args.attn_every} Gated DeltaNet "
                               f"layers, every layer MoE 512x top-{args.top_k} + shared expert), MTP K={K}, "
                               f"{N} new tokens after a {ctx}-token synthetic prompt"
                               f"{' (cache contents synthetic, prompt not run)' if args.synthetic_cache else ''}, "
                               f"vocab {args.vocab}",
                   "step": "one HIP graph replay per step, verify [x, d1..dK]",
                   "accept_hist": hist, "avg_accept_len": round(st.avg_accept_len, 3),
                   "speculative_equals_greedy": same, "first_divergence": first_diff,
                   "greedy_graph_tokens_per_s": round(gr_tps, 2),
                   "spec_over_greedy": round(tps / gr_tps, 4),
                   "planted_agreement": args.plant_rate, "planted_tokens_per_s": round(sp_tps, 2),
                   "planted_over_greedy": round(sp_tps / gr_tps, 4),
                   "planted_avg_accept_len": round(sp.avg_accept_len, 3), "planted_equals_greedy": sp_same,
                   "adaptive_tau": args.tau, "adaptive_tokens_per_s": round(ad_tps, 2),
                   "adaptive_depths": [ad.depths.count(d) for d in range(1, K + 1)],
                   "adaptive_equals_greedy": ad_same,
                   "sampled": {"temperature": 0.7, "top_p": 0.9, "seed": SEED, "tokens_per_s": round(smp_tps, 2),
                               "ms_per_step": round(smp.seconds * 1e3 / smp.steps, 4),
                               "avg_accept_len": round(smp.avg_accept_len, 3), "accept_hist": smp_hist,
                               "over_greedy": round(smp_tps / gr_tps, 4),
                               "step": "sampled MTP drafts (vmi_sample_top_p), verify, vmi_accept_stochastic, "
                                       "vmi_spec_commit: one HIP graph replay"}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": None,
                     "unit_of_work": "one speculative step (K MTP drafts, verify of K+1 tokens, MTP update)",
                     "bytes_per_step": {k: int(v) for k, v in step_bytes.items()},
                     "us_per_step": round(ms_step * 1e3, 2)},
        "cpu_baseline": cpu, "cpu_baseline_1core": cpu1,
    }


def bench_decode(args) -> int:
    line = decode_record(args)
    print(json.dumps(line), flush=True)
    return 0 if line["config"]["speculative_equals_greedy"] else 3


PEAK_MFMA_TFLOPS = 2500.0  # dense fp16/bf16


def bench_prefill(args) -> int:
    """Expert-major prefill of one MoE layer (hidden 2048, 512 experts top-10,
    inter 512, 8-bit router, shared expert, Zipf(1.1) routing) on a T-token
    prompt, bf16 activations N(0,1).  FLOPs per launch = (T*k + T) * 6*H*I
    (routed assignments and the shared expert: gate, up, down) + 2*T*E*H
    (router); algorithmic HBM bytes = distinct experts * 1,769,472 + shared
    1,769,472 + router 1,114,112 + x in, residual in, out (3*T*H*2)."""
    import torch
    from vates_amd.synth import synth_bf16
    from vates_amd.workload import make_layer, synth_layer

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T, H, k, E, I = args.T, args.hidden, args.top_k, args.experts, args.inter
    w = synth_layer(SEED, 0, hidden=H, inter=I, num_experts=E, zipf_s=ZIPF_S, zipf_alpha=1.0, device=dev)
    moe = make_layer(w, top_k=k)
    xs = synth_bf16(SEED, 0x9F11, (2, T, H), device=dev)
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    ids = torch.empty((T, k), dtype=torch.int32, device=dev)
    for s in range(args.warmup):
        moe.prefill(xs[s % 2], residual=xs[s % 2], out=out, ids_out=ids)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for s in range(args.steps):
        moe.prefill(xs[s % 2], residual=xs[s % 2], out=out, ids_out=ids)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)
    us = ms * 1e3 / args.steps
    U = int(np.unique(ids.cpu().numpy()).size)
    flops = (T * k + T) * 6.0 * H * I + 2.0 * T * E * H
    nbytes = U * EXPERT_BYTES + EXPERT_BYTES + ROUTER8_BYTES + 3 * T * H * 2
    tfs = flops / (us * 1e-6) / 1e12
    gbs = nbytes / (us * 1e-6) / 1e9
    hbm_bound = flops / nbytes < PEAK_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
    eprint(f"[bench] prefill T={T}: {us:.1f} us per layer, {tfs:.1f} TFLOP/s, {gbs:.1f} GB/s, {U} experts touched")
    mf = measure_mfma_peak()
    eprint(f"[bench] measured MFMA ceiling {mf['tflops']} TFLOP/s")
    from vates_amd.moe import workspace, workspace_status
    ws = workspace(moe.prefill_workspace_bytes(T), dev, torch.cuda.current_stream().cuda_stream, tag="prefill")
    if workspace_status(ws):
        eprint("[bench] device status flags set")
        return 3
    cpu = None
    if args.cpu_baseline_s > 0:
        from oracle import oracle as orc
        from oracle.torch_bridge import layer_np, u16
        L = layer_np(w, k, True)
        xn = u16(xs[0])
        rows = 32
        done, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_baseline_s:
            orc.moe_layer(xn[done % (T // rows) * rows:(done % (T // rows) + 1) * rows], L, residual=True)
            done += 1
        el = time.perf_counter() - t0
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
        threads = min(threads, len(os.sched_getaffinity(0)))
        cpu = {"value": round(done * rows * (k + 1) * 6.0 * H * I / el / 1e12, 6), "unit": "TFLOP/s",
               "cores": threads, "kind": "port",
               "sample": f"{done} oracle layer calls of {rows} tokens each, {el:.1f} s, float64 with OpenMP"}
    line = {
        "metric": "expert-major MoE prefill " + ("HBM GB/s" if hbm_bound else "MFMA TFLOP/s"),
        "value": round(gbs if hbm_bound else tfs, 2), "unit": "GB/s" if hbm_bound else "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u4 weights x f16/bf16 MFMA, f32 accumulate (bf16 in/out)", "data": "synthetic",
        "config": {"workload": f"expert-major prefill of one MoE layer, T={T}, {E} experts top-{k}, hidden {H}, "
                               f"inter {I}, Zipf(1.1) routing, shared expert",
                   "T": T, "experts_touched": U, "tflops_per_s": round(tfs, 2), "hbm_gbs": round(gbs, 2)},
        "roofline": {"bound": "hbm" if hbm_bound else "mfma",
                     "achieved": round(gbs if hbm_bound else tfs, 2),
                     "peak": PEAK_HBM_GBS if hbm_bound else PEAK_MFMA_TFLOPS,
                     "unit": "GB/s" if hbm_bound else "TFLOP/s",
                     "frac": round((gbs / PEAK_HBM_GBS) if hbm_bound else (tfs / PEAK_MFMA_TFLOPS), 4),
                     "peak_measured": None if hbm_bound else mf["tflops"],
                     "frac_measured": None if hbm_bound else round(tfs / mf["tflops"], 4),
                     "peak_measured_source": None if hbm_bound else mf,
                     "traffic": None, "unit_of_work": "one vmi_moe_prefill call",
                     "flops_per_launch": flops, "bytes_per_launch": nbytes, "us_per_launch": round(us, 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--eager", action="store_true", help="decode: launch every kernel from Python instead of graph replays")
    ap.add_argument("--plant-rate", type=float, default=0.7, help="decode: per-position draft agreement of the planted run")
    ap.add_argument("--T", type=int, default=4)
    ap.add_argument("--top-k", type=int, default=10)
    ap.add_argument("--hidden", type=int, default=2048)
    ap.add_argument("--inter", type=int, default=512)
    ap.add_argument("--experts", type=int, default=512)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--cpu-baseline-s", type=float, default=15.0)
    ap.add_argument("--path", choices=["moe", "lm_head", "prefill", "decode", "copy", "stream"], default="moe",
                    help="moe: the 48-layer verify stack (default); lm_head: the vocabulary GEMV + argmax; "
                         "prefill: one expert-major MoE layer on a T-token prompt; decode: K=3 MTP speculative "
                         "decoding end to end; copy: a plain elementwise copy of known size (calibrates the "
                         "HBM byte counters); stream: the measured HBM read and dense MFMA ceilings")
    ap.add_argument("--copy-mib", type=int, default=512)
    ap.add_argument("--stream-mib", type=int, default=4096, help="stream: buffer size (a power of two)")
    ap.add_argument("--context", type=int, default=32768)
    ap.add_argument("--new-tokens", type=int, default=512)
    ap.add_argument("--K", type=int, default=3)
    ap.add_argument("--attn-every", type=int, default=4)
    ap.add_argument("--tau", type=float, default=0.3, help="decode: adaptive-depth confidence threshold")
    ap.add_argument("--no-decode", action="store_true", help="default path: skip the decode record")
    ap.add_argument("--synthetic-cache", action="store_true",
                    help="decode: random cache contents instead of running the prompt (profiling runs)")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="default path: skip the latency pass and the measured read ceiling (counter passes)")
    ap.add_argument("--vocab", type=int, default=151936)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this path is single-device (all weights resident in one "
              "MI355X's HBM); run with --gpus 1", file=sys.stderr)
        return 2

    if args.path == "lm_head":
        return bench_lm_head(args)
    if args.path == "prefill":
        return bench_prefill(args)
    if args.path == "decode":
        return bench_decode(args)
    if args.path == "copy":
        return bench_copy(args)
    if args.path == "stream":
        return bench_stream(args)

    import torch
    from vates_amd.synth import synth_bf16
    from vates_amd.workload import make_layer, synth_layer

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    T, H, k = args.T, args.hidden, args.top_k
    t0 = time.time()
    ws_list, layers = [], []
    for l in range(args.layers):
        w = synth_layer(SEED, l, hidden=H, inter=args.inter, num_experts=args.experts, zipf_s=ZIPF_S,
                        zipf_alpha=ZIPF_ALPHA, device=dev)
        if l < 2:
            ws_list.append(w)  # the oracle legs read the first two layers' weights
        layers.append(make_layer(w, top_k=k))
    n_in = args.steps + args.warmup
    x_bank = synth_bf16(SEED, 0xBEEF, (n_in, T, H), device=dev)
    torch.cuda.synchronize()
    eprint(f"[bench] weights resident: {torch.cuda.memory_allocated() / 2**30:.1f} GiB in {time.time() - t0:.1f} s")

    xa = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    xb = torch.empty_like(xa)
    ids = torch.zeros((args.layers, T, k), dtype=torch.int32, device=dev)
    ws = torch.zeros(layers[0].workspace_bytes(T), dtype=torch.uint8, device=dev)

    def one_step(events=None):
        cur, nxt = xa, xb
        for l, layer in enumerate(layers):
            if events is not None:
                events[l].record()
            layer(cur, residual=cur, out=nxt, ids_out=ids[l], ws=ws)
            cur, nxt = nxt, cur
        if events is not None:
            events[len(layers)].record()
        return cur

    graph = None
    if not args.no_graph:
        try:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                xa.copy_(x_bank[0])
                one_step()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                one_step()
            torch.cuda.synchronize()
        except Exception as exc:  # capture unsupported: run the same launches eagerly
            eprint(f"[bench] graph capture failed ({exc!r}); running eagerly")
            graph = None
    run = graph.replay if graph is not None else one_step

    for s in range(args.warmup):
        xa.copy_(x_bank[args.steps + s])
        run()
    torch.cuda.synchronize()

    ids_hist = torch.empty((args.steps, args.layers, T, k), dtype=torch.int32, device=dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for s in range(args.steps):
        xa.copy_(x_bank[s])
        run()
        ids_hist[s].copy_(ids)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end)

    ids_np = ids_hist.cpu().numpy().reshape(args.steps, args.layers, T * k)
    U = np.array([[len(np.unique(ids_np[s, l])) for l in range(args.layers)] for s in range(args.steps)])
    total_bytes = float(layer_bytes(U, T, H).sum())
    gbs = total_bytes / (ms / 1e3) / 1e9
    per_layer_us = ms * 1e3 / (args.steps * args.layers)
    per_layer_bytes = total_bytes / (args.steps * args.layers)
    eprint(f"[bench] {args.steps} steps in {ms:.1f} ms; distinct experts/layer mean {U.mean():.2f} "
           f"min {U.min()} max {U.max()}; {per_layer_us:.2f} us/layer; graph={graph is not None}")

    from vates_amd.moe import workspace_status
    status = workspace_status(ws)
    if status:
        eprint(f"[bench] device status flags {status:#x}")
        return 3

    lat = peak = None
    if not args.no_ceiling:
        lat = layer_latency(one_step, len(layers), xa, x_bank, min(args.steps, 40))
        eprint(f"[bench] layer call latency: p50 {lat['p50_us']} us, p99 {lat['p99_us']} us, "
               f"mean {lat['mean_us']} us over {lat['samples']} calls ({lat['marker_cost_us']} us of event markers)")
        peak = measure_stream_peak()
        eprint(f"[bench] measured read ceiling {peak['gbs']} GB/s (nt {peak['nontemporal_gbs']}, "
               f"cached {peak['cached_gbs']})")

    parity = moe_parity(layers, ws_list, x_bank[0], args)
    eprint(f"[bench] first two layers against the oracle: {parity}")
    cpu = cpu1 = None
    if args.cpu_baseline_s > 0:
        xs_host = x_bank[: args.steps].view(torch.int16).cpu().numpy().view(np.uint16)
        cpu = cpu_baseline(ws_list, xs_host, args, args.cpu_baseline_s)
        cpu1 = cpu_baseline(ws_list, xs_host, args, max(2.0, args.cpu_baseline_s / 3), threads=1)
        eprint(f"[bench] oracle on the host: {cpu['value']} GB/s ({cpu['cores']} cores), {cpu1['value']} GB/s (1 core)")
    hip_graph = graph is not None
    decode = None
    if not args.no_decode and args.layers == 48 and args.hidden == 2048:
        del layers, ws_list, graph, run
        torch.cuda.empty_cache()
        decode = decode_record(args)

    achieved = per_layer_bytes / (per_layer_us * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 weights x f16 MFMA, f32 accumulate (bf16 in/out)",
        "data": "synthetic",
        "config": {
            "workload": f"{args.layers}-layer MoE-only verify stack, T={T}, {args.experts} experts top-{k}, "
                        f"hidden {H}, inter {args.inter}, 4-bit g64 experts, 8-bit router, shared expert, "
                        f"Zipf(1.1) routing bias, {args.steps} steps",
            "layers": args.layers, "T": T, "top_k": k, "experts": args.experts, "hidden": H, "inter": args.inter,
            "distinct_experts_per_layer": round(float(U.mean()), 2),
            "hip_graph": hip_graph,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "peak_measured": peak["gbs"] if peak else None,
            "frac_measured": round(achieved / peak["gbs"], 4) if peak else None,
            "peak_measured_source": peak,
            "traffic": round(MOE_TRAFFIC_RATIO * per_layer_bytes) if args.hidden == 2048 and T == 4 else None,
            "traffic_ratio": MOE_TRAFFIC_RATIO if args.hidden == 2048 and T == 4 else None,
            "traffic_source": MOE_TRAFFIC_SOURCE if args.hidden == 2048 and T == 4 else None,
            "p50_us": lat["p50_us"] if lat else None,
            "p99_us": lat["p99_us"] if lat else None,
            "latency": lat,
            "unit_of_work": "one MoE layer call (router+topk, gate/up, down+combine kernels)",
            "bytes_per_launch": round(per_layer_bytes),
            "us_per_launch": round(per_layer_us, 3),
        },
        "cpu_baseline": cpu,
        "cpu_baseline_1core": cpu1,
        "parity": parity,
        "decode": decode,
    }
    print(json.dumps(line), flush=True)
    return 0 if parity["ok"] and (decode is None or decode["config"]["speculative_equals_greedy"]) else 3


if __name__ == "__main__":
    sys.exit(main())
