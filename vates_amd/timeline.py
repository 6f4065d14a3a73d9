"""Stage timeline of one MoE verify layer call, read from the kernels' own
stamps.

The stamped tuning build (``python -m vates_amd.build --timeline`` writes
vates_amd/libvmi_timeline.so) makes the first lane of every workgroup record
the 100 MHz real-time counter at fixed points of the layer's three kernels:

  k_router       0 start, 1 end (first wave), 8.. every wave's end
  k_experts      0 start, 9 top-k keys loaded, 10 top-k rounds done,
                 1 routing done, 2 slot dedup done, 3 gate/up weights landed,
                 4 SwiGLU barrier passed, 7 down loop start, 6 end
  k_moe_combine  0 start, 1 end

Usage: python -m vates_amd.timeline [--T 4] [--reps 20]

Runs a 4-layer stack of the 48-layer benchmark's layer (hidden 2048, 512
experts top-10, inter 512, 8-bit router, shared expert, Zipf(1.1) routing
bias alpha 0.5) captured in one HIP graph, replayed `reps` times with 512 MiB
of unrelated writes between replays (so the weights come from HBM as in the
48-layer stack), and prints the medians over replays of the last layer's
stage boundaries in microseconds from its router's first stamp: per stage the
median workgroup and the last one.
"""
from __future__ import annotations

import argparse
import ctypes
import sys
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent


def run(T: int = 4, reps: int = 20) -> list:
    import vates_amd._lib as L
    L.LIB_PATH = PKG / "libvmi_timeline.so"  # before the first load in this process
    if not L.LIB_PATH.exists():
        raise SystemExit(f"{L.LIB_PATH} is not built: python -m vates_amd.build --timeline")
    lib = L.load()
    import torch
    from vates_amd.synth import synth_bf16
    from vates_amd.workload import make_layer, synth_layer

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    NL = 4
    layers = [make_layer(synth_layer(1234, l, hidden=2048, inter=512, num_experts=512, zipf_s=1.1, zipf_alpha=0.5,
                                     device=dev), top_k=10) for l in range(NL)]
    buf = torch.zeros(3 * 4096 * 16, dtype=torch.int64, device=dev)
    lib.vmi_timeline_set.argtypes = [ctypes.c_void_p]
    if lib.vmi_timeline_set(buf.data_ptr()) != 0:
        raise RuntimeError("vmi_timeline_set failed")
    xs = synth_bf16(1234, 0x7171, (16, T, 2048), device=dev)
    xa, xb, xc = (torch.empty((T, 2048), dtype=torch.bfloat16, device=dev) for _ in range(3))
    ws = torch.zeros(layers[0].workspace_bytes(T), dtype=torch.uint8, device=dev)
    fill = torch.zeros(512 * 2**20 // 4, dtype=torch.float32, device=dev)

    def step():
        cur = xa
        for i, layer in enumerate(layers):
            nxt = (xb, xc)[i % 2]
            layer(cur, residual=cur, out=nxt, ws=ws)
            cur = nxt

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        xa.copy_(xs[0])
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()

    stages = [("router", 0, 0, "start (first)"), ("router", 0, 1, "end (first wave)"),
              ("router", 0, -8, "end (last wave)"),
              ("experts", 1, 0, "start"), ("experts", 1, 9, "top-k keys loaded"),
              ("experts", 1, 10, "top-k rounds done"), ("experts", 1, 1, "routing done"),
              ("experts", 1, 2, "slot dedup done"), ("experts", 1, 3, "gate/up weights landed"),
              ("experts", 1, 4, "SwiGLU barrier passed"), ("experts", 1, 7, "down loop start"),
              ("experts", 1, 6, "end"), ("combine", 2, 0, "start"), ("combine", 2, 1, "end")]
    med = {i: [] for i in range(len(stages))}
    last = {i: [] for i in range(len(stages))}
    for rep in range(reps):
        xa.copy_(xs[rep % 16])
        fill.add_(1.0)
        buf.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        b = buf.view(3, 4096, 16).cpu().numpy()
        t0 = b[0, :, 0][b[0, :, 0] > 0].min()
        real = b[1, :, 6] > 0  # expert workgroups that ran an item (the rest exit after routing)
        for i, (_, kid, slot, _) in enumerate(stages):
            v = b[kid, :, slot] if slot >= 0 else b[kid, :, -slot:-slot + 4].max(axis=1)
            sel = (v > 0) & (real if kid == 1 and slot in (3, 4, 7, 6) else True)
            us = (v[sel] - t0) * 0.01
            med[i].append(float(np.median(us)) if us.size else float("nan"))
            last[i].append(float(us.max()) if us.size else float("nan"))
    rows = []
    for i, (kern, _, slot, what) in enumerate(stages):
        m, x = np.array(med[i][2:]), np.array(last[i][2:])  # the first two replays warm up
        rows.append((kern, slot, what, float(np.median(m)), float(np.median(x))))
    return rows


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--T", type=int, default=4)
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()
    rows = run(args.T, args.reps)
    print(f"| kernel | stamp | point | median workgroup (us) | last workgroup (us) |")
    print("|---|---|---|---|---|")
    for kern, slot, what, m, x in rows:
        print(f"| {kern} | {slot} | {what} | {m:.2f} | {x:.2f} |")
    sys.stdout.flush()
    return 0


if __name__ == "__main__":
    sys.exit(main())
