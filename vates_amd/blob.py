"""Expert blob v1 reader: the reference's on-disk expert layout into HBM pools.

The reference stores the routed experts of one layer in ``layerNN.blob``:
expert e at byte e * stride, its segments in the order gate, up, down and,
for each, weight (uint32 [out, in*bits/32]), scales and biases (bf16 bits,
uint16 [out, in/group]) (layout: mlx_streaming/prep/blob_layout.py:18-32;
reader: BlobExpertSource, mlx_streaming/core/cache/blob_loader.py:24-120;
writer and index files: build_main_core_and_blobs,
mlx_streaming/prep/runtime_bundle.py:162-310).  The reference reads experts
on demand with pread; here every expert of a layer is resident, so a layer is
read in large chunks into pinned host memory, copied to the device in one
transfer per chunk, and scattered on the device into the proj-major pool
stacks ([cap, out, in*bits/32], [cap, out, in/group]) the kernels read.
"""
from __future__ import annotations

import json
import os
from pathlib import Path
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch

from ._lib import VmiError
from .moe import QuantizedProj

BLOB_V1_AFFINE = "expert_blob_v1"


@dataclass(frozen=True)
class BlobSegment:
    """One tensor of an expert's record in a v1 blob."""
    proj: str               # gate_proj, up_proj or down_proj
    tensor: str             # weight, scales or biases
    dtype: str              # uint32: packed quantised words; uint16: bf16 bits
    shape: Tuple[int, int]  # per expert
    offset: int             # bytes from the start of the expert's record
    nbytes: int


def blob_layout(hidden: int, inter: int, bits: int = 4, group: int = 64) -> Tuple[List[BlobSegment], int]:
    """The tensors of one expert's record, in file order, and the record size
    (the expert stride) in bytes.  File order (blob_layout.py:18-32): the
    gate, up and down projections, each as its packed words, then one bf16
    scale and one bf16 bias per quantisation group of each output row."""
    if hidden % group or inter % group or 32 % bits:
        raise VmiError(f"hidden={hidden} inter={inter} must be multiples of group={group}; bits={bits}")
    # (projection, output rows, input columns)
    shapes = (("gate_proj", inter, hidden), ("up_proj", inter, hidden), ("down_proj", hidden, inter))
    segs: List[BlobSegment] = []
    offset = 0
    for proj, rows, cols in shapes:
        per_row = (("weight", "uint32", cols * bits // 32, 4),
                   ("scales", "uint16", cols // group, 2),
                   ("biases", "uint16", cols // group, 2))
        for tensor, dtype, width, itemsize in per_row:
            nbytes = rows * width * itemsize
            segs.append(BlobSegment(proj, tensor, dtype, (rows, width), offset, nbytes))
            offset += nbytes
    return segs, offset


_TORCH = {"uint32": torch.int32, "uint16": torch.int16}


def _pools(segs: List[BlobSegment], num_experts: int, device) -> Dict[str, torch.Tensor]:
    return {f"{sg.proj}.{sg.tensor}": torch.empty((num_experts, *sg.shape), dtype=_TORCH[sg.dtype], device=device)
            for sg in segs}


def load_layer_blob(path, hidden: int, inter: int, *, bits: int = 4, group: int = 64,
                    num_experts: Optional[int] = None, device=None, chunk_bytes: int = 256 << 20,
                    stream=None) -> Dict[str, QuantizedProj]:
    """Reads one layer's blob into device pools; returns {"gate", "up", "down"}
    as QuantizedProj stacks with one entry per expert (slot e = expert e)."""
    device = torch.device(device or "cuda")
    segs, stride = blob_layout(hidden, inter, bits, group)
    size = os.path.getsize(path)
    if size % stride:
        raise VmiError(f"{path}: {size} bytes is not a whole number of {stride}-byte experts")
    E = size // stride
    if num_experts is not None and num_experts != E:
        raise VmiError(f"{path}: holds {E} experts, expected {num_experts}")
    pools = _pools(segs, E, device)
    per = max(1, min(E, chunk_bytes // stride))
    stream = stream or torch.cuda.current_stream(device)
    host = [torch.empty(per * stride, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    dev = [torch.empty(per * stride, dtype=torch.uint8, device=device) for _ in range(2)]
    done = [None, None]
    with open(path, "rb", buffering=0) as f, torch.cuda.stream(stream):
        for n, e0 in enumerate(range(0, E, per)):
            b = n % 2
            cnt = min(per, E - e0)
            if done[b] is not None:
                done[b].synchronize()  # the previous transfer out of this staging pair has finished
            view = memoryview(host[b].numpy())[:cnt * stride]
            got = 0
            while got < cnt * stride:
                r = f.readinto(view[got:])
                if not r:
                    raise VmiError(f"{path}: short read at expert {e0}")
                got += r
            dev[b][:cnt * stride].copy_(host[b][:cnt * stride], non_blocking=True)
            raw = dev[b][:cnt * stride].view(cnt, stride)
            for sg in segs:
                dst = pools[f"{sg.proj}.{sg.tensor}"][e0:e0 + cnt].view(torch.uint8).view(cnt, sg.nbytes)
                dst.copy_(raw[:, sg.offset:sg.offset + sg.nbytes])
            ev = torch.cuda.Event()
            ev.record(stream)
            done[b] = ev
    stream.synchronize()
    return {name: QuantizedProj(pools[f"{proj}.weight"], pools[f"{proj}.scales"], pools[f"{proj}.biases"])
            for name, proj in (("gate", "gate_proj"), ("up", "up_proj"), ("down", "down_proj"))}


def write_layer_blob(path, gate: QuantizedProj, up: QuantizedProj, down: QuantizedProj) -> int:
    """Writes pool stacks as a v1 blob (expert-major, the writer's byte order of
    runtime_bundle.py:230-245); returns the stride."""
    E = gate.weight.shape[0]
    parts = []
    for proj in (gate, up, down):
        for t in (proj.weight, proj.scales, proj.biases):
            parts.append(t.detach().contiguous().cpu().view(torch.uint8).reshape(E, -1))
    raw = torch.cat(parts, dim=1).contiguous()
    with open(path, "wb") as f:
        f.write(raw.numpy().tobytes())
    return raw.shape[1]


def read_blob_index(blob_dir) -> dict:
    """The bundle's experts/blobs/blob_index.json (runtime_bundle.py:298-307):
    format, stride, num_experts, layers, bits, group_size."""
    meta = json.loads((Path(blob_dir) / "blob_index.json").read_text(encoding="utf-8"))
    if meta.get("format") != BLOB_V1_AFFINE or meta.get("quant_mode", "affine") != "affine":
        raise VmiError(f"unsupported blob format {meta.get('format')!r} / {meta.get('quant_mode')!r}")
    return meta


def load_bundle_layers(blob_dir, hidden: int, inter: int, *, device=None) -> Dict[int, Dict[str, QuantizedProj]]:
    """Every layer listed by blob_index.json, checked against its stride."""
    meta = read_blob_index(blob_dir)
    bits, group = int(meta["bits"]), int(meta["group_size"])
    _, stride = blob_layout(hidden, inter, bits, group)
    if int(meta["stride"]) != stride:
        raise VmiError(f"blob stride {meta['stride']} != {stride} for hidden={hidden} inter={inter}")
    return {int(l): load_layer_blob(Path(blob_dir) / f"layer{int(l):02d}.blob", hidden, inter, bits=bits,
                                    group=group, num_experts=int(meta["num_experts"]), device=device)
            for l in meta["layers"]}
