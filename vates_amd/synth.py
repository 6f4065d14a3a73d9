"""Synthetic weights and activations generated on the GPU by libvmi.

Element i of (seed, stream) is ((sum of the four 16-bit words of
Philox4x32-10 block i//2, half i%2) - 131070) * scale with
scale = std / IRWIN_HALL_STD, i.e. an Irwin-Hall(4) approximation of
N(0, std^2).  Quantised tensors use per-64-column min/max affine groups with
bf16 scale and bias.  The CPU oracle implements the same integer recipe, so
both sides see bit-identical tensors.
"""
from __future__ import annotations

import math

import torch

from ._lib import check, load
from .moe import QuantizedProj

# std of the sum of four independent uniform 16-bit words
IRWIN_HALL_STD = math.sqrt(4.0 * (65536.0 ** 2 - 1.0) / 12.0)


def scale_for(std: float) -> float:
    return std / IRWIN_HALL_STD


def _stream(stream) -> int:
    return (stream or torch.cuda.current_stream()).cuda_stream


def synth_proj(seed: int, stream_id: int, n: int, out_dim: int, in_dim: int, *, bits: int = 4, std: float = 0.02,
               group: int = 64, device=None, stream=None) -> QuantizedProj:
    """A [n, out_dim, in_dim] projection stack, rows drawn as one stream."""
    device = torch.device(device or "cuda")
    w = torch.empty((n, out_dim, in_dim * bits // 32), dtype=torch.int32, device=device)
    s = torch.empty((n, out_dim, in_dim // group), dtype=torch.int16, device=device)
    b = torch.empty_like(s)
    rc = load().vmi_synth_quantized(seed, stream_id, n * out_dim, in_dim, group, bits, scale_for(std), w.data_ptr(),
                                    s.data_ptr(), b.data_ptr(), _stream(stream))
    check(rc, "vmi_synth_quantized")
    return QuantizedProj(w, s, b)


def synth_bf16(seed: int, stream_id: int, shape, *, std: float = 1.0, device=None, stream=None) -> torch.Tensor:
    device = torch.device(device or "cuda")
    out = torch.empty(tuple(shape), dtype=torch.bfloat16, device=device)
    rc = load().vmi_synth_bf16(seed, stream_id, out.numel(), scale_for(std), out.data_ptr(), _stream(stream))
    check(rc, "vmi_synth_bf16")
    return out
