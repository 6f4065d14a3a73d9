"""The expert-pool layouts MoELayer stores (host-side tensor permutations, CPU).

gateup_mfma_major: word (c, w, m, l, j) of expert n holds the reference
layout's word at row 64 c + 16 w + (l % 16), word 16 m + 4 (l // 16) + j (the
16 bytes at byte 64 m + 16 q of that row for lane l = 16 q + r).
down_group_major: word (n, g, h, j) holds the reference word (n, h, 8 g + j),
scales and biases (n, g, h) hold (n, h, g).
Both are checked element by element against those formulas and round-tripped
through their inverses bit for bit.
"""
import numpy as np
import torch

from vates_amd.moe import (QuantizedProj, down_group_major, down_reference_layout, gateup_mfma_major,
                           gateup_reference_layout)


def _proj(rng, n, rows, words, groups):
    w = torch.from_numpy(rng.integers(-2**31, 2**31 - 1, (n, rows, words), dtype=np.int64).astype(np.int32))
    s = torch.from_numpy(rng.integers(0, 2**16, (n, rows, groups), dtype=np.int64).astype(np.int16)).view(
        torch.bfloat16)
    b = torch.from_numpy(rng.integers(0, 2**16, (n, rows, groups), dtype=np.int64).astype(np.int16)).view(
        torch.bfloat16)
    return QuantizedProj(w, s, b)


def _bits(t):
    return t.contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32).numpy()


def test_gateup_mfma_major_positions_and_inverse():
    rng = np.random.default_rng(3)
    n, inter, hidden = 3, 128, 512
    words = hidden * 4 // 32
    p = _proj(rng, n, inter, words, hidden // 64)
    q = gateup_mfma_major(p)
    W = _bits(p.weight)
    M = _bits(q.weight).reshape(n, inter // 64, 4, words // 16, 64, 4)
    for _ in range(400):
        e, c, w, m, l, j = (int(rng.integers(0, v)) for v in (n, inter // 64, 4, words // 16, 64, 4))
        assert M[e, c, w, m, l, j] == W[e, 64 * c + 16 * w + (l % 16), 16 * m + 4 * (l // 16) + j]
    # one wave's block is 1 KB of contiguous memory
    flat = _bits(q.weight).reshape(-1)
    blk = flat[(((1 * (inter // 64) + 1) * 4 + 2) * (words // 16) + 3) * 256:][:256].reshape(64, 4)
    rows = 64 + 32 + np.arange(64) % 16
    cols = 48 + 4 * (np.arange(64) // 16)
    assert np.array_equal(blk, np.stack([W[1, rows, cols + j] for j in range(4)], axis=1))
    assert np.array_equal(_bits(q.scales), _bits(p.scales)) and np.array_equal(_bits(q.biases), _bits(p.biases))
    r = gateup_reference_layout(q)
    for a, b in ((r.weight, p.weight), (r.scales, p.scales), (r.biases, p.biases)):
        assert a.shape == b.shape and np.array_equal(_bits(a), _bits(b))


def test_down_group_major_positions_and_inverse():
    rng = np.random.default_rng(4)
    n, hidden, inter = 2, 512, 192
    G = inter // 64
    p = _proj(rng, n, hidden, inter * 4 // 32, G)
    q = down_group_major(p)
    assert tuple(q.weight.shape) == (n, G, hidden, 8) and tuple(q.scales.shape) == (n, G, hidden)
    W, M = _bits(p.weight), _bits(q.weight)
    S, MS = _bits(p.scales), _bits(q.scales)
    for _ in range(400):
        e, g, h, j = (int(rng.integers(0, v)) for v in (n, G, hidden, 8))
        assert M[e, g, h, j] == W[e, h, 8 * g + j]
        assert MS[e, g, h] == S[e, h, g]
    r = down_reference_layout(q)
    for a, b in ((r.weight, p.weight), (r.scales, p.scales), (r.biases, p.biases)):
        assert a.shape == b.shape and np.array_equal(_bits(a), _bits(b))
