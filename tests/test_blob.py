"""The expert blob v1 layout and writer (CPU).

Known answers: the Qwen3-Next expert is 1,769,472 bytes (gate and up weights
524,288 B, scales and biases 32,768 B each; down the same sizes transposed),
the stride the reference's layout_for returns (mlx_streaming/prep/
blob_layout.py:18-32).  The writer's byte order is checked with the
reference's byte-pattern idea (tests/test_demand_dual_native.py:28-60: expert
e's bytes are (e + 1) & 0xFF, so every slot's truth is known).
"""
import json

import numpy as np
import pytest
import torch

from vates_amd.blob import BLOB_V1_AFFINE, blob_layout, read_blob_index, write_layer_blob
from vates_amd.moe import QuantizedProj
from vates_amd._lib import VmiError


def test_layout_qwen3_next_known_answer():
    segs, stride = blob_layout(2048, 512, 4, 64)
    assert stride == 1_769_472
    assert [(sg.proj, sg.tensor) for sg in segs] == [(p, t) for p in ("gate_proj", "up_proj", "down_proj")
                                                      for t in ("weight", "scales", "biases")]
    sizes = {(sg.proj, sg.tensor): sg.nbytes for sg in segs}
    assert sizes[("gate_proj", "weight")] == 524_288 and sizes[("up_proj", "weight")] == 524_288
    assert sizes[("down_proj", "weight")] == 524_288
    assert all(sizes[(p, t)] == 32_768 for p in ("gate_proj", "up_proj", "down_proj") for t in ("scales", "biases"))
    shapes = {(sg.proj, sg.tensor): sg.shape for sg in segs}
    # each segment starts where the one before it ends
    assert segs[0].offset == 0 and all(a.offset + a.nbytes == b.offset for a, b in zip(segs, segs[1:]))
    assert segs[-1].offset + segs[-1].nbytes == stride
    assert shapes[("gate_proj", "weight")] == (512, 256) and shapes[("down_proj", "weight")] == (2048, 64)
    assert shapes[("down_proj", "scales")] == (2048, 8)
    # 8-bit: twice the words
    assert blob_layout(2048, 512, 8, 64)[1] == 3 * (512 * 512 * 4 + 2 * 512 * 32 * 2)


def _pattern_proj(E, out_d, in_d, bits, group, tag):
    w = torch.empty((E, out_d, in_d * bits // 32), dtype=torch.int32)
    s = torch.empty((E, out_d, in_d // group), dtype=torch.int16)
    b = torch.empty_like(s)
    for e in range(E):
        for t, v in ((w, (e + 1) & 0xFF), (s, (e + 100) & 0xFF), (b, (e + 7 * tag) & 0xFF)):
            t[e].view(torch.uint8).fill_(v)
    return QuantizedProj(w, s, b)


def test_writer_byte_order(tmp_path):
    E, H, I = 5, 128, 64
    g, u, d = (_pattern_proj(E, I, H, 4, 64, 1), _pattern_proj(E, I, H, 4, 64, 2), _pattern_proj(E, H, I, 4, 64, 3))
    path = tmp_path / "layer00.blob"
    stride = write_layer_blob(path, g, u, d)
    segs, want = blob_layout(H, I, 4, 64)
    assert stride == want
    raw = np.fromfile(path, dtype=np.uint8)
    assert raw.size == E * stride
    for e in range(E):
        for sg, val in zip(segs, [((e + 1) & 0xFF), ((e + 100) & 0xFF), ((e + 7) & 0xFF),
                                  ((e + 1) & 0xFF), ((e + 100) & 0xFF), ((e + 14) & 0xFF),
                                  ((e + 1) & 0xFF), ((e + 100) & 0xFF), ((e + 21) & 0xFF)]):
            off = e * stride + sg.offset
            assert np.all(raw[off:off + sg.nbytes] == val), (e, sg.proj, sg.tensor)


def test_blob_index(tmp_path):
    meta = {"format": BLOB_V1_AFFINE, "quant_mode": "affine", "stride": 1769472, "num_experts": 512,
            "layers": [0, 1], "bits": 4, "group_size": 64, "page_aligned": True}
    (tmp_path / "blob_index.json").write_text(json.dumps(meta))
    assert read_blob_index(tmp_path)["stride"] == 1769472
    meta["format"] = "expert_blob_v2_mxfp4"
    (tmp_path / "blob_index.json").write_text(json.dumps(meta))
    with pytest.raises(VmiError):
        read_blob_index(tmp_path)
