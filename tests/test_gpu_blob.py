"""Expert blob v1 into device pools: bit-exact round trip, the byte-pattern
known answer per slot (tests/test_demand_dual_native.py:28-60's idea), and a
MoE layer built from loaded pools equal to one built from the originals."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_blob_round_trip_and_layer(gpu, tmp_path):
    import torch
    from vates_amd.blob import load_layer_blob, write_layer_blob
    from vates_amd.synth import synth_bf16
    from vates_amd.workload import make_layer, synth_layer
    log("case: blob round trip E=64 H=1024 I=256")
    w = synth_layer(61, 2, hidden=1024, inter=256, num_experts=64, device=gpu)
    path = tmp_path / "layer02.blob"
    write_layer_blob(path, w.gate, w.up, w.down)
    got = load_layer_blob(path, 1024, 256, num_experts=64, device=gpu, chunk_bytes=5 << 20)  # several chunks
    for name, ref in (("gate", w.gate), ("up", w.up), ("down", w.down)):
        for a, b in ((got[name].weight, ref.weight), (got[name].scales, ref.scales), (got[name].biases, ref.biases)):
            assert torch.equal(a, b), name
    a = make_layer(w, top_k=8)
    w2 = type(w)(**{**w.__dict__, "gate": got["gate"], "up": got["up"], "down": got["down"]})
    b = make_layer(w2, top_k=8)
    x = synth_bf16(61, 9, (4, 1024), device=gpu)
    ya, yb = a(x, residual=x), b(x, residual=x)
    torch.cuda.synchronize()
    assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))


def test_blob_byte_pattern_per_slot(gpu, tmp_path):
    import torch
    from vates_amd.blob import blob_layout, load_layer_blob
    log("case: blob byte pattern E=33")
    E, H, I = 33, 512, 128
    segs, stride = blob_layout(H, I)
    raw = np.empty((E, stride), dtype=np.uint8)
    for e in range(E):
        for j, sg in enumerate(segs):
            raw[e, sg.offset:sg.offset + sg.nbytes] = (e + 1 + 17 * j) & 0xFF
    path = tmp_path / "layer07.blob"
    raw.tofile(path)
    got = load_layer_blob(path, H, I, device=gpu, chunk_bytes=stride * 4)
    for j, (name, t) in enumerate((n, t) for n in ("gate", "up", "down") for t in ("weight", "scales", "biases")):
        arr = getattr(got[name], t).view(torch.uint8).reshape(E, -1).cpu().numpy()
        for e in range(E):
            assert np.all(arr[e] == ((e + 1 + 17 * j) & 0xFF)), (name, t, e)
    with pytest.raises(Exception):
        load_layer_blob(path, H, I, num_experts=E + 1, device=gpu)
