"""vmi_moe_layer_noalloc (static device scratch, no workspace argument, no
allocation) against vmi_moe_layer on the same inputs, through the C ABI.

Bar: bit-exact (the same kernels run on a different buffer).  Two calls in a
row on the shared scratch, the second with a smaller batch, so that a result
depending on the first call's leftovers would show.
"""
import ctypes
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_noalloc_equals_workspace_entry(gpu):
    import torch
    import vates_amd._lib as L
    from vates_amd.synth import synth_bf16
    from vates_amd.workload import make_layer, synth_layer

    lib = L.load()
    w = synth_layer(31, 0, hidden=2048, inter=512, num_experts=512, zipf_alpha=0.5, device=gpu)
    moe = make_layer(w, top_k=10)
    stream = torch.cuda.current_stream().cuda_stream
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    for T, seed in ((9, 901), (4, 902)):
        log(f"case: noalloc vs workspace entry, hidden 2048, 512 experts top-10, T={T}")
        x = synth_bf16(seed, 1, (T, 2048), device=gpu)
        res = synth_bf16(seed, 2, (T, 2048), device=gpu)
        ref = torch.empty_like(x)
        ids_ref = torch.empty((T, 10), dtype=torch.int32, device=gpu)
        sc_ref = torch.empty((T, 10), dtype=torch.float32, device=gpu)
        ws = torch.zeros(moe.workspace_bytes(T), dtype=torch.uint8, device=gpu)
        rc = lib.vmi_moe_layer(ctypes.byref(moe.desc), x.data_ptr(), T, res.data_ptr(), ref.data_ptr(),
                               ids_ref.data_ptr(), sc_ref.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        L.check(rc, "vmi_moe_layer")
        got = torch.full_like(x, float("nan"))
        ids = torch.full((T, 10), -7, dtype=torch.int32, device=gpu)
        sc = torch.full((T, 10), float("nan"), dtype=torch.float32, device=gpu)
        rc = lib.vmi_moe_layer_noalloc(ctypes.byref(moe.desc), x.data_ptr(), T, res.data_ptr(), got.data_ptr(),
                                       ids.data_ptr(), sc.data_ptr(), status.data_ptr(), stream)
        L.check(rc, "vmi_moe_layer_noalloc")
        torch.cuda.synchronize()
        assert np.array_equal(got.view(torch.int16).cpu().numpy(), ref.view(torch.int16).cpu().numpy()), T
        assert np.array_equal(ids.cpu().numpy(), ids_ref.cpu().numpy()), T
        assert np.array_equal(sc.view(torch.int32).cpu().numpy(), sc_ref.view(torch.int32).cpu().numpy()), T
        assert int(status.item()) == 0
    # a bad slot table entry reaches the caller's status word
    log("case: noalloc status word")
    bad = moe.desc.slot_table
    table = torch.full((512,), 10**6, dtype=torch.int32, device=gpu)
    moe.desc.slot_table = table.data_ptr()
    x = synth_bf16(903, 1, (2, 2048), device=gpu)
    out = torch.empty_like(x)
    rc = lib.vmi_moe_layer_noalloc(ctypes.byref(moe.desc), x.data_ptr(), 2, None, out.data_ptr(), None, None,
                                   status.data_ptr(), stream)
    moe.desc.slot_table = bad
    L.check(rc, "vmi_moe_layer_noalloc")
    torch.cuda.synchronize()
    assert int(status.item()) & L.VMI_STATUS_BAD_SLOT


def test_noalloc_rejects_bad_arguments(gpu):
    import vates_amd._lib as L
    from vates_amd.workload import make_layer, synth_layer

    lib = L.load()
    w = synth_layer(32, 0, hidden=512, inter=128, num_experts=64, device=gpu)
    moe = make_layer(w, top_k=4)
    rc = lib.vmi_moe_layer_noalloc(ctypes.byref(moe.desc), None, 4, None, None, None, None, None, None)
    assert rc == L.VMI_ERR_INVALID
