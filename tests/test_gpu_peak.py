"""The measurement kernels behind the benchmark's measured ceilings.

vmi_stream_read must read every byte it is given: the XOR of its per-workgroup
words equals numpy's XOR of the buffer, for nontemporal and cached loads, with
a tail that is not a whole 32 KB chunk.  vmi_mfma_peak's checksum equals the
product the MFMA lane layout defines (lane l supplies A[l % 16][8 (l / 16) + s] and
B[8 (l / 16) + s][l % 16], and holds D[4 (l / 16) + e][l % 16]), built here
from that layout with numpy: a wrong operand order or layout fails it.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_stream_read_reads_every_word(gpu):
    import torch
    from vates_amd._lib import check, load
    lib = load()
    rng = np.random.default_rng(5)
    for nbytes in (16, 32768 * 3 + 48, (1 << 22) + 16 * 37):
        host = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
        buf = torch.from_numpy(host.view(np.int32)).to(gpu)
        for nt in (1, 0):
            for wgs in (1, 7, 512):
                log(f"case: stream_read bytes={nbytes} nt={nt} workgroups={wgs}")
                sink = torch.full((wgs,), -1, dtype=torch.int32, device=gpu)
                check(lib.vmi_stream_read(buf.data_ptr(), nbytes, nt, wgs, sink.data_ptr(),
                                          torch.cuda.current_stream().cuda_stream), "vmi_stream_read")
                torch.cuda.synchronize()
                got = int(np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)))
                assert got == int(np.bitwise_xor.reduce(host))


def test_stream_read_rejects_bad_arguments(gpu):
    import torch
    from vates_amd._lib import VMI_ERR_INVALID, load
    lib = load()
    buf = torch.zeros(64, dtype=torch.int32, device=gpu)
    sink = torch.zeros(1, dtype=torch.int32, device=gpu)
    assert lib.vmi_stream_read(buf.data_ptr(), 20, 1, 4, sink.data_ptr(), None) == VMI_ERR_INVALID
    assert lib.vmi_stream_read(buf.data_ptr() + 4, 16, 1, 4, sink.data_ptr(), None) == VMI_ERR_INVALID
    assert lib.vmi_stream_read(buf.data_ptr(), 64, 1, 0, sink.data_ptr(), None) == VMI_ERR_INVALID
    assert lib.vmi_mfma_peak(0, 4, sink.data_ptr(), None) == VMI_ERR_INVALID


def _operand(lane_vals):
    """[64 lanes][8] operand values -> (A [16][32], B [32][16]) per the layout."""
    A = np.zeros((16, 32))
    B = np.zeros((32, 16))
    for l in range(64):
        for s in range(8):
            A[l % 16, 8 * (l // 16) + s] = lane_vals[l][s]
            B[8 * (l // 16) + s, l % 16] = lane_vals[l][s]
    return A, B


def test_mfma_peak_checksum_matches_layout(gpu):
    import torch
    from vates_amd._lib import check, load
    lib = load()
    av = [[((l + i) & 7) / 1024.0 for i in range(8)] for l in range(64)]
    bv = [[((l * 3 + i) & 7) / 1024.0 for i in range(8)] for l in range(64)]
    Aa, Ba = _operand(av)
    Ab, Bb = _operand(bv)
    # chains (A operand, B operand): (a, b), (b, a), (a, a), (b, b); lane 0
    # holds D[e][0] in element e, and the kernel sums chain j's element j
    D = [Aa @ Bb, Ab @ Ba, Aa @ Ba, Ab @ Bb]
    for iters in (1, 3):
        log(f"case: mfma_peak iters={iters}")
        want = np.float32(sum(np.float32(iters * D[j][j, 0]) for j in range(4)))
        sink = torch.full((5,), -1.0, dtype=torch.float32, device=gpu)
        check(lib.vmi_mfma_peak(5, iters, sink.data_ptr(), torch.cuda.current_stream().cuda_stream),
              "vmi_mfma_peak")
        torch.cuda.synchronize()
        got = sink.cpu().numpy()
        assert np.all(got == want), (got, want)
