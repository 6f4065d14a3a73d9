"""GPU acceptance kernels against the CPU oracle: every result record is
bit-exact (integer work and IEEE-double decisions on integer masses).

Greedy: the reference's literal accept_prefix answers
(tests/test_mtp_generate.py:211-223, kept in tests/golden), random chains in
both verify layouts and P-path trees.  Stochastic: random small vocabularies
with and without draft logits, the full 151,936 vocabulary with target logits
N(0, 3) and a planted argmax agreement of 0.7 at temperature 0.7 / top-p 0.9,
and the edge cases (identical draft, a row without finite logits: the failure
record, VMI_STATUS_BAD_LOGITS in the caller's status word, VmiError without
one); a device-side counter offset adds to the host one; a wait bound of one
poll makes the co-residency waits give up, which every workgroup survives: the
failure record, VMI_STATUS_WAIT_GAVE_UP, the workspace counters back at zero.
"""
import json
import sys
from pathlib import Path

import numpy as np
import pytest

from vates_amd._lib import VMI_STATUS_BAD_LOGITS, VMI_STATUS_WAIT_GAVE_UP, VmiError

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_known_answers.json"


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _t(a, dev, dtype=None):
    import torch
    return torch.as_tensor(np.ascontiguousarray(a), device=dev, dtype=dtype)


def test_greedy_reference_known_answers(gpu, orc):
    log("case: greedy accept, reference known answers")
    import torch
    from vates_amd.accept import accept_greedy, decode_result
    for case in json.loads(GOLDEN.read_text())["accept_prefix"]:
        d = _t(np.array(case["drafts"], np.int32), gpu)
        p = _t(np.array(case["preds"], np.int32), gpu)
        r = decode_result(accept_greedy(d, p, mode=0).cpu())
        assert r["matched"] == case["matched"]


@pytest.mark.parametrize("mode", [0, 1])
def test_greedy_random_chains(gpu, orc, mode):
    log(f"case: greedy accept random chains mode={mode}")
    import torch
    from vates_amd.accept import accept_greedy, decode_result
    rng = np.random.default_rng(40 + mode)
    for _ in range(200):
        K = int(rng.integers(1, 16))
        drafts = rng.integers(0, 4, K).astype(np.int32)
        preds = np.where(rng.random(K + mode) < 0.7, np.append(drafts, 0)[:K + mode],
                         rng.integers(0, 4, K + mode)).astype(np.int32)
        em, m, acc = orc.accept_greedy(drafts, preds, mode)
        r = decode_result(accept_greedy(_t(drafts, gpu), _t(preds, gpu), mode=mode).cpu())
        assert (r["emitted"], r["matched"], r["accepted_len"], r["path"]) == (em, m, acc, 0)


def test_greedy_tree_paths(gpu, orc):
    log("case: greedy tree verify winners")
    import torch
    from vates_amd.accept import accept_greedy, decode_result
    rng = np.random.default_rng(42)
    for _ in range(200):
        P, K = int(rng.integers(1, 70)), int(rng.integers(1, 6))
        paths = rng.integers(0, 3, (P, K)).astype(np.int32)
        preds = rng.integers(0, 3, (P, K)).astype(np.int32)
        best, em, m, acc = orc.accept_tree(paths, preds)
        r = decode_result(accept_greedy(_t(paths, gpu), _t(preds, gpu), mode=0).cpu())
        assert (r["path"], r["emitted"], r["matched"], r["accepted_len"]) == (best, em, m, acc)


def _record(orc, target, draft, drafts, temp, top_p, seed, offset):
    return orc.accept_stochastic(target, draft, drafts, temp, top_p, seed, offset)[3]


@pytest.mark.parametrize("with_draft", [True, False])
def test_stochastic_small_vocab_bit_exact(gpu, orc, with_draft):
    log(f"case: stochastic accept small vocab with_draft={with_draft}")
    import torch
    from vates_amd.accept import accept_stochastic
    rng = np.random.default_rng(50 + with_draft)
    for case in range(120):
        K = int(rng.integers(1, 6))
        V = int(rng.choice([2, 7, 64, 1000, 4099]))
        temp = float(rng.choice([0.7, 1.0, 1.7]))
        top_p = float(rng.choice([0.9, 1.0, 0.5]))
        target = rng.normal(0, 3, (K + 1, V)).astype(np.float32)
        draft = rng.normal(0, 3, (K, V)).astype(np.float32) if with_draft else None
        if case % 3 == 0 and with_draft:
            draft = target[:K] + rng.normal(0, 0.3, (K, V)).astype(np.float32)
        drafts = (orc.sample_top_p(draft, temp, top_p, 7, case) if with_draft
                  else np.argmax(target[:K] + rng.normal(0, 2, (K, V)), axis=1).astype(np.int32))
        seed, offset = int(rng.integers(0, 2**63)), case
        want = _record(orc, target, draft, drafts, temp, top_p, seed, offset)
        got = accept_stochastic(_t(target, gpu), None if draft is None else _t(draft, gpu), _t(drafts, gpu),
                                temperature=temp, top_p=top_p, seed=seed, offset=offset).cpu().numpy()
        assert np.array_equal(got[:4 + want[0]], want[:4 + want[0]]), (case, K, V, got, want)


def test_stochastic_full_vocab_planted(gpu, orc):
    log("case: stochastic accept V=151936 K=3, N(0,3) logits, planted agreement 0.7")
    import torch
    from vates_amd.accept import accept_stochastic
    rng = np.random.default_rng(60)
    K, V = 3, 151936
    hist = np.zeros(K + 1, int)
    for case in range(6):
        target = rng.normal(0, 3, (K + 1, V)).astype(np.float32)
        draft = rng.normal(0, 3, (K, V)).astype(np.float32)
        drafts = np.argmax(draft, axis=1).astype(np.int32)
        for i in range(K):
            if rng.random() < 0.7:
                target[i, drafts[i]] = target[i].max() + 1.0
        for dl in (draft, None):
            want = _record(orc, target, dl, drafts, 0.7, 0.9, 99, case)
            got = accept_stochastic(_t(target, gpu), None if dl is None else _t(dl, gpu), _t(drafts, gpu),
                                    temperature=0.7, top_p=0.9, seed=99, offset=case).cpu().numpy()
            assert np.array_equal(got[:4 + want[0]], want[:4 + want[0]]), (case, got, want)
            hist[want[1]] += 1
    log(f"matched histogram {hist.tolist()}")


def test_stochastic_edges(gpu, orc):
    log("case: stochastic accept edges (identical draft, NaN row)")
    import torch
    from vates_amd.accept import accept_stochastic, decode_result, sample_top_p
    rng = np.random.default_rng(61)
    K, V = 4, 5000
    target = rng.normal(0, 3, (K + 1, V)).astype(np.float32)
    tt = _t(target, gpu)
    for s in range(10):
        drafts = sample_top_p(tt[:K].contiguous(), temperature=0.7, top_p=0.9, seed=3, offset=s)
        r = decode_result(accept_stochastic(tt, tt[:K].contiguous(), drafts, temperature=0.7, top_p=0.9, seed=4,
                                            offset=s).cpu())
        assert r["matched"] == K and r["emitted"][:K] == drafts.cpu().tolist()
    bad = target.copy()
    bad[2] = np.nan
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    r = decode_result(accept_stochastic(_t(bad, gpu), None, _t(np.zeros(K, np.int32), gpu), temperature=0.7,
                                        top_p=0.9, seed=1, offset=0, status=status).cpu())
    assert r["path"] == -1 and r["emitted"] == []
    assert int(status.item()) == VMI_STATUS_BAD_LOGITS
    with pytest.raises(VmiError, match="finite"):
        accept_stochastic(_t(bad, gpu), None, _t(np.zeros(K, np.int32), gpu), temperature=0.7, top_p=0.9, seed=1,
                          offset=0)
    # the status word is the caller's: a later good call leaves it as it was
    accept_stochastic(tt, None, _t(np.zeros(K, np.int32), gpu), temperature=0.7, top_p=0.9, seed=1, offset=0,
                      status=status)
    assert int(status.item()) == VMI_STATUS_BAD_LOGITS


def test_offset_device_adds_to_offset(gpu, orc):
    """offset_device (a device word read when the kernel runs) adds to offset:
    the draws equal the oracle's at the sum."""
    log("case: sampling and stochastic accept with a device-side counter offset")
    import torch
    from vates_amd.accept import accept_stochastic, sample_top_p
    rng = np.random.default_rng(62)
    K, V = 3, 3000
    target = rng.normal(0, 3, (K + 1, V)).astype(np.float32)
    draft = rng.normal(0, 3, (K, V)).astype(np.float32)
    dev_off = torch.tensor([1 << 40], dtype=torch.int64, device=gpu)
    for off in (0, 5, 63):
        got = sample_top_p(_t(draft, gpu), temperature=0.7, top_p=0.9, seed=8, offset=off,
                           offset_device=dev_off).cpu().numpy()
        assert np.array_equal(got, orc.sample_top_p(draft, 0.7, 0.9, 8, (1 << 40) + off))
        drafts = got.astype(np.int32)
        want = _record(orc, target, draft, drafts, 0.7, 0.9, 9, (1 << 40) + off)
        rec = accept_stochastic(_t(target, gpu), _t(draft, gpu), _t(drafts, gpu), temperature=0.7, top_p=0.9,
                                seed=9, offset=off, offset_device=dev_off).cpu().numpy()
        assert np.array_equal(rec[:4 + want[0]], want[:4 + want[0]])


def test_wait_give_up_is_reported_and_leaves_workspace_clean(gpu, orc):
    """A wait bound of one poll (vmi_set_wait_limit) makes the co-residency
    waits give up while their peers are still on the way: every workgroup
    still exits, the call writes the failure record and sets
    VMI_STATUS_WAIT_GAVE_UP in the caller's status word (and raises without
    one), and the workspace's counters are back at zero for the next call,
    which, with the default bound restored, equals the oracle."""
    log("case: stochastic accept / top-p sampling with a one-poll wait bound")
    import torch
    from vates_amd.accept import accept_stochastic, sample_top_p, set_wait_limit
    from vates_amd.moe import workspace
    rng = np.random.default_rng(63)
    K, V = 3, 151936
    target = rng.normal(0, 3, (K + 1, V)).astype(np.float32)
    draft = rng.normal(0, 3, (K, V)).astype(np.float32)
    drafts = orc.sample_top_p(draft, 0.7, 0.9, 4, 0)
    tt, dd, dr = _t(target, gpu), _t(draft, gpu), _t(drafts, gpu)
    want = _record(orc, target, draft, drafts, 0.7, 0.9, 5, 1)
    sync_bytes = 64 * 64 + 256 + 64 * 4 + 64 * 2048 + 64 * 64  # the counters at the workspace's start
    gave_up = 0
    prev = set_wait_limit(1)
    try:
        for attempt in range(4):
            status = torch.zeros(1, dtype=torch.int32, device=gpu)
            rec = accept_stochastic(tt, dd, dr, temperature=0.7, top_p=0.9, seed=5, offset=1,
                                    status=status).cpu().numpy()
            bits = int(status.item())
            if bits:
                assert bits == VMI_STATUS_WAIT_GAVE_UP and list(rec[:4]) == [0, 0, 0, -1], (bits, rec)
                gave_up += 1
            else:
                assert np.array_equal(rec[:4 + want[0]], want[:4 + want[0]])
            ws = workspace(1, gpu, torch.cuda.current_stream().cuda_stream, tag="accept")
            assert int(ws[:sync_bytes].count_nonzero().item()) == 0
            st2 = torch.zeros(1, dtype=torch.int32, device=gpu)
            toks = sample_top_p(dd, temperature=0.7, top_p=0.9, seed=4, offset=0, status=st2).cpu().numpy()
            if int(st2.item()):
                assert int(st2.item()) == VMI_STATUS_WAIT_GAVE_UP and (toks == -1).any()
                gave_up += 1
        log(f"{gave_up} of 8 calls gave up")
        assert gave_up > 0, "a one-poll bound never gave up"
        with pytest.raises(VmiError):
            for _ in range(8):  # raises at the first call that gives up
                accept_stochastic(tt, dd, dr, temperature=0.7, top_p=0.9, seed=5, offset=1)
    finally:
        set_wait_limit(prev)
    rec = accept_stochastic(tt, dd, dr, temperature=0.7, top_p=0.9, seed=5, offset=1).cpu().numpy()
    assert np.array_equal(rec[:4 + want[0]], want[:4 + want[0]])
    assert np.array_equal(sample_top_p(dd, temperature=0.7, top_p=0.9, seed=4, offset=0).cpu().numpy(), drafts)


@pytest.mark.parametrize("V", [3, 1000, 151936])
def test_sample_top_p_bit_exact(gpu, orc, V):
    log(f"case: sample_top_p V={V}")
    import torch
    from vates_amd.accept import sample_top_p
    rng = np.random.default_rng(70)
    rows = 5
    logits = rng.normal(0, 3, (rows, V)).astype(np.float32)
    for temp, top_p in ((0.7, 0.9), (1.0, 1.0), (0.3, 0.5)):
        want = orc.sample_top_p(logits, temp, top_p, 1234, 77)
        got = sample_top_p(_t(logits, gpu), temperature=temp, top_p=top_p, seed=1234, offset=77).cpu().numpy()
        assert np.array_equal(got, want)


@pytest.mark.parametrize("mode,T,m", [(1, 4, 0), (1, 4, 1), (1, 4, 3), (0, 3, 0), (0, 3, 2), (0, 3, 3), (0, 1, 1),
                                      (0, 2, 0)])
def test_spec_commit_state_update(gpu, orc, mode, T, m):
    """vmi_spec_commit after an acceptance record of either layout (mode 1:
    T = K + 1 rows; mode 0: the reference's T = K rows, accepted_len =
    min(m + 1, T), x = the last draft when all match): H = hid[acc - 1],
    x = the last emitted token, pos += acc, mtp_len += acc,
    mtp_pos = mtp_len + i; expectations from the record's definition."""
    log(f"case: spec_commit mode={mode} T={T} matched={m}")
    import torch
    from vates_amd.accept import accept_greedy, spec_commit
    K = T - mode          # drafts checked
    hidden = 2048
    g = torch.Generator().manual_seed(11 + 7 * m + T + mode)
    drafts = torch.randint(0, 151936, (K,), generator=g, dtype=torch.int32)
    preds = torch.randint(0, 151936, (T,), generator=g, dtype=torch.int32)
    preds[:m] = drafts[:m]
    if m < K:
        preds[m] = (drafts[m] + 1) % 151936
    rec = accept_greedy(drafts.to(gpu), preds.to(gpu), mode=mode)
    hid = torch.randn((T, hidden), generator=g).to(torch.bfloat16).to(gpu)
    H = torch.zeros((1, hidden), dtype=torch.bfloat16, device=gpu)
    x = torch.zeros(1, dtype=torch.int32, device=gpu)
    state = torch.tensor([1000, 400], dtype=torch.int32, device=gpu)
    mtp_pos = torch.zeros(3, dtype=torch.int32, device=gpu)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    spec_commit(rec, hid, H, x, state[0:1], state[1:2], mtp_pos, rows=T, status=status)
    torch.cuda.synchronize()
    r = rec.cpu().tolist()
    acc = m + 1 if mode == 1 else min(m + 1, T)
    assert r[1] == m and r[2] == acc
    emitted = drafts[:m].tolist() + [int(preds[m])] if m < K or mode == 1 else drafts[:K].tolist()
    assert r[4:4 + r[0]] == emitted
    assert torch.equal(H[0].view(torch.int16), hid[acc - 1].view(torch.int16))
    assert int(x) == emitted[-1]
    assert state.cpu().tolist() == [1000 + acc, 400 + acc]
    assert mtp_pos.cpu().tolist() == [400 + acc + i for i in range(3)]
    assert int(status) == 0


def test_spec_commit_rejects_bad_record(gpu):
    """A record whose accepted length exceeds the verify rows (here a mode-1
    record of 4 rows committed as 2) changes nothing and sets
    VMI_STATUS_BAD_RECORD."""
    log("case: spec_commit with an out-of-range record")
    import torch
    from vates_amd._lib import VMI_STATUS_BAD_RECORD
    from vates_amd.accept import accept_greedy, spec_commit
    drafts = torch.tensor([5, 6, 7], dtype=torch.int32, device=gpu)
    preds = torch.tensor([5, 6, 7, 8], dtype=torch.int32, device=gpu)
    rec = accept_greedy(drafts, preds, mode=1)          # accepted_len 4
    hid = torch.ones((4, 512), dtype=torch.bfloat16, device=gpu)
    H = torch.zeros((1, 512), dtype=torch.bfloat16, device=gpu)
    x = torch.full((1,), 99, dtype=torch.int32, device=gpu)
    state = torch.tensor([10, 20], dtype=torch.int32, device=gpu)
    mtp_pos = torch.zeros(3, dtype=torch.int32, device=gpu)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    spec_commit(rec, hid[:2], H, x, state[0:1], state[1:2], mtp_pos, rows=2, status=status)
    torch.cuda.synchronize()
    assert int(status) == VMI_STATUS_BAD_RECORD
    assert state.cpu().tolist() == [10, 20] and int(x) == 99 and not H.float().any()
