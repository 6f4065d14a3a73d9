"""Commit of a verify step on the caches (host logic only, CPU tensors).

The reference's known answers (tests/golden/reference_known_answers.json,
written from mlx_streaming/tests/test_mtp_generate.py:575-606):
* commit_kv_trim: an attention cache holding 5 verified positions, committed
  with accepted_len 3, keeps 3 (offset_after);
* commit_checkpoint: a linear-attention cache with per-token checkpoints
  [conv, ssm] = [1, 10], [2, 20], [3, 30] for 3 verified tokens, committed with
  accepted_len 2, continues from checkpoint 1: every conv element 2 (sum 24
  over [1, 3, 4]) and every state element 20 (sum 80 over [1, 2, 2]).
Here the conv state after a token is the ring's last three conv rows ending at
that token and the recurrent state sits in the ring slot of the next position;
the test fills the rows and slots with the checkpoint values and checks the
committed cache reads back checkpoint 1's.
"""
import json
from pathlib import Path

import pytest

FIX = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def test_commit_kv_trim_known_answer():
    from vates_amd.attention import KVCache
    from vates_amd.decode import commit_verified_prefix
    fx = FIX["commit_kv_trim"]
    c = KVCache(2, 64, "cpu")
    c.length = fx["tokens"]
    assert commit_verified_prefix([c, None], verified_len=fx["verified_len"], accepted_len=fx["accepted_len"])
    assert c.length == fx["offset_after"]


def test_commit_checkpoint_known_answer():
    """The reference's checkpoint commit (kv_cache.py:222-251) on its own
    fixture, translated to the rings: the reference keeps, per verified token
    j, a (conv window, state) checkpoint and restores token acc-1's; here
    token j's conv input is ring row (pos0 + j) % 32 and the state after it is
    state slot (pos0 + j + 1) % n_slots, so committing is setting the length to
    pos0 + acc.  The state before that length must be the fixture's state sum
    (80 over its 4 elements), and the whole 3-row conv window before it must be
    the rows of positions pos0 + acc - 3 .. pos0 + acc - 1: the row before the
    batch (never written, zero), then tokens 0 and 1, the newest carrying the
    fixture's conv sum (24 over its 12 elements).  (The fixture fills each
    checkpoint uniformly, so only its newest row has a counterpart here.)"""
    import torch
    from vates_amd.decode import commit_verified_prefix
    from vates_amd.gdn import GdnCache
    fx = FIX["commit_checkpoint"]
    n, acc = fx["verified_len"], fx["accepted_len"]
    conv_vals = [ck[0] for ck in fx["checkpoints"]]
    ssm_vals = [ck[1] for ck in fx["checkpoints"]]
    pos0 = 37  # the verify batch's first position
    c = GdnCache(1, 1, n + 1, "cpu")
    for j in range(n):  # token j: its conv row and the state after it
        c.conv[(pos0 + j) % c.conv.shape[0]] = conv_vals[j]
        c.state[(pos0 + j + 1) % c.n_slots] = ssm_vals[j]
    c.length = pos0 + n
    assert commit_verified_prefix([c], verified_len=n, accepted_len=acc)
    assert c.length == pos0 + acc
    st = c.state_before(c.length)
    assert torch.all(st == fx["sums_after"][1] / 4.0)          # 80 over the fixture's 4 elements
    rows = c.conv_rows(c.length)
    assert tuple(rows.shape) == (3, c.conv_dim)
    assert torch.all(rows[-1] == fx["sums_after"][0] / 12.0)   # 24 over the fixture's 12 elements
    assert torch.all(rows[-2] == conv_vals[acc - 2])
    assert acc == 2 and torch.all(rows[-3] == 0)               # position pos0 - 1: before the batch


def test_commit_rejects_bad_lengths():
    from vates_amd._lib import VmiError
    from vates_amd.attention import KVCache
    from vates_amd.decode import commit_verified_prefix
    c = KVCache(2, 64, "cpu")
    c.length = 4
    with pytest.raises(VmiError):
        commit_verified_prefix([c], verified_len=3, accepted_len=4)
    with pytest.raises(VmiError):
        commit_verified_prefix([c], verified_len=9, accepted_len=1)  # more than the cache holds
