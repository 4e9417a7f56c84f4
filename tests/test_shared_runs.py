"""Host logic of ``SharedRuns`` (the shared-run decode's work split): every
key of a request's shared part lies in exactly one run piece it reads or in
its tail, and a block table that does not start with the named runs is
refused."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd.ccpe import SharedRuns

BS = 16


def build(n_runs=5, run_blocks=32, slots=3, batch=8, own=3, seed=3):
    rng = np.random.default_rng(seed)
    runs = torch.arange(n_runs * run_blocks, dtype=torch.int32).view(n_runs, run_blocks)
    request_runs = torch.tensor(np.stack([rng.permutation(n_runs)[:slots] for _ in range(batch)]))
    table = torch.cat([runs[request_runs].reshape(batch, -1),
                       n_runs * run_blocks + torch.arange(batch * own, dtype=torch.int32).view(batch, own)], 1)
    return table, runs, request_runs


@pytest.mark.parametrize("margin, pieces", [(256, 2), (16, 1), (512, 4), (1040, 2)])
def test_every_shared_key_is_read_once(margin, pieces):
    table, runs, request_runs = build()
    shared = SharedRuns(table, runs, request_runs, BS, margin=margin, pieces=pieces)
    n_runs, run_blocks = runs.shape
    run_keys, piece_keys = run_blocks * BS, run_blocks * BS // pieces
    tail_key = shared.tail_block * BS
    assert tail_key == request_runs.shape[1] * run_keys - margin
    assert torch.equal(shared.tail_table, table[:, shared.tail_block:])
    qpos = shared.head_qpos.numpy()
    for b in range(table.shape[0]):
        seen = np.zeros(request_runs.shape[1] * run_keys, dtype=int)
        for item in range(shared.head_items):
            r, k = divmod(item, pieces)
            # the piece's blocks are the run's blocks k * piece .. (k + 1) * piece
            assert torch.equal(shared.head_table[item], runs[r, k * (run_blocks // pieces):(k + 1) * (run_blocks // pieces)])
            slot = np.flatnonzero(request_runs[b].numpy() == r)
            if qpos[item, b] < 0:
                continue
            assert len(slot) == 1, "a run the request does not hold is read for it"
            start = slot[0] * run_keys + k * piece_keys
            seen[start:start + qpos[item, b] + 1] += 1
        assert (seen[:tail_key] == 1).all() and (seen[tail_key:] == 0).all()


def test_tail_lengths_follow_the_context():
    table, runs, request_runs = build()
    shared = SharedRuns(table, runs, request_runs, BS, margin=256)
    ctx = torch.tensor([3 * 512 + 5 + b for b in range(8)], dtype=torch.int32)
    tail_nk, tail_q = shared.tail_lens(ctx)
    assert torch.equal(tail_nk, ctx - (3 * 512 - 256)) and torch.equal(tail_q, (tail_nk - 1).long())


def test_refuses_a_table_that_does_not_start_with_the_runs():
    table, runs, request_runs = build()
    bad = table.clone()
    bad[3, 5] += 1
    with pytest.raises(ValueError, match="does not start with"):
        SharedRuns(bad, runs, request_runs, BS)
    twice = request_runs.clone()
    twice[0, 1] = twice[0, 0]
    with pytest.raises(ValueError, match="at most once"):
        SharedRuns(table, runs, twice, BS)
    with pytest.raises(ValueError, match="margin"):
        SharedRuns(table, runs, request_runs, BS, margin=20)
    with pytest.raises(ValueError, match="pieces"):
        SharedRuns(table, runs, request_runs, BS, pieces=3)
