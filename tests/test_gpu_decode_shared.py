"""The decode step (position.py:404-560 at one query row, as runtime.py:489-508
calls it) over a paged cache whose requests share runs of blocks, through
``ccpe_decode_shared``: each run is read once for the batch with every
position P-1, each request's tail with exact positions, and the two softmax
states merged; where a tail's gate mass stays below P-1 the exact decode runs
instead.  Checked against ``ccpe_decode_paged`` on the same block table and
against the oracle on the gathered keys."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd.ccpe import SharedRuns, ccpe_decode_paged, ccpe_decode_shared
from oracle import ccpe as orc
from tests._helpers import acc_np, assert_close_bf16, seeded
from tests.test_gpu_ccpe import cope_on

pytestmark = pytest.mark.gpu

HQ, HKV, BS, P = 8, 2, 16, 64
RUN_BLOCKS = 32                       # 512 keys per run
N_RUNS, SLOTS, B = 5, 3, 8


def layout(seed: int, low_gates: bool):
    """B requests, each holding SLOTS of the N_RUNS runs in its own order
    (two runs unused by some requests), then its own blocks: 40 + 7 b keys.
    Low gates: queries and keys anti-aligned (logits ~ -2.8, gates ~ 0.06),
    so a request's last 256 shared keys and its own keys do not reach P-1."""
    rng = np.random.default_rng(seed)
    own = [40 + 7 * b for b in range(B)]
    own_blocks = [(n + BS - 1) // BS for n in own]
    shared_blocks = N_RUNS * RUN_BLOCKS
    nb = shared_blocks + sum(own_blocks) + 1
    runs = torch.arange(shared_blocks, dtype=torch.int32).view(N_RUNS, RUN_BLOCKS)
    request_runs = torch.tensor(np.stack([rng.permutation(N_RUNS)[:SLOTS] for _ in range(B)]))
    max_blocks = SLOTS * RUN_BLOCKS + max(own_blocks)
    table = torch.zeros((B, max_blocks), dtype=torch.int32)
    nxt = shared_blocks
    for b in range(B):
        table[b, :SLOTS * RUN_BLOCKS] = runs[request_runs[b]].reshape(-1)
        for i in range(own_blocks[b]):
            table[b, SLOTS * RUN_BLOCKS + i] = nxt
            nxt += 1
    lens = [SLOTS * RUN_BLOCKS * BS + own[b] for b in range(B)]
    q = seeded((B, HQ, 128), seed + 1, dtype=torch.bfloat16)
    if low_gates:
        q = (seeded((B, HQ, 128), seed + 1, scale=0.05) + 0.5).to(torch.bfloat16)
        cache = (seeded((nb, HKV, BS, 256), seed + 2, scale=0.05) - 0.5).to(torch.bfloat16)
    else:
        cache = seeded((nb, HKV, BS, 256), seed + 2, dtype=torch.bfloat16)
    return table, runs, request_runs, lens, q, cache


def gathered(cache, table, n):
    """Keys and values of a request in key order, from its block table row."""
    blocks = table[: (n + BS - 1) // BS].long()
    rec = cache[blocks].permute(0, 2, 1, 3).reshape(-1, HKV, 256)[:n]
    return rec[..., :128], rec[..., 128:]


@pytest.mark.parametrize("margin", [256, 1024])
@pytest.mark.parametrize("low_gates", [False, True])
def test_shared_runs_decode_matches_paged_and_oracle(device, low_gates, margin):
    """Saturating positions: the merged states equal the exact decode within
    the bf16 tolerance (and are not its bits: the shared path ran).  Low
    gates: every tail stays below P-1, the exact decode runs, and the result
    is that decode's, bit for bit.  Margins of 256 and 1024 keys (tails of up
    to 345 and 1113 keys)."""
    table, runs, request_runs, lens, q, cache = layout(91 + int(low_gates), low_gates)
    e = seeded((128, P), 95, scale=0.1)
    cope = cope_on(device, 128, P, table=e)
    dtable, dcache, dq = table.to(device), cache.to(device), q.to(device)
    ctx = torch.tensor(lens, dtype=torch.int32, device=device)
    shared = SharedRuns(dtable, runs, request_runs, BS, margin=margin, pieces=2)
    out = ccpe_decode_shared(dq, dcache, dtable, ctx, cope, shared, max_context=max(lens), split=256)
    ref = ccpe_decode_paged(dq, dcache, dtable, ctx, cope, max_context=max(lens), split=256)
    if low_gates:
        assert torch.equal(out, ref)
    else:
        assert_close_bf16(out, ref.float().cpu().numpy())
        assert not torch.equal(out, ref)
    for b in (0, B - 1):
        k, v = gathered(cache, table[b], lens[b])
        expected = orc.cope_attention(acc_np(q[b:b + 1]), acc_np(k), acc_np(v), e.numpy(), np.array([lens[b] - 1]))
        assert_close_bf16(out[b:b + 1], expected)
