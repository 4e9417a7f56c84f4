"""The MFMA prefill kernel against the oracle (position.py:404-560) at shapes
of hundreds to thousands of rows per request.

Cases cover the three K/V sources (dense rows, a block table, a slot map with
sidecar rows and several LDS windows of the map), GQA groups 1, 2, 4 and 8,
tables of 2, 8, 33 and 64 positions, ragged contexts with suffix query rows,
sparse unsorted query rows, long unsaturated stretches (small gates), a
strong table with outlier query channels (the fp32 bias table), scores that
rise tile after tile (the running-max rescale of O), small blocks (the
per-lane DMA path), and an invalid block.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd import CoPE, cope_attention
from cacheslide_amd.ccpe import ccpe_prefill_paged
from oracle import ccpe as orc
from tests._helpers import assert_close_bf16

pytestmark = pytest.mark.gpu

D = 128


def say(msg: str) -> None:
    print(f"[prefill] {msg}", flush=True)


def cope_with(device, e: np.ndarray) -> CoPE:
    cope = CoPE(D, e.shape[1], device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(torch.from_numpy(e))
    return cope


def randn(shape, seed, scale=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(shape, generator=g) * scale


def paged(keys, values, bs, hkv, seed, extra=5):
    """Cache [blocks, hkv, bs, 256] holding each request's K/V through a random
    block table (int32 [B, max_blocks], -1 padded)."""
    per = [(k.shape[0] + bs - 1) // bs for k in keys]
    total = sum(per) + extra
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(seed)).tolist()
    cache = torch.zeros((total, hkv, bs, 2 * D), dtype=torch.bfloat16)
    table = torch.full((len(keys), max(per)), -1, dtype=torch.int32)
    cur = 0
    for b, (k, v) in enumerate(zip(keys, values)):
        row = perm[cur:cur + per[b]]
        cur += per[b]
        table[b, :per[b]] = torch.tensor(row, dtype=torch.int32)
        n = k.shape[0]
        idx = torch.arange(n)
        blk = torch.tensor(row)[idx // bs]
        cache[blk, :, idx % bs, :D] = k
        cache[blk, :, idx % bs, D:] = v
    return cache, table


def run_paged_case(device, *, lens, nq, hq, hkv, npos, bs=16, seed=0, e_scale=0.02, q_fn=None, k_fn=None,
                   qpos_fn=None, sample=None):
    B = len(lens)
    rng = np.random.default_rng(seed)
    keys, values, qs, qposes = [], [], [], []
    for b, n in enumerate(lens):
        q = randn((nq, hq, D), seed + 10 * b + 1)
        k = randn((n, hkv, D), seed + 10 * b + 2)
        v = randn((n, hkv, D), seed + 10 * b + 3)
        if q_fn is not None:
            q = q_fn(q)
        if k_fn is not None:
            k = k_fn(k)
        qs.append(q.to(torch.bfloat16))
        keys.append(k.to(torch.bfloat16))
        values.append(v.to(torch.bfloat16))
        qposes.append(qpos_fn(n, rng) if qpos_fn else np.arange(n - nq, n))
    e = (randn((D, npos), seed + 7) * e_scale).numpy().astype(np.float32)
    cope = cope_with(device, e)
    cache, table = paged(keys, values, bs, hkv, seed + 5)
    q = torch.stack(qs).to(device)
    qpos = torch.from_numpy(np.stack(qposes)).to(device)
    out = ccpe_prefill_paged(q, cache.to(device), table.to(device),
                             torch.tensor(lens, dtype=torch.int32, device=device), cope, qpos)
    out = out.cpu()
    for b, n in enumerate(lens):
        rows = np.arange(nq) if sample is None else np.unique(rng.choice(nq, sample, replace=False))
        expected = orc.cope_attention(qs[b][rows].float().numpy(), keys[b].float().numpy(),
                                      values[b].float().numpy(), e, qposes[b][rows])
        assert_close_bf16(out[b, rows], expected)
    return out


@pytest.mark.parametrize("bs", [16, 2, 64])
def test_large_paged_ragged_suffix_rows(device, bs):
    say(f"paged ragged bs={bs}")
    run_paged_case(device, lens=[512, 700, 933, 517], nq=512, hq=32, hkv=8, npos=64, bs=bs, seed=100 + bs)


@pytest.mark.parametrize("hq,hkv,nq,batch", [(16, 16, 1024, 4), (16, 8, 1024, 4), (64, 8, 512, 2)])
def test_large_group_sizes(device, hq, hkv, nq, batch):
    say(f"group {hq // hkv}")
    run_paged_case(device, lens=[nq + 37 * b for b in range(batch)], nq=nq, hq=hq, hkv=hkv, npos=64,
                   seed=200 + hq + hkv, sample=96)


@pytest.mark.parametrize("npos", [2, 8, 33, 64])
def test_large_table_sizes(device, npos):
    say(f"P={npos}")
    run_paged_case(device, lens=[600, 512, 777, 530], nq=512, hq=32, hkv=8, npos=npos, e_scale=0.3,
                   seed=300 + npos, sample=128)


def test_large_strong_table_outlier_query_channels(device):
    """q with outlier channels (|q| about 30) and a table of std 0.5: large
    q.E biases, which the fp32 table keeps to fp32 accuracy."""
    say("strong table, outlier channels")

    def outliers(q):
        q[..., 5] = 30.0
        q[..., 77] = -28.0
        return q

    run_paged_case(device, lens=[512, 640, 800, 512], nq=512, hq=32, hkv=8, npos=64, e_scale=0.5,
                   q_fn=outliers, seed=400, sample=128)


def test_large_small_gates_stay_unsaturated(device):
    """Negative logits give gates near 0.05: positions grow slowly, so most
    tiles of every row take the CCPE path."""
    say("small gates")

    def pos_q(q):
        return q.abs() * 0.6

    def neg_k(k):
        return -k.abs() * 0.6

    run_paged_case(device, lens=[1024, 900, 700, 1024], nq=512, hq=32, hkv=8, npos=64, e_scale=0.2,
                   q_fn=pos_q, k_fn=neg_k, seed=500, sample=128)


def test_large_rising_scores_rescale(device):
    """Scores that grow from right to left by several units per key: the
    running max moves on tile after tile and O is rescaled each time."""
    say("rising scores")

    def aligned_q(q):
        return torch.full_like(q, 0.25)

    def rising_k(k):
        # raw scores 32 x ramp: about 130 more per 32-key tile, walking left
        n = k.shape[0]
        ramp = torch.linspace(100.0, 0.0, n)[:, None, None]
        return k * 0.05 + ramp

    run_paged_case(device, lens=[768, 512, 640, 900], nq=512, hq=32, hkv=8, npos=64, q_fn=aligned_q,
                   k_fn=rising_k, seed=600, sample=96)


def test_large_sparse_unsorted_rows(device):
    """Query rows at scattered positions in random order (the reuse call's
    active rows), some past the end of the context."""
    say("sparse rows")

    def scattered(n, rng):
        pos = rng.choice(n + 40, 512, replace=False)
        return pos.astype(np.int64)

    run_paged_case(device, lens=[4096, 3000, 2049, 1500], nq=512, hq=32, hkv=8, npos=64,
                   qpos_fn=scattered, seed=700, sample=64)


def test_large_paged_windows_small_blocks(device):
    """Block size 2: one block-table window in LDS covers 63 tiles (2016
    keys), so these contexts take two windows, with every key loaded on its
    own."""
    say("bs 2 windows")
    run_paged_case(device, lens=[2500, 2100, 3000, 2048], nq=512, hq=32, hkv=8, npos=64, bs=2, seed=650,
                   sample=64)


def test_large_dense_cope_attention(device):
    """cope_attention's dense fast path (one request, K/V rows)."""
    n, hq, hkv, npos = 2048, 32, 8, 64
    say("dense")
    q = randn((n, hq, D), 801).to(torch.bfloat16)
    k = randn((n, hkv, D), 802).to(torch.bfloat16)
    v = randn((n, hkv, D), 803).to(torch.bfloat16)
    e = (randn((D, npos), 804) * 0.05).numpy().astype(np.float32)
    cope = cope_with(device, e)
    out = cope_attention(q.to(device), k.to(device), v.to(device), cope, torch.arange(n, device=device)).cpu()
    rows = np.unique(np.concatenate([[0, 1, 31, 32, 63, 64, n - 1], np.random.default_rng(805).choice(n, 90)]))
    expected = orc.cope_attention(q[rows].float().numpy(), k.float().numpy(), v.float().numpy(), e, rows)
    assert_close_bf16(out[rows], expected)


def test_large_slot_map_sidecar_and_windows(device):
    """Per-token slot maps with native slots in scrambled order, runs split
    across blocks, sidecar rows, and contexts past one 1024-key window."""
    say("slot map")
    hq, hkv, nq, npos, bs = 32, 8, 1024, 64, 16
    lens = [2500, 1100]
    run_blocks = [(n + bs - 1) // bs for n in lens]
    spare = 64
    blocks = sum(run_blocks) + spare
    side_rows = 300
    rng = np.random.default_rng(900)
    order = rng.permutation(blocks)
    # block-contiguous runs come from the first blocks of the permutation, the
    # scattered slots from the spare blocks (64 x 16 = 1024 slots)
    scatter_pool = np.concatenate([np.arange(int(blk) * bs, int(blk) * bs + bs) for blk in order[sum(run_blocks):]])
    scatter_pool = rng.permutation(scatter_pool)
    free_side = rng.permutation(side_rows)
    native = blocks * bs
    cache = torch.zeros((blocks, hkv, bs, 2 * D), dtype=torch.bfloat16)
    side_k = torch.zeros((side_rows, hkv, D), dtype=torch.bfloat16)
    side_v = torch.zeros((side_rows, hkv, D), dtype=torch.bfloat16)
    slots = torch.full((len(lens), max(lens)), -1, dtype=torch.long)
    keys, values, qs, qposes = [], [], [], []
    cur_blk, cur_scatter, cur_side = 0, 0, 0
    for b, n in enumerate(lens):
        k = randn((n, hkv, D), 910 + b).to(torch.bfloat16)
        v = randn((n, hkv, D), 920 + b).to(torch.bfloat16)
        q = randn((nq, hq, D), 930 + b).to(torch.bfloat16)
        mine = order[cur_blk:cur_blk + run_blocks[b]]
        cur_blk += run_blocks[b]
        for t in range(n):
            if t % 11 == 5 and cur_side < side_rows:
                r = int(free_side[cur_side])
                cur_side += 1
                slots[b, t] = native + r
                side_k[r], side_v[r] = k[t], v[t]
                continue
            if t % 7 == 3:
                s = int(scatter_pool[cur_scatter])
                cur_scatter += 1
            else:
                s = int(mine[t // bs]) * bs + t % bs
            slots[b, t] = s
            cache[s // bs, :, s % bs, :D] = k[t]
            cache[s // bs, :, s % bs, D:] = v[t]
        keys.append(k)
        values.append(v)
        qs.append(q)
        qposes.append(np.arange(n - nq, n))
    e = (randn((D, npos), 940) * 0.05).numpy().astype(np.float32)
    cope = cope_with(device, e)
    out = ccpe_prefill_paged(torch.stack(qs).to(device), cache.to(device), None,
                             torch.tensor(lens, dtype=torch.int32, device=device), cope,
                             torch.from_numpy(np.stack(qposes)).to(device), slots=slots.to(device),
                             side_k=side_k.to(device), side_v=side_v.to(device)).cpu()
    for b, n in enumerate(lens):
        rows = np.unique(np.concatenate([[0, nq - 1], rng.choice(nq, 100)]))
        expected = orc.cope_attention(qs[b][rows].float().numpy(), keys[b].float().numpy(),
                                      values[b].float().numpy(), e, qposes[b][rows])
        assert_close_bf16(out[b, rows], expected)


def test_large_invalid_block_raises(device):
    say("invalid block")
    hq, hkv, nq, npos, bs = 32, 8, 512, 64, 16
    lens = [512] * 4
    cache = torch.zeros((4 * 32 + 2, hkv, bs, 2 * D), dtype=torch.bfloat16, device=device)
    table = torch.arange(4 * 32, dtype=torch.int32).view(4, 32).contiguous()
    table[2, 5] = 10_000
    cope = CoPE(D, npos, device=device)
    q = torch.zeros((4, nq, hq, D), dtype=torch.bfloat16, device=device)
    qpos = torch.arange(nq, device=device).repeat(4, 1).contiguous()
    with pytest.raises(ValueError, match="outside the cache"):
        ccpe_prefill_paged(q, cache, table.to(device), torch.tensor(lens, dtype=torch.int32, device=device),
                           cope, qpos)


def test_small_call_strong_table_outlier_query_channels(device):
    """A small call (2-wave workgroups) on the outlier-channel case: the fp32
    bias table keeps large q.E biases within the bf16 tolerance."""
    say("small call, outlier channels")
    hq, hkv, n, npos = 8, 2, 300, 64
    q = randn((n, hq, D), 1001)
    q[..., 5] = 30.0
    q[..., 77] = -28.0
    q = q.to(torch.bfloat16)
    k = randn((n, hkv, D), 1002).to(torch.bfloat16)
    v = randn((n, hkv, D), 1003).to(torch.bfloat16)
    e = (randn((D, npos), 1004) * 0.5).numpy().astype(np.float32)
    cope = cope_with(device, e)
    out = cope_attention(q.to(device), k.to(device), v.to(device), cope, torch.arange(n, device=device)).cpu()
    expected = orc.cope_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), e, np.arange(n))
    assert_close_bf16(out, expected)
