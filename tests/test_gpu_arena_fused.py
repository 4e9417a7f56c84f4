"""Fused CCPE decode and prefill reading a SLIDE arena through its slot map.

The reference decode step writes the new token (``NativePagedKV.decode``, with
hole reuse), gathers the whole logical K/V (``gather(arange(n))``) and runs
``cope_attention`` on it (src/cacheslide_vllm/runtime.py:489-508).  After a
selected-token promotion the canonical slot of a selected token is vacated,
decode reuses it for a new token, and the selected token's row is reachable
only through the slot map and the sidecar (paged.py:6-7, 474-524; slide.py:
401-459).  The fused kernels must read exactly what ``gather`` reads; the
oracle runs on the gathered K/V.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd import CoPE, NativePagedKV
from cacheslide_amd.ccpe import (
    ccpe_decode_arena,
    ccpe_decode_paged,
    ccpe_prefill_arena,
    ccpe_prefill_paged,
    decode_workspace,
    decode_workspace_bytes,
)
from oracle import ccpe as orc
from tests._helpers import acc_np, assert_close_bf16, seeded

pytestmark = pytest.mark.gpu


def cope_with(device, e):
    cope = CoPE(128, e.shape[1], device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(e)
    return cope


def relocated_arena(device, n=600, decoded=24, hkv=2, bs=16, seed=900, mover=None):
    """An arena after promote_selected (sidecar rows, vacated holes), a baseline
    write, update_selected with one mirror skipped under a pin, and decode hole
    reuse.  Returns the arena and its block table (int32, on ``device``)."""
    blocks_needed = (n + decoded + bs - 1) // bs
    nb = blocks_needed + 7
    table = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))[:blocks_needed].tolist()
    cache = seeded((nb, hkv, bs, 256), seed + 1, dtype=torch.bfloat16).to(device)
    arena = NativePagedKV(cache, table, n, 64, request_id="r", layer_index=3, mover=mover)
    key = seeded((n, hkv, 128), seed + 2, dtype=torch.bfloat16).to(device)
    value = seeded((n, hkv, 128), seed + 3, dtype=torch.bfloat16).to(device)
    rng = np.random.default_rng(seed)
    selected = sorted(rng.choice(n - 1, 40, replace=False).tolist())
    sel_k = seeded((len(selected), hkv, 128), seed + 4, dtype=torch.bfloat16).to(device)
    sel_v = seeded((len(selected), hkv, 128), seed + 5, dtype=torch.bfloat16).to(device)
    upd_k = seeded((len(selected), hkv, 128), seed + 6, dtype=torch.bfloat16).to(device)
    upd_v = seeded((len(selected), hkv, 128), seed + 7, dtype=torch.bfloat16).to(device)
    arena.write_prefill(key, value)
    # a reader pins the first selected token's canonical slot across the
    # promotion and the fused-row update, so that slot gets no mirror
    with arena.slot_map.pin_slots([arena.canonical_slot(selected[0])]):
        arena.promote_selected(selected, sel_k, sel_v).result()   # published once written
        arena.update_selected(selected, upd_k, upd_v)
    for t in range(n, n + decoded):
        dk = seeded((hkv, 128), seed + 100 + t, dtype=torch.bfloat16).to(device)
        dv = seeded((hkv, 128), seed + 200 + t, dtype=torch.bfloat16).to(device)
        arena.decode(t, dk, dv, arena.canonical_slot(t))
    stats = arena.stats()
    assert stats["physical_hole_reuse"] > 0 and stats["sidecar_allocated_slots"] > 0
    return arena, torch.tensor(table, dtype=torch.int32, device=device)


def test_fused_decode_on_relocated_arena_equals_gather(device):
    arena, table = relocated_arena(device)
    n = arena.logical_length()
    gk, gv = arena.gather(range(n))
    # the arena really is relocated: the block table's canonical reading differs
    with arena.device_slots(range(n)) as (slots, _, _):
        canonical = torch.tensor([arena.canonical_slot(t) for t in range(n)], device=device)
        assert bool((slots != canonical).any())
    e = seeded((128, 64), 950, scale=0.02)
    cope = cope_with(device, e.to(device))
    q = seeded((1, 8, 128), 951, dtype=torch.bfloat16)
    out = ccpe_decode_arena(q.to(device), arena, cope, split=128)
    expected = orc.cope_attention(acc_np(q), acc_np(gk), acc_np(gv), e.numpy(), np.array([n - 1]))
    assert_close_bf16(out, expected)
    # the block-table reading of the same cache is a different attention input
    lens = torch.tensor([n], dtype=torch.int32, device=device)
    stale = ccpe_decode_paged(q.to(device), arena.cache, table[None].contiguous(), lens, cope, split=128)
    assert not torch.equal(stale, out)


def test_fused_prefill_on_relocated_arena_equals_gather(device):
    arena, _ = relocated_arena(device, n=900, decoded=5, seed=960)
    n = arena.logical_length()
    gk, gv = arena.gather(range(n))
    e = seeded((128, 64), 970, scale=0.02)
    cope = cope_with(device, e.to(device))
    rows = np.sort(np.random.default_rng(971).choice(n, 150, replace=False))[::-1].copy()
    q = seeded((len(rows), 8, 128), 972, dtype=torch.bfloat16)
    out = ccpe_prefill_arena(q.to(device), arena, cope, torch.from_numpy(rows).to(device))
    expected = np.concatenate([
        orc.cope_attention(acc_np(q[i:i + 1]), acc_np(gk), acc_np(gv), e.numpy(), rows[i:i + 1])
        for i in range(len(rows))], axis=0)
    assert_close_bf16(out, expected)


@pytest.mark.parametrize("bs", [4, 16])
def test_slot_map_batches_with_sidecar_rows(device, bs):
    """Batched decode and prefill through random slot maps: runs of consecutive
    native slots (the scalar-base loads), scattered native slots and sidecar
    rows, over requests of different lengths."""
    lens = [1, 333, 1500]
    hq, hkv = 8, 2
    nb, side_rows = 160, 200
    gen = torch.Generator().manual_seed(700 + bs)
    cache = seeded((nb, hkv, bs, 256), 701, dtype=torch.bfloat16).to(device)
    side_k = seeded((side_rows, hkv, 128), 702, dtype=torch.bfloat16).to(device)
    side_v = seeded((side_rows, hkv, 128), 703, dtype=torch.bfloat16).to(device)
    native = nb * bs
    width = max(lens)
    slots = torch.full((len(lens), width + 5), -7, dtype=torch.long)
    rng = np.random.default_rng(704 + bs)
    for b, n in enumerate(lens):
        row = torch.randint(0, native + side_rows, (n,), generator=gen)
        # runs of consecutive native slots, as after whole-block placement
        # (with 4-slot blocks a run of 8 spans two blocks)
        for start in range(0, n - 8, 64):
            blk = int(rng.integers(0, nb - 2))
            run = torch.arange(blk * bs, blk * bs + 8)
            row[start:start + 8] = run
        slots[b, :n] = row
    # distinct slots per request are not required by the kernel; the oracle
    # gathers what each slot names
    full_k = torch.cat([cache[..., :128].permute(0, 2, 1, 3).reshape(native, hkv, 128), side_k])
    full_v = torch.cat([cache[..., 128:].permute(0, 2, 1, 3).reshape(native, hkv, 128), side_v])
    e = seeded((128, 64), 705, scale=0.02)
    cope = cope_with(device, e.to(device))
    lens_t = torch.tensor(lens, dtype=torch.int32, device=device)
    slots_d = slots.to(device)
    q = seeded((len(lens), hq, 128), 706, dtype=torch.bfloat16)
    out = ccpe_decode_paged(q.to(device), cache, None, lens_t, cope, slots=slots_d, side_k=side_k,
                            side_v=side_v, split=256)
    nq = 40
    qs = seeded((len(lens), nq, hq, 128), 707, dtype=torch.bfloat16)
    qpos = np.stack([np.sort(rng.choice(max(n, nq), nq, replace=n < nq)) % n for n in lens]).astype(np.int64)
    pout = ccpe_prefill_paged(qs.to(device), cache, None, lens_t, cope, torch.from_numpy(qpos).to(device),
                              slots=slots_d, side_k=side_k, side_v=side_v)
    for b, n in enumerate(lens):
        idx = slots[b, :n].to(device)
        kb, vb = full_k[idx].cpu(), full_v[idx].cpu()
        expected = orc.cope_attention(acc_np(q[b:b + 1]), acc_np(kb), acc_np(vb), e.numpy(), np.array([n - 1]))
        assert_close_bf16(out[b:b + 1], expected)
        pexp = np.concatenate([
            orc.cope_attention(acc_np(qs[b, r:r + 1]), acc_np(kb), acc_np(vb), e.numpy(), qpos[b, r:r + 1])
            for r in range(nq)], axis=0)
        assert_close_bf16(pout[b], pexp)


def test_slot_outside_cache_raises(device):
    cache = torch.zeros((4, 1, 16, 256), dtype=torch.bfloat16, device=device)
    cope = CoPE(128, 8, device=device)
    slots = torch.tensor([[0, 1, 64]], dtype=torch.long, device=device)  # 64 = first sidecar row, none given
    lens = torch.tensor([3], dtype=torch.int32, device=device)
    q = torch.zeros((1, 4, 128), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="outside the cache"):
        ccpe_decode_paged(q, cache, None, lens, cope, slots=slots, split=64)
    with pytest.raises(ValueError, match="outside the cache"):
        ccpe_prefill_paged(q[:, None], cache, None, lens, cope, torch.tensor([[2]], device=device), slots=slots)


def test_decode_context_and_workspace_checks(device):
    """position.py:149-150 (no key) and the workspace bound of the C ABI."""
    cache = torch.zeros((8, 1, 16, 256), dtype=torch.bfloat16, device=device)
    table = torch.arange(8, dtype=torch.int32, device=device)[None].repeat(2, 1).contiguous()
    cope = CoPE(128, 8, device=device)
    q = torch.zeros((2, 4, 128), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError, match="at least one key"):
        ccpe_decode_paged(q, cache, table, torch.tensor([5, 0], dtype=torch.int32, device=device), cope,
                          split=64)
    with pytest.raises(ValueError, match="exceeds max_context"):
        ccpe_decode_paged(q, cache, table, torch.tensor([5, 100], dtype=torch.int32, device=device), cope,
                          split=64, max_context=64)
    small = decode_workspace(2, 4, 64, 64, device)
    with pytest.raises(ValueError, match="workspace holds"):
        ccpe_decode_paged(q, cache, table, torch.tensor([5, 100], dtype=torch.int32, device=device), cope,
                          split=64, max_context=100, workspace=small)
    # an adequate caller workspace is accepted and reused
    ws = decode_workspace(2, 4, 100, 64, device)
    assert ws.numel() >= decode_workspace_bytes(2, 4, 100, 64)
    out = ccpe_decode_paged(q, cache, table, torch.tensor([5, 100], dtype=torch.int32, device=device), cope,
                            split=64, max_context=100, workspace=ws)
    assert out.shape == (2, 4, 128) and bool(torch.isfinite(out.float()).all())


def test_decode_context_past_slot_map_raises(device):
    """A context longer than max_context with a slot map exactly max_context
    wide: the decode clamps its reads to the map and flags the call."""
    cache = seeded((8, 2, 16, 256), 950, dtype=torch.bfloat16).to(device)
    cope = CoPE(128, 8, device=device)
    max_context = 64
    slots = torch.arange(max_context, dtype=torch.long, device=device)[None].repeat(2, 1).contiguous()
    lens = torch.tensor([40, 100], dtype=torch.int32, device=device)
    q = seeded((2, 8, 128), 951, dtype=torch.bfloat16).to(device)
    with pytest.raises(ValueError, match="exceeds max_context"):
        ccpe_decode_paged(q, cache, None, lens, cope, slots=slots, max_context=max_context, split=64)
    # the in-range request of the same call is unaffected by the clamp
    ok = ccpe_decode_paged(q[:1], cache, None, lens[:1], cope, slots=slots[:1], max_context=max_context,
                           split=64)
    assert bool(torch.isfinite(ok.float()).all())


def test_prefill_slot_map_narrower_than_context_raises(device):
    """Keys past the slot map's width read zeros and flag the call rather
    than reading past the map."""
    cache = seeded((8, 1, 16, 256), 952, dtype=torch.bfloat16).to(device)
    cope = CoPE(128, 8, device=device)
    slots = torch.arange(20, dtype=torch.long, device=device)[None].contiguous()
    lens = torch.tensor([48], dtype=torch.int32, device=device)
    q = seeded((1, 48, 4, 128), 953, dtype=torch.bfloat16).to(device)
    qpos = torch.arange(48, dtype=torch.long, device=device)[None].contiguous()
    with pytest.raises(ValueError, match="outside the cache"):
        ccpe_prefill_paged(q, cache, None, lens, cope, qpos, slots=slots)
    # the same map covering every key is accepted
    full = torch.arange(48, dtype=torch.long, device=device)[None].contiguous()
    out = ccpe_prefill_paged(q, cache, None, lens, cope, qpos, slots=full)
    assert bool(torch.isfinite(out.float()).all())
