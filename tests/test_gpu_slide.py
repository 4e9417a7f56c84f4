"""SLIDE slot kernels on the MI355X: bit-exact against the oracle and the
reference's NativePagedKV fixtures (tests/test_paged.py of the reference)."""

from __future__ import annotations

from concurrent.futures import Future

import numpy as np
import pytest
import torch

from cacheslide_amd import CacheCapacityError, CoPE, NativePagedKV, cope_attention
from cacheslide_amd import relocate
from oracle import slide as orc

pytestmark = pytest.mark.gpu


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.view(torch.int64).numpy().view(np.uint64)


def random_bf16(shape, seed):
    gen = torch.Generator().manual_seed(seed)
    raw = torch.randint(-(2**15), 2**15, shape, generator=gen, dtype=torch.int16)
    return raw.view(torch.bfloat16)


# ------------------------------------------------------------ kernels vs oracle
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16, torch.float64])
def test_slot_scatter_gather_bit_exact(device, dtype):
    blocks, heads, bs, d = 12, 3, 4, 40
    gen = torch.Generator().manual_seed(1)
    backing = torch.randn((blocks, heads, bs, 4 * d), generator=gen).to(dtype)
    cache_cpu = backing[..., ::2].clone() if dtype != torch.bfloat16 else random_bf16((blocks, heads, bs, 2 * d), 2)
    n = 20
    slots = np.random.default_rng(0).choice(blocks * bs + 6, n, replace=False)
    key = torch.randn((n, heads, d), generator=gen).to(dtype)
    value = torch.randn((n, heads, d), generator=gen).to(dtype)
    side = torch.zeros((6, heads, d), dtype=dtype)
    # oracle on raw bits
    cb, sk, sv = bits(cache_cpu).copy(), bits(side).copy(), bits(side).copy()
    orc.slot_scatter(cb, sk, sv, slots.tolist(), bits(key), bits(value))
    # device: the cache is a strided view of a wider backing buffer
    wide = torch.zeros((blocks, heads, bs, 4 * d), dtype=dtype, device=device)
    cache = wide[..., ::2]
    cache.copy_(cache_cpu.to(device))
    side_k, side_v = side.to(device), side.to(device)
    from cacheslide_amd.paged import HipSlotMover

    mover = HipSlotMover()
    mover.scatter(cache, side_k, side_v, slots.tolist(), key.to(device), value.to(device))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(cache), cb)
    np.testing.assert_array_equal(bits(side_k), sk)
    np.testing.assert_array_equal(bits(side_v), sv)
    assert (bits(wide[..., 1::2]) == 0).all()  # the backing's other columns are untouched
    gk = torch.empty_like(key, device=device)
    gv = torch.empty_like(value, device=device)
    mover.gather(cache, side_k, side_v, slots.tolist(), gk, gv)
    np.testing.assert_array_equal(bits(gk), bits(key))
    np.testing.assert_array_equal(bits(gv), bits(value))


def test_relocation_page_and_slot_copy_bit_exact(device):
    layers, blocks, heads, bs, d = 3, 40, 2, 16, 128
    cache_cpu = random_bf16((layers, blocks, heads, bs, 2 * d), 5)
    ref = bits(cache_cpu).copy()
    cache = cache_cpu.to(device)
    src_b, dst_b = [1, 7, 30], [2, 8, 39]
    orc.page_copy(ref, src_b, dst_b)
    relocate.copy_pages(cache, torch.tensor(src_b, device=device), torch.tensor(dst_b, device=device))
    src_s = [5 * 16 + 3, 5 * 16 + 4, 20 * 16 + 15]
    dst_s = [33 * 16 + 0, 33 * 16 + 1, 34 * 16 + 9]
    orc.slot_copy(ref, src_s, dst_s)
    relocate.copy_slots(cache, torch.tensor(src_s, device=device), torch.tensor(dst_s, device=device))
    np.testing.assert_array_equal(bits(cache), ref)


def test_mapping_scatter_gather(device):
    mapping = torch.full((50,), -1, dtype=torch.long, device=device)
    tokens = torch.tensor([3, 17, 49, 0], device=device)
    slots = torch.tensor([100, 5, 7, 42], device=device)
    relocate.scatter_mapping(mapping, tokens, slots)
    got = relocate.gather_mapping(mapping, torch.tensor([0, 3, 17, 49, 60], device=device))
    assert got.tolist() == [42, 100, 5, 7, -1]


def test_free_list_follows_fresh_slot_order(device):
    # LayerSlotMap._fresh_slot: returned slots lowest-first, then the never-used tail
    fl = relocate.SlotFreeList(100, device, free_from=10)
    fl.release(torch.tensor([7, 2], device=device))
    got = fl.acquire(5).tolist()
    assert got == orc.fresh_slot_sequence({7, 2}, 10, 5)
    with pytest.raises(CacheCapacityError):
        fl.acquire(1000)
    mask = fl.free_mask()
    assert mask[:10].sum() == 0 and mask[13:].all() and not mask[10:13].any()


def test_free_list_large_random(device):
    nbits = 100_000
    rng = np.random.default_rng(4)
    free = rng.random(nbits) < 0.3
    fl = relocate.SlotFreeList(nbits, device, free_from=nbits)
    fl.release(torch.from_numpy(np.flatnonzero(free)).to(device))
    want = orc.acquire_lowest(free.copy(), 20_000)
    got = fl.acquire(20_000)
    np.testing.assert_array_equal(got.cpu().numpy(), want)


# ------------------------------------------------------------ reference fixtures
def fixture_arena(device, max_selected=2):
    # tests/test_paged.py:13-23 (non-contiguous cache: every second element)
    backing = torch.full((8, 2, 2, 12), -999.0, device=device)
    cache = backing[..., ::2]
    assert not cache.is_contiguous()
    arena = NativePagedKV(cache, [4, 1, 6, 3], 5, max_selected, request_id="request-a", layer_index=2)
    key = torch.arange(30, dtype=cache.dtype, device=device).reshape(5, 2, 3) / 30
    value = key + 10
    arena.write_prefill(key, value)
    return arena, key, value, backing


def native_row(arena, token):
    block, offset = divmod(arena.canonical_slot(token), arena.block_size)
    return (arena.cache[block, :, offset, : arena.head_dim], arena.cache[block, :, offset, arena.head_dim :])


def test_native_noncontiguous_prefill_staged_wca_decode_and_gqa(device):
    # tests/test_paged.py:245-310
    arena, key, value, backing = fixture_arena(device)
    assert arena.snapshot() == {0: 8, 1: 9, 2: 2, 3: 3, 4: 12}
    loading = Future()
    selected = torch.tensor([3, 1])
    raw_key, raw_value = key[selected] + 1, value[selected] + 2
    mapping = arena.promote_selected(selected, raw_key, raw_value, load_future=loading).result()
    assert mapping[3] == 16 and mapping[1] == 17
    assert arena.stats()["vacated_slots"] == 2
    for row in selected:
        original_k, original_v = native_row(arena, int(row))
        torch.testing.assert_close(original_k, key[row])
        torch.testing.assert_close(original_v, value[row])
    with pytest.raises(RuntimeError, match="load must complete"):
        arena.write_prefill(key, value)
    with pytest.raises(RuntimeError, match="load must complete"):
        arena.update_selected(selected, raw_key, raw_value)
    loading.set_result(None)
    arena.write_prefill(key, value)
    updates = [1, 3, 4]
    final_key, final_value = key[updates] + 0.5, value[updates] + 0.75
    arena.update_selected(updates, final_key, final_value)
    key[updates], value[updates] = final_key, final_value
    for row in updates:
        original_k, original_v = native_row(arena, row)
        torch.testing.assert_close(original_k, key[row])
        torch.testing.assert_close(original_v, value[row])
    order = [4, 1, 0, 3, 2]
    gathered_k, gathered_v = arena.gather(order)
    torch.testing.assert_close(gathered_k, key[order], rtol=0, atol=0)
    torch.testing.assert_close(gathered_v, value[order], rtol=0, atol=0)
    assert arena.decode(5, key[0] + 2, value[0] + 2, 13) == 3
    assert arena.decode(6, key[0] + 3, value[0] + 3, 6) == 9
    assert arena.decode(7, key[0] + 4, value[0] + 4, 7) == 7
    expected_k = torch.cat((key, key[:1] + 2, key[:1] + 3, key[:1] + 4))
    expected_v = torch.cat((value, value[:1] + 2, value[:1] + 3, value[:1] + 4))
    gathered_k, gathered_v = arena.gather(range(8))
    torch.testing.assert_close(gathered_k, expected_k, rtol=0, atol=0)
    torch.testing.assert_close(gathered_v, expected_v, rtol=0, atol=0)
    for token in (5, 6, 7):
        canonical_k, canonical_v = native_row(arena, token)
        torch.testing.assert_close(canonical_k, expected_k[token])
        torch.testing.assert_close(canonical_v, expected_v[token])
    query = torch.linspace(-1, 1, 12, device=device).reshape(1, 4, 3)
    cope = CoPE(3, 16, device=device)
    actual = cope_attention(query, gathered_k, gathered_v, cope, torch.tensor([7], device=device))
    expected = cope_attention(query, expected_k, expected_v, cope, torch.tensor([7], device=device))
    torch.testing.assert_close(actual, expected)
    assert torch.all(arena.cache[0] == -999)
    assert torch.all(backing[..., 1::2] == -999)
    stats = arena.stats()
    assert stats["physical_hole_reuse"] == 2 and stats["decode_native_bind"] == 1
    assert stats["native_pool_capacity_slots"] == 16 and stats["sidecar_capacity_slots"] == 2
    with pytest.raises(RuntimeError, match="after decode"):
        arena.write_prefill(key, value)
    with pytest.raises(RuntimeError, match="precede decode"):
        arena.update_selected(updates, final_key, final_value)


@pytest.mark.parametrize("max_selected", [0, 2])
def test_load_first_selected_writes_stay_native(device, max_selected):
    # tests/test_paged.py:34-54
    arena, key, value, _ = fixture_arena(device, max_selected=max_selected)
    original = arena.snapshot()
    assert arena.stats()["sidecar_allocated_slots"] == 0
    assert arena.write_selected_ready([1, 3], key[[1, 3]] + 1, value[[1, 3]] + 2) == original
    key[[1, 3]] += 1
    value[[1, 3]] += 2
    gathered_key, gathered_value = arena.gather(range(5))
    torch.testing.assert_close(gathered_key, key)
    torch.testing.assert_close(gathered_value, value)
    assert arena.stats()["selected_ready_inplace_writes"] == 2
    assert arena.decode(5, key[0], value[0]) == 13


def test_selected_update_skips_pinned_mirror(device):
    # tests/test_paged.py:334-361 (pin_slots variant)
    arena, key, value, _ = fixture_arena(device)
    with arena.slot_map.pin_slots([9]):
        arena.promote_selected([1, 3], key[[1, 3]] + 1, value[[1, 3]] + 1).result()
        arena.update_selected([1, 3], key[[1, 3]] + 2, value[[1, 3]] + 2)
        torch.testing.assert_close(native_row(arena, 1)[0], key[1])
        torch.testing.assert_close(native_row(arena, 3)[0], key[3] + 2)
        torch.testing.assert_close(arena.gather([1, 3])[0], key[[1, 3]] + 2)
        assert arena.stats()["canonical_mirror_writes"] == 1
    arena.update_selected([1], key[1:2] + 3, value[1:2] + 3)
    torch.testing.assert_close(native_row(arena, 1)[0], key[1] + 3)
    assert arena.decode(5, key[0], value[0]) == 3
    assert arena.decode(6, key[0], value[0]) == 9


def test_bf16_arena_round_trip_bit_exact(device):
    cache = torch.zeros((64, 8, 16, 256), dtype=torch.bfloat16, device=device)
    table = torch.randperm(64, generator=torch.Generator().manual_seed(3))[:40].tolist()
    n = 40 * 16 - 5
    arena = NativePagedKV(cache, table, n, 32)
    key = random_bf16((n, 8, 128), 10).to(device)
    value = random_bf16((n, 8, 128), 11).to(device)
    arena.write_prefill(key, value)
    sel = list(range(3, n, 37))[:30]
    newk = random_bf16((len(sel), 8, 128), 12).to(device)
    newv = random_bf16((len(sel), 8, 128), 13).to(device)
    arena.promote_selected(sel, newk, newv).result()
    gk, gv = arena.gather(range(n))
    expect_k, expect_v = key.clone(), value.clone()
    expect_k[sel], expect_v[sel] = newk, newv
    np.testing.assert_array_equal(bits(gk), bits(expect_k))
    np.testing.assert_array_equal(bits(gv), bits(expect_v))


@pytest.mark.parametrize("layers, blocks, heads, bs, d, dtype", [
    (2, 64, 8, 16, 128, torch.bfloat16),
    (1, 100, 1, 8, 64, torch.float32),
    (4, 50, 4, 32, 32, torch.float16),
])
def test_relocation_random_geometry_bit_exact(device, layers, blocks, heads, bs, d, dtype):
    gen = torch.Generator().manual_seed(blocks + heads)
    cache_cpu = torch.randn((layers, blocks, heads, bs, 2 * d), generator=gen, dtype=torch.float64).to(dtype)
    ref = bits(cache_cpu).copy()
    cache = cache_cpu.to(device)
    perm = torch.randperm(blocks, generator=gen).tolist()
    q = blocks // 4
    src_b, dst_b = perm[:q], perm[q:2 * q]                                   # disjoint block sets
    orc.page_copy(ref, src_b, dst_b)
    relocate.copy_pages(cache, torch.tensor(src_b, device=device), torch.tensor(dst_b, device=device))
    # slots inside the untouched blocks, disjoint sources and destinations
    rest = perm[2 * q:]
    slots = [blk * bs + off for blk in rest for off in range(bs)]
    order = torch.randperm(len(slots), generator=gen).tolist()
    k = min(40, len(slots) // 2)
    src_s = [slots[i] for i in order[:k]]
    dst_s = [slots[i] for i in order[k:2 * k]]
    orc.slot_copy(ref, src_s, dst_s)
    relocate.copy_slots(cache, torch.tensor(src_s, device=device), torch.tensor(dst_s, device=device))
    np.testing.assert_array_equal(bits(cache), ref)


def test_empty_moves_leave_the_cache_alone(device):
    cache = random_bf16((2, 6, 2, 4, 16), 3).to(device)
    before = bits(cache).copy()
    empty = torch.zeros(0, dtype=torch.long, device=device)
    relocate.copy_pages(cache, empty, empty)
    relocate.copy_slots(cache, empty, empty)
    mapping = torch.arange(10, dtype=torch.long, device=device)
    relocate.scatter_mapping(mapping, empty, empty)
    assert relocate.gather_mapping(mapping, empty).shape == (0,)
    from cacheslide_amd.paged import HipSlotMover

    layer = cache[0]
    kv = torch.zeros((0, 2, 8), dtype=torch.bfloat16, device=device)
    HipSlotMover().scatter(layer, None, None, [], kv, kv)
    HipSlotMover().gather(layer, None, None, [], kv, kv)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(cache), before)
    assert torch.equal(mapping.cpu(), torch.arange(10))


def test_relocation_rejects_overlaps_and_short_buffers(device):
    """Overlapping sources/destinations would race inside one launch; a short
    slot list or output buffer would be read or written past its end."""
    cache = random_bf16((1, 8, 2, 4, 16), 5).to(device)
    before = bits(cache).copy()
    t = lambda xs: torch.tensor(xs, dtype=torch.long, device=device)  # noqa: E731
    with pytest.raises(ValueError, match="disjoint"):
        relocate.copy_pages(cache, t([1, 2]), t([2, 3]))
    with pytest.raises(ValueError, match="distinct"):
        relocate.copy_pages(cache, t([1, 2]), t([4, 4]))
    with pytest.raises(ValueError, match="disjoint"):
        relocate.copy_slots(cache, t([0, 5]), t([9, 0]))
    np.testing.assert_array_equal(bits(cache), before)   # nothing moved
    mapping = torch.full((10,), -1, dtype=torch.long, device=device)
    with pytest.raises(ValueError, match="same length"):
        relocate.scatter_mapping(mapping, t([1, 2, 3]), t([7, 8]))
    fl = relocate.SlotFreeList(64, device)
    with pytest.raises(ValueError, match="acquire needs 5"):
        fl.acquire(5, out=torch.empty(4, dtype=torch.long, device=device))
    assert fl.acquire(4, out=torch.empty(4, dtype=torch.long, device=device)).tolist() == [0, 1, 2, 3]
