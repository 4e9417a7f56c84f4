"""NativePagedKV's host rules on the CPU (src/cacheslide_vllm/paged.py:57-581).

The records move through ``HostMover`` (tests/_helpers.py), a host stand-in
for the slot kernels; the same scenarios' bytes are checked on the device by
tests/test_gpu_slide.py.  The arena below: 4 blocks x 2 KV heads x block 4 x
head dim 3, block table [2, 0, 3, -1], a 10-token prompt, so
  tokens 0-3 -> slots 8-11, tokens 4-7 -> slots 0-3, tokens 8-9 -> slots 12-13,
the next decode tokens 10 and 11 own slots 14 and 15, and sidecar slots start
at 16 (= 4 blocks x 4).  Expected values follow the reference's rules; the
scenarios are this package's own.
"""

from __future__ import annotations

from concurrent.futures import Future

import pytest
import torch

from cacheslide_amd import paged
from cacheslide_amd.paged import NativePagedKV
from cacheslide_amd.errors import CacheCapacityError, StaleCompletionError
from tests._helpers import HostMover

CANONICAL = {0: 8, 1: 9, 2: 10, 3: 11, 4: 0, 5: 1, 6: 2, 7: 3, 8: 12, 9: 13}


def kv(n: int, seed: int):
    gen = torch.Generator("cpu").manual_seed(seed)
    return torch.randn((n, 2, 3), generator=gen), torch.randn((n, 2, 3), generator=gen)


def arena(max_selected: int = 2, **kwargs) -> NativePagedKV:
    cache = torch.full((4, 2, 4, 6), -1.0)
    return NativePagedKV(cache, [2, 0, 3, -1], 10, max_selected, mover=HostMover(), **kwargs)


def record(a: NativePagedKV, slot: int):
    block, offset = divmod(slot, a.block_size)
    return a.cache[block, :, offset, :3], a.cache[block, :, offset, 3:]


def test_layout_and_canonical_slots():
    a = arena()
    assert a.snapshot() == CANONICAL
    assert (a.block_size, a.kv_heads, a.head_dim, a.native_total_slots) == (4, 2, 3, 16)
    assert a.canonical_slot(10) == 14 and a.canonical_slot(11) == 15
    with pytest.raises(ValueError, match="no caller-owned native block"):
        a.canonical_slot(12)
    stats = a.stats()
    assert stats["sidecar_capacity_slots"] == 2 and stats["sidecar_allocated_slots"] == 0
    assert stats["native_pool_capacity_slots"] == 16 and stats["native_pool_capacity_blocks"] == 4
    assert stats["native_pool_capacity_delta"] == 0 and stats["native_pool_blocks_released"] == 0


def test_load_first_branch_overwrites_native_slots_only():
    a = arena()
    k, v = kv(10, 1)
    with pytest.raises(RuntimeError, match="baseline device writes must complete"):
        a.write_selected_ready([2, 5], k[[2, 5]], v[[2, 5]])
    a.write([0, 1, 2, 3, 4], k[:5], v[:5])
    with pytest.raises(RuntimeError, match="baseline device writes must complete"):
        a.write_selected_ready([2, 5], k[[2, 5]], v[[2, 5]])
    a.write([5, 6, 7, 8, 9], k[5:], v[5:])
    assert a.write_selected_ready([2, 5], k[[2, 5]] + 1, v[[2, 5]] + 1) == CANONICAL
    assert a.stats()["sidecar_allocated_slots"] == 0
    assert a.stats()["selected_ready_inplace_writes"] == 2
    with pytest.raises(ValueError, match="already selected"):
        a.write_selected_ready([2], k[[2]], v[[2]])
    gk, gv = a.gather([5, 2, 0])
    torch.testing.assert_close(gk, torch.stack([k[5] + 1, k[2] + 1, k[0]]), rtol=0, atol=0)
    torch.testing.assert_close(gv, torch.stack([v[5] + 1, v[2] + 1, v[0]]), rtol=0, atol=0)
    assert a.decode(10, k[0], v[0]) == 14  # no holes: the owned canonical slot
    with pytest.raises(RuntimeError, match="precede decode"):
        a.write_selected_ready([3], k[[3]], v[[3]])


def test_pending_load_relocates_and_blocks_hole_reuse_until_it_lands():
    a = arena()
    k, v = kv(12, 2)
    a.write_prefill(k[:10], v[:10])
    load = Future()
    mapping = a.promote_selected([1, 6], k[[1, 6]] + 5, v[[1, 6]] + 5, load_future=load).result()
    assert mapping[1] == 16 and mapping[6] == 17  # sidecar, in the given order
    assert a.stats()["sidecar_allocated_slots"] == 2
    torch.testing.assert_close(record(a, 9)[0], k[1])  # the sources keep their bytes
    with pytest.raises(RuntimeError, match="load must complete"):
        a.write_prefill(k[:10], v[:10])
    assert a.decode(10, k[10], v[10]) == 14  # holes 2 and 9 still receive the load
    load.set_result(None)
    assert a.decode(11, k[11], v[11]) == 2  # lowest hole, mirrored into slot 15
    torch.testing.assert_close(record(a, 15)[0], k[11], rtol=0, atol=0)
    torch.testing.assert_close(record(a, 2)[1], v[11], rtol=0, atol=0)
    stats = a.stats()
    assert (stats["physical_hole_reuse"], stats["decode_native_bind"], stats["canonical_mirror_writes"]) == (1, 1, 1)
    expect_k = k.clone()
    expect_k[[1, 6]] += 5
    gk, _ = a.gather(range(12))
    torch.testing.assert_close(gk, expect_k, rtol=0, atol=0)
    with pytest.raises(RuntimeError, match="after decode"):
        a.write_prefill(k[:10], v[:10])
    with pytest.raises(RuntimeError, match="precede decode"):
        a.promote_selected([3], k[[3]], v[[3]])


def test_failed_load_blocks_baseline_and_decode():
    a = arena()
    k, v = kv(11, 3)
    load = Future()
    a.promote_selected([4], k[[4]], v[[4]], load_future=load)
    load.set_exception(OSError("load lost"))
    with pytest.raises(OSError, match="load lost"):
        a.write_prefill(k[:10], v[:10])
    with pytest.raises(OSError, match="load lost"):
        a.decode(10, k[10], v[10])


def test_update_selected_mirrors_except_where_a_reader_pins_the_canonical_slot():
    a = arena()
    k, v = kv(10, 4)
    a.write_prefill(k, v)
    with a.slot_map.pin_slots([9]):  # a reader holds token 1's original record
        a.promote_selected([1, 6], k[[1, 6]] + 1, v[[1, 6]] + 1).result()
        a.update_selected([1, 6], k[[1, 6]] + 2, v[[1, 6]] + 2)
        torch.testing.assert_close(record(a, 9)[0], k[1], rtol=0, atol=0)  # pinned: no mirror
        torch.testing.assert_close(record(a, 2)[0], k[6] + 2, rtol=0, atol=0)  # mirrored
        assert a.stats()["canonical_mirror_writes"] == 1
        gk, _ = a.gather([6, 1])
        torch.testing.assert_close(gk, torch.stack([k[6] + 2, k[1] + 2]), rtol=0, atol=0)
    a.update_selected([1], k[[1]] + 3, v[[1]] + 3)
    torch.testing.assert_close(record(a, 9)[0], k[1] + 3, rtol=0, atol=0)
    assert a.stats()["canonical_mirror_writes"] == 2


def test_guarded_destinations_are_rejected_before_any_copy():
    a = arena()
    k, v = kv(10, 5)
    a.write_prefill(k, v)
    with a.slot_map.pin_slots([9]):
        with pytest.raises(RuntimeError, match="pinned or in-flight"):
            a.write_selected_ready([1], k[[1]] + 1, v[[1]] + 1)
    torch.testing.assert_close(record(a, 9)[0], k[1], rtol=0, atol=0)
    a.promote_selected([1], k[[1]] + 1, v[[1]] + 1).result()
    side_before = a._side[0].clone()
    with a.slot_map.pin_slots([16]):
        with pytest.raises(RuntimeError, match="pinned or in-flight"):
            a.update_selected([1], k[[1]] + 9, v[[1]] + 9)
    torch.testing.assert_close(a._side[0], side_before, rtol=0, atol=0)
    with a.slot_map.pin_slots([8]):
        with pytest.raises(RuntimeError, match="pinned or in-flight"):
            a.write([0], k[[0]], v[[0]])


def test_promotion_publishes_only_when_the_device_write_completes(monkeypatch):
    a = arena()
    k, v = kv(10, 6)
    a.write_prefill(k, v)
    landed = Future()
    monkeypatch.setattr(paged, "_completion_future", lambda device: landed)
    promotion = a.promote_selected([3], k[[3]] + 1, v[[3]] + 1)
    assert not promotion.done()
    assert a.snapshot() == CANONICAL
    with pytest.raises(RuntimeError, match="selected writes must complete"):
        a.update_selected([3], k[[3]], v[[3]])
    with pytest.raises(ValueError, match="use update_selected"):
        a.promote_selected([3], k[[3]], v[[3]])
    landed.set_result(None)
    assert promotion.result()[3] == 16
    assert a.snapshot()[3] == 16


def test_a_failed_promotion_write_keeps_the_mapping_and_frees_its_slot(monkeypatch):
    a = arena()
    k, v = kv(10, 7)
    a.write_prefill(k, v)
    failed = Future()
    monkeypatch.setattr(paged, "_completion_future", lambda device: failed)
    promotion = a.promote_selected([3], k[[3]] + 1, v[[3]] + 1)
    failed.set_exception(OSError("device write failed"))
    assert isinstance(promotion.exception(), OSError)
    assert a.snapshot() == CANONICAL
    assert a.slot_map.promote_selected({5: b"x"}, lambda runs: None).result()[5] == 16


def test_retirement_rejects_a_late_promotion(monkeypatch):
    a = arena()
    k, v = kv(10, 8)
    landed = Future()
    monkeypatch.setattr(paged, "_completion_future", lambda device: landed)
    promotion = a.promote_selected([0], k[[0]], v[[0]])
    a.invalidate()
    landed.set_result(None)
    with pytest.raises(StaleCompletionError):
        promotion.result()
    with pytest.raises(StaleCompletionError):
        a.snapshot()
    with pytest.raises(StaleCompletionError):
        a.canonical_slot(0)


class FailingMover(HostMover):
    """Copies the first record, then fails: a partial, nontransactional write."""

    def scatter(self, cache, side_k, side_v, slots, key, value, rows=None):
        super().scatter(cache, side_k, side_v, slots[:1], key, value, None if rows is None else rows[:1])
        raise OSError("copy interrupted")


@pytest.mark.parametrize("operation", ["baseline", "fused", "decode"])
def test_a_failed_copy_retires_the_arena(operation):
    a = arena()
    k, v = kv(11, 9)
    if operation != "baseline":
        a.write_prefill(k[:10], v[:10])
    if operation == "fused":
        a.promote_selected([1], k[[1]], v[[1]]).result()
    a._mover = FailingMover()
    with pytest.raises(OSError, match="interrupted"):
        if operation == "baseline":
            a.write_prefill(k[:10], v[:10])
        elif operation == "fused":
            a.update_selected([1], k[[1]], v[[1]])
        else:
            a.decode(10, k[10], v[10])
    with pytest.raises(StaleCompletionError):
        a.snapshot()
    assert a.stats()["inflight_slots"] == 0
    assert a.stats()["mapped_tokens"] == 10  # a failed decode never publishes its token


def test_the_sidecar_bound_is_never_exceeded():
    a = arena(max_selected=1)
    k, v = kv(10, 10)
    with pytest.raises(CacheCapacityError):
        a.promote_selected([1, 6], k[[1, 6]], v[[1, 6]])
    assert a.snapshot() == CANONICAL
    assert a.stats()["inflight_slots"] == 0
    assert a.promote_selected([6], k[[6]], v[[6]]).result()[6] == 16
    z = arena(max_selected=0)
    with pytest.raises(CacheCapacityError):
        z.promote_selected([1], k[[1]], v[[1]])
    z.write_prefill(k, v)
    assert z.decode(10, k[0], v[0]) == 14


def test_decode_follows_the_callers_block_table():
    a = arena()
    k, v = kv(13, 11)
    a.write_prefill(k[:10], v[:10])
    with pytest.raises(ValueError, match="next logical token"):
        a.decode(11, k[11], v[11])
    with pytest.raises(ValueError, match="not owned"):
        a.decode(10, k[10], v[10], 15)
    assert a.decode(10, k[10], v[10], 14) == 14
    assert a.decode(11, k[11], v[11]) == 15
    with pytest.raises(ValueError, match="no caller-owned native block"):
        a.decode(12, k[12], v[12])
    with pytest.raises(ValueError, match="moved an existing native token"):
        a.update_block_table([2, 1, 3, -1])
    a.update_block_table(torch.tensor([2, 0, 3, 1]))
    assert a.decode(12, k[12], v[12]) == 4
    torch.testing.assert_close(a.gather(range(13))[0], k, rtol=0, atol=0)


def test_shared_prefix_slots_are_never_written_or_reused():
    a = arena(shared_slots={8, 9})
    k, v = kv(11, 12)
    with pytest.raises(ValueError, match="shared"):
        a.write_prefill(k[:10], v[:10])
    a.write(list(range(2, 10)), k[2:10], v[2:10])
    a.promote_selected([1], k[[1]] + 1, v[[1]] + 1).result()  # copied out of the shared slot
    assert a.snapshot()[1] == 16
    assert a.stats()["vacated_slots"] == 0
    with pytest.raises(ValueError, match="shared"):
        a.update_selected([0], k[[0]], v[[0]])
    assert a.decode(10, k[10], v[10]) == 14


def test_page_metadata_and_spill_order_follow_relocation():
    a = arena()
    k, v = kv(10, 13)
    a.write_prefill(k, v)
    a.write_selected_ready([4], k[[4]], v[[4]])  # page 0 holds a selected token in place
    a.promote_selected([9], k[[9]], v[[9]]).result()  # token 9 moves to sidecar page 4
    pages = {p["page_id"]: p for p in a.page_metadata()}
    assert sorted(pages) == [0, 2, 3, 4]
    assert (pages[0]["mapped_tokens"], pages[0]["selected_count"]) == (4, 1)
    assert (pages[3]["mapped_tokens"], pages[3]["selected_count"]) == (1, 0)
    assert (pages[4]["mapped_tokens"], pages[4]["selected_count"], pages[4]["dirty"]) == (1, 1, True)
    assert a.spill_order() == (2, 3, 0, 4)
    with a.slot_map.pin_slots([8]):
        assert a.spill_order() == (3, 0, 4)


def test_argument_validation():
    cache = torch.zeros((4, 2, 4, 6))
    for bad in (torch.zeros((4, 2, 4, 5)), torch.zeros((4, 2, 4)), torch.zeros((4, 2, 4, 6), dtype=torch.int32)):
        with pytest.raises(ValueError, match="cache must be floating"):
            NativePagedKV(bad, [0], 1, 0, mover=HostMover())
    for table in ([], [4], [0, -2], torch.tensor([[0]])):
        with pytest.raises(ValueError, match="block_table"):
            NativePagedKV(cache, table, 1, 0, mover=HostMover())
    with pytest.raises(ValueError, match="distinct native slots"):
        NativePagedKV(cache, [0, 0], 8, 0, mover=HostMover())
    with pytest.raises(ValueError, match="prompt_length"):
        NativePagedKV(cache, [0], 0, 0, mover=HostMover())
    with pytest.raises(ValueError, match="max_selected"):
        NativePagedKV(cache, [0], 1, -1, mover=HostMover())
    with pytest.raises(ValueError, match="layer_index"):
        NativePagedKV(cache, [0], 1, 0, layer_index=-1, mover=HostMover())
    with pytest.raises(ValueError, match="cacheslide_amd computes on the HIP device"):
        NativePagedKV(cache, [0], 1, 0)  # the product mover needs device tensors
    a = arena()
    k, v = kv(3, 14)
    with pytest.raises(ValueError, match="K/V must match"):
        a.write([0, 1], k, v)
    with pytest.raises(ValueError, match="distinct"):
        a.write([0, 0, 1], k, v)
    with pytest.raises(ValueError, match="nonnegative"):
        a.gather([-1])
    with pytest.raises(KeyError):
        a.write([10, 11, 12], k, v)
    with pytest.raises(TypeError):
        a.promote_selected([0], k[:1], v[:1], load_future=object())


def test_relocated_arena_sequence_on_the_host():
    """The arena sequence the fused-kernel GPU tests build (promotion to the
    sidecar, baseline write, pinned-mirror update, decode hole reuse), run
    with the host mover: the slot map names sidecar rows and reused holes,
    and device_slots yields exactly the slots gather reads."""
    from tests._helpers import HostMover
    from tests.test_gpu_arena_fused import relocated_arena

    arena, _ = relocated_arena(torch.device("cpu"), mover=HostMover())
    n = arena.logical_length()
    assert n == 624
    stats = arena.stats()
    assert stats["physical_hole_reuse"] > 0 and stats["canonical_mirror_writes"] > 0
    with arena.device_slots(range(n)) as (slots, side_k, side_v):
        snap = arena.snapshot()
        assert slots.tolist() == [snap[t] for t in range(n)]
        assert side_k is not None and side_v is not None
        canonical = [arena.canonical_slot(t) for t in range(n)]
        assert any(s >= arena.native_total_slots for s in slots.tolist())
        assert slots.tolist() != canonical
    gk, _ = arena.gather(range(n))
    assert gk.shape == (n, 2, 128)
