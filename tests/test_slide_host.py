"""Host metadata of SLIDE (slot maps and write runs) on the CPU.

Rules under test follow src/cacheslide_vllm/slide.py:
  coalesce_slot_writes       :27-51   adjacent equal-size records merge into runs
  _fresh_slot                :103-112 lowest returned slot first, else the next never-used slot
  promote_selected           :243-372 copy-on-write vs in-place, publication after completion
  allocate/bind_decode       :374-459 lowest reusable hole, native slots below the floor
  pin/write guards           :158-241 pins, in-flight reservations, retirement
The scenarios are this package's own; expected values are derived from those rules
(the reference's tests in tests/test_slide.py exercise the same rules).
"""

from __future__ import annotations

from concurrent.futures import Future

import pytest

from cacheslide_amd.slide import LayerSlotMap, SlotWrite, coalesce_slot_writes
from cacheslide_amd.errors import CacheCapacityError, StaleCompletionError


def done(value=None) -> Future:
    f = Future()
    f.set_result(value)
    return f


# ------------------------------------------------------------- write runs
def test_coalesce_merges_consecutive_slots_in_slot_order():
    runs = coalesce_slot_writes({7: b"q", 5: b"o", 6: b"p", 10: b"z", 12: b"y", 11: b"x"})
    assert runs == [SlotWrite(5, 3, b"opq"), SlotWrite(10, 3, b"zxy")]
    assert coalesce_slot_writes({}) == []
    with pytest.raises(ValueError):
        coalesce_slot_writes({3: b"aa", 4: b"b"})  # one record size per call
    with pytest.raises(ValueError):
        coalesce_slot_writes({-1: b"a"})
    with pytest.raises(ValueError):
        coalesce_slot_writes({0: b""})


# ------------------------------------------------------- allocation order
def test_fresh_slots_follow_the_highest_mapped_slot_and_holes_are_reused_lowest_first():
    m = LayerSlotMap({0: 3, 1: 4}, max_slots=8)
    assert m.promote_selected({0: b"k"}, lambda runs: None).result() == {0: 5, 1: 4}
    assert m.stats()["vacated_slots"] == 1
    assert m.allocate_decode(2) == 3  # the vacated source
    assert m.allocate_decode(3) == 6
    assert m.allocate_decode(4) == 7
    with pytest.raises(CacheCapacityError):
        m.allocate_decode(5)
    assert m.snapshot() == {0: 5, 1: 4, 2: 3, 3: 6, 4: 7}


def test_pending_load_keeps_the_source_unavailable_until_it_lands():
    m = LayerSlotMap({0: 0, 1: 1, 2: 2}, max_slots=6)
    load, write, runs = Future(), Future(), []
    completion = m.promote_selected({2: b"n"}, lambda r: runs.extend(r) or write, load_future=load)
    assert runs == [SlotWrite(3, 1, b"n")]  # a load in flight forces a copy
    assert m.snapshot() == {0: 0, 1: 1, 2: 2}  # nothing is published before the write
    assert m.allocate_decode(3) == 4  # neither source nor destination is a hole yet
    write.set_result(None)
    assert completion.result() == {0: 0, 1: 1, 2: 3, 3: 4}
    assert m.allocate_decode(4) == 5  # slot 2 still receives its load
    with pytest.raises(CacheCapacityError):
        m.allocate_decode(5)
    load.set_result(None)
    assert m.allocate_decode(5) == 2


def test_ready_unshared_unguarded_source_is_written_in_place():
    m = LayerSlotMap({0: 0, 1: 1}, max_slots=2)
    runs = []
    result = m.promote_selected({0: b"y"}, lambda r: runs.extend(r), load_future=done(),
                                allow_inplace=True)
    assert result.result() == {0: 0, 1: 1}
    assert runs == [SlotWrite(0, 1, b"y")]
    assert m.stats()["vacated_slots"] == 0


def test_shared_sources_are_copied_and_never_reclaimed():
    m = LayerSlotMap({0: 0, 1: 1}, shared_slots={0}, max_slots=3)
    runs = []
    assert m.promote_selected({0: b"s"}, lambda r: runs.extend(r), allow_inplace=True).result() == {0: 2, 1: 1}
    assert runs[0].start_slot == 2
    assert m.stats()["vacated_slots"] == 0
    with pytest.raises(CacheCapacityError):
        m.allocate_decode(2)


def test_a_source_mapped_twice_is_copied():
    m = LayerSlotMap({0: 4, 1: 4}, max_slots=6)
    assert m.promote_selected({0: b"d"}, lambda r: None, allow_inplace=True).result() == {0: 5, 1: 4}
    assert m.stats()["vacated_slots"] == 0  # slot 4 still backs token 1


def test_pins_force_copy_on_write_and_delay_reclamation():
    m = LayerSlotMap({0: 0, 1: 1}, max_slots=3)
    with m.pin_slots([0]):
        assert m.promote_selected({0: b"p"}, lambda r: None, allow_inplace=True).result()[0] == 2
        with pytest.raises(CacheCapacityError):
            m.allocate_decode(2)  # the vacated slot is pinned
    assert m.allocate_decode(2) == 0


def test_an_existing_write_guard_forces_an_independent_destination():
    m = LayerSlotMap({0: 0}, max_slots=2)
    write = Future()
    with m.write_guard([0]):
        completion = m.promote_selected({0: b"w"}, lambda r: write, allow_inplace=True)
        write.set_result(None)
        assert completion.result() == {0: 1}
        with pytest.raises(CacheCapacityError):
            m.allocate_decode(1)
    assert m.allocate_decode(1) == 0


def test_load_landing_during_the_write_keeps_the_copy_destination():
    m = LayerSlotMap({0: 0}, max_slots=2)
    load, write, runs = Future(), Future(), []

    def writer(r):
        runs.extend(r)
        load.set_result(None)  # the load finishes while the write is running
        return write

    completion = m.promote_selected({0: b"x"}, writer, load_future=load, allow_inplace=True)
    assert runs[0].start_slot == 1
    write.set_result(None)
    assert completion.result() == {0: 1}
    assert m.allocate_decode(1) == 0


# ------------------------------------------------------ failures and retirement
def test_a_failed_write_publishes_nothing_and_returns_its_destination():
    m = LayerSlotMap({0: 0, 1: 1}, max_slots=4)
    arena = {0: b"a", 1: b"b"}
    write = Future()

    def writer(r):
        arena[r[0].start_slot] = r[0].payload
        return write

    completion = m.promote_selected({0: b"Z"}, writer)
    write.set_exception(OSError("device lost"))
    with pytest.raises(OSError, match="device lost"):
        completion.result()
    assert m.snapshot() == {0: 0, 1: 1}
    assert arena[0] == b"a"  # the source record is untouched
    assert m.allocate_decode(2) == 2  # the failed destination is free again

    def raising(r):
        raise ValueError("writer refused")

    failed = m.promote_selected({1: b"Q"}, raising)
    assert isinstance(failed.exception(), ValueError)
    assert m.allocate_decode(3) == 3
    assert m.stats()["inflight_slots"] == 0


def test_a_multi_token_reservation_that_runs_out_leaks_nothing():
    m = LayerSlotMap({0: 0, 1: 1, 2: 2}, max_slots=4)
    with pytest.raises(CacheCapacityError):
        m.promote_selected({0: b"a", 1: b"b"}, lambda r: None)
    assert m.snapshot() == {0: 0, 1: 1, 2: 2}
    assert m.stats()["inflight_slots"] == 0
    assert m.allocate_decode(3) == 3


def test_retirement_rejects_late_completions_and_every_later_use():
    m = LayerSlotMap({5: 9})
    write = Future()
    completion = m.promote_selected({5: b"x"}, lambda r: write)
    m.invalidate()
    write.set_result(None)
    with pytest.raises(StaleCompletionError):
        completion.result()
    with pytest.raises(StaleCompletionError):
        m.snapshot()
    with pytest.raises(StaleCompletionError):
        m.allocate_decode(6)
    assert m.stats()["inflight_slots"] == 0
    assert m.stats()["generation"] == 1


def test_duplicate_pending_writes_unknown_tokens_and_failed_loads_are_rejected():
    m = LayerSlotMap({0: 0})
    write = Future()
    first = m.promote_selected({0: b"a"}, lambda r: write)
    with pytest.raises(RuntimeError):
        m.promote_selected({0: b"b"}, lambda r: None)
    write.set_result(None)
    assert first.result() == {0: 1}
    with pytest.raises(KeyError):
        m.promote_selected({7: b"x"}, lambda r: None)
    with pytest.raises(ValueError):
        m.promote_selected({0: b"ab", 7: b"c"}, lambda r: None)
    lost = Future()
    lost.set_exception(OSError("load lost"))
    with pytest.raises(OSError, match="load lost"):
        m.promote_selected({0: b"c"}, lambda r: None, load_future=lost)
    assert m.promote_selected({}, lambda r: None).result() == {0: 1}


# ---------------------------------------------------------- native slots
def test_sidecar_slots_start_at_the_allocation_floor():
    m = LayerSlotMap({0: 5, 1: 6}, allocation_floor=64, max_slots=66)
    runs = []
    assert m.promote_selected({0: b"a", 1: b"b"}, lambda r: runs.extend(r)).result() == {0: 64, 1: 65}
    assert runs == [SlotWrite(64, 2, b"ab")]
    assert m.bind_decode(2, 30) == 30
    with pytest.raises(ValueError):
        m.bind_decode(3, 64)  # not a native slot
    with pytest.raises(CacheCapacityError):
        m.bind_decode(3, 30)  # already mapped
    assert m.bind_decode(3, 40, reuse_vacated=True) == 5  # lowest hole below the floor
    assert m.bind_decode(4, 41, reuse_vacated=True) == 6
    assert m.bind_decode(5, 42, reuse_vacated=True) == 42
    assert m.snapshot() == {0: 64, 1: 65, 2: 30, 3: 5, 4: 6, 5: 42}


def test_native_binding_skips_holes_that_are_still_loading():
    m = LayerSlotMap({0: 0, 1: 1}, allocation_floor=16, max_slots=20)
    load, write = Future(), Future()
    completion = m.promote_selected({0: b"x"}, lambda r: write, load_future=load)
    write.set_result(None)
    assert completion.result() == {0: 16, 1: 1}
    assert m.bind_decode(2, 7, reuse_vacated=True) == 7
    load.set_result(None)
    assert m.bind_decode(3, 8, reuse_vacated=True) == 0


def test_native_binding_rejects_shared_and_pinned_slots():
    m = LayerSlotMap({0: 0, 1: 1}, shared_slots={0}, allocation_floor=10)
    with pytest.raises(CacheCapacityError):
        m.bind_decode(2, 0)
    with m.pinned_mapping([1]) as view:
        m.promote_selected({1: b"v"}, lambda r: None).result()
        assert view == {1: 1}  # the pinned snapshot keeps the old slot
        with pytest.raises(CacheCapacityError):
            m.bind_decode(2, 1)
    assert m.bind_decode(2, 1) == 1


def test_decode_write_guard_reserves_both_slots_and_publishes_after_the_body():
    m = LayerSlotMap({0: 0, 1: 1}, allocation_floor=16, max_slots=18)
    m.promote_selected({0: b"s"}, lambda r: None).result()
    before = m.snapshot()
    assert before == {0: 16, 1: 1}
    with m.decode_write_guard(2, 5, reuse_vacated=True) as chosen:
        assert chosen == 0
        assert m.snapshot() == before
        assert m.stats()["inflight_slots"] == 2
        with pytest.raises(KeyError):
            with m.pinned_mapping([2]):
                pass
        with pytest.raises(ValueError):
            with m.pin_slots([0]):
                pass
        with pytest.raises(RuntimeError, match="in-flight"):
            with m.write_guard([5]):
                pass
        with pytest.raises(CacheCapacityError):
            m.bind_decode(3, 5)
        with pytest.raises(ValueError):
            m.allocate_decode(2)
        with m.pinned_mapping([1]) as view:
            assert view == {1: 1}
    assert m.snapshot() == {**before, 2: 0}
    assert m.stats()["inflight_slots"] == 0
    with m.decode_write_guard(3, 6) as chosen:
        assert chosen == 6
    assert m.snapshot()[3] == 6


def test_a_failed_decode_write_retires_the_map():
    m = LayerSlotMap({0: 0}, allocation_floor=8)
    with pytest.raises(OSError):
        with m.decode_write_guard(1, 1):
            raise OSError("copy failed")
    assert m.stats()["mapped_tokens"] == 1
    assert m.stats()["inflight_slots"] == 0
    with pytest.raises(StaleCompletionError):
        m.snapshot()


def test_an_invalid_decode_destination_fails_before_the_body():
    m = LayerSlotMap({0: 0}, allocation_floor=8)
    with pytest.raises(CacheCapacityError):
        with m.decode_write_guard(1, 0):
            pytest.fail("the body must not run")
    assert m.snapshot() == {0: 0}
    with m.decode_write_guard(1, 3):
        pass
    assert m.snapshot() == {0: 0, 1: 3}


# ------------------------------------------------------------ write guards
def test_write_guard_drops_blocked_optional_slots():
    m = LayerSlotMap({0: 0, 1: 1, 2: 2, 3: 3}, shared_slots={3}, allocation_floor=8, max_slots=12)
    with m.pin_slots([0]):
        with m.write_guard([8], optional_slots=[0, 1, 2, 3]) as mirrors:
            assert mirrors == {1, 2}
            assert m.stats()["inflight_slots"] == 3
            with pytest.raises(RuntimeError, match="being written"):
                with m.pin_slots([1]):
                    pass
    assert m.stats()["inflight_slots"] == 0
    with m.pin_slots([0, 1, 2]):
        pass


def test_a_rejected_required_guard_reserves_nothing():
    m = LayerSlotMap({0: 0, 1: 1})
    with m.pin_slots([1]):
        with pytest.raises(RuntimeError, match="pinned or in-flight"):
            with m.write_guard([0, 1]):
                pytest.fail("the body must not run")
        with m.pin_slots([0]):
            pass
    with m.write_guard([0, 1]):
        assert m.stats()["inflight_slots"] == 2
    assert m.stats()["inflight_slots"] == 0


def test_write_guard_validation_errors_and_release():
    m = LayerSlotMap({0: 0, 1: 1}, shared_slots={1})
    with pytest.raises(ValueError, match="shared"):
        with m.write_guard([1]):
            pass
    for bad in (-2, True, 0.0):
        with pytest.raises(ValueError, match="nonnegative integers"):
            with m.write_guard([], optional_slots=[0, bad]):
                pass
    with pytest.raises(OSError):
        with m.write_guard([0]):
            raise OSError("copy failed")
    assert m.stats()["inflight_slots"] == 0
    with pytest.raises(StaleCompletionError):
        with m.write_guard([0]):
            m.invalidate()
    assert m.stats()["inflight_slots"] == 0


# ------------------------------------------------------------- construction
@pytest.mark.parametrize("floor", [-3, False, 2.0])
def test_allocation_floor_must_be_a_nonnegative_integer(floor):
    with pytest.raises(ValueError, match="allocation_floor"):
        LayerSlotMap({0: 0}, allocation_floor=floor)


def test_constructor_rejects_small_arenas_and_foreign_shared_slots():
    with pytest.raises(ValueError):
        LayerSlotMap({0: 5}, max_slots=5)
    with pytest.raises(ValueError):
        LayerSlotMap({0: 0}, shared_slots={4})
    with pytest.raises(ValueError):
        LayerSlotMap({-1: 0})


# ------------------------------------------------------------- page metadata
def test_page_metadata_counts_selected_tokens_and_guards_per_page():
    m = LayerSlotMap({0: 0, 1: 1, 2: 17, 3: 18, 4: 40}, shared_slots={17}, max_slots=64)
    with m.pin_slots([40]):
        pages = m.page_metadata(16, [1, 3])
    assert [p["page_id"] for p in pages] == [0, 1, 2]
    p0, p1, p2 = pages
    assert (p0["mapped_tokens"], p0["selected_count"], p0["dirty"], p0["spill_eligible"]) == (2, 1, True, True)
    assert (p1["mapped_tokens"], p1["selected_count"], p1["shared"], p1["spill_eligible"]) == (2, 1, True, False)
    assert (p2["mapped_tokens"], p2["dirty"], p2["pinned"], p2["spill_eligible"]) == (1, False, True, False)
    with pytest.raises(ValueError):
        m.page_metadata(0, [])
    with pytest.raises(ValueError):
        m.page_metadata(16, [9])
