"""Per-layer SLIDE slot redirection with completion-ordered publication.

Host metadata counterpart of src/cacheslide_vllm/slide.py:20-520 with the same
allocation order, guard rules and exceptions.  It owns no device memory; the
bytes behind the slots are moved by the slot kernels (see paged.py).

Slot allocation order (``_fresh_slot``, slide.py:103-112): the lowest slot
returned to the unused pool first, otherwise the next never-used slot.
Decode reuse (slide.py:374-459) takes the lowest vacated slot that is not
mapped, shared, pinned or in flight.
"""

from __future__ import annotations

import threading
from collections import Counter
from collections.abc import Callable, Iterable, Iterator, Mapping
from concurrent.futures import Future
from contextlib import contextmanager
from dataclasses import dataclass

from .storage import CacheCapacityError, StaleCompletionError


@dataclass(frozen=True)
class SlotWrite:
    start_slot: int
    slot_count: int
    payload: bytes


def coalesce_slot_writes(writes: Mapping[int, bytes]) -> list[SlotWrite]:
    """Merge records of consecutive slots into runs (slide.py:27-51)."""
    if not writes:
        return []
    sizes = {len(payload) for payload in writes.values()}
    if len(sizes) != 1 or 0 in sizes:
        raise ValueError("token records must have one positive byte size")
    for slot, payload in writes.items():
        if type(slot) is not int or slot < 0 or not isinstance(payload, bytes):
            raise ValueError("slots must be nonnegative integers and records bytes")
    runs: list[SlotWrite] = []
    run_start = None
    run_parts: list[bytes] = []
    previous = None
    for slot in sorted(writes):
        if run_parts and slot != previous + 1:
            runs.append(SlotWrite(run_start, len(run_parts), b"".join(run_parts)))
            run_parts = []
        if not run_parts:
            run_start = slot
        run_parts.append(writes[slot])
        previous = slot
    runs.append(SlotWrite(run_start, len(run_parts), b"".join(run_parts)))
    return runs


class LayerSlotMap:
    """Thread-safe token -> slot map for one request and one model layer."""

    def __init__(
        self,
        initial_slots: Mapping[int, int],
        *,
        shared_slots: Iterable[int] = (),
        max_slots: int | None = None,
        allocation_floor: int = 0,
    ):
        self._map = dict(initial_slots)
        for token, slot in self._map.items():
            if type(token) is not int or token < 0 or type(slot) is not int or slot < 0:
                raise ValueError("tokens and slots must be nonnegative integers")
        self._shared = set(shared_slots)
        if not self._shared <= set(self._map.values()):
            raise ValueError("shared slots must be present in the initial mapping")
        if type(allocation_floor) is not int or allocation_floor < 0:
            raise ValueError("allocation_floor must be a nonnegative integer")
        self.allocation_floor = allocation_floor
        highest = max(self._map.values(), default=-1)
        self._next_slot = max(allocation_floor, highest + 1)
        if max_slots is not None and (
            type(max_slots) is not int or max_slots < self._next_slot or max_slots < 0
        ):
            raise ValueError("max_slots is smaller than the initial arena")
        self.max_slots = max_slots
        self._mutex = threading.RLock()
        self._pins: Counter[int] = Counter()
        self._inflight: Counter[int] = Counter()
        self._writes: Counter[int] = Counter()
        self._pending_tokens: set[int] = set()
        self._vacated: set[int] = set()
        self._unused: set[int] = set()
        self._generation = 0
        self._closed = False

    # -- helpers (mutex held) -------------------------------------------------
    def _check_open(self) -> None:
        if self._closed:
            raise StaleCompletionError("layer slot map is retired")

    def _fresh_slot(self) -> int:
        if self._unused:
            slot = min(self._unused)
            self._unused.discard(slot)
            return slot
        if self.max_slots is not None and self._next_slot >= self.max_slots:
            raise CacheCapacityError("sidecar slot arena is full")
        slot = self._next_slot
        self._next_slot += 1
        return slot

    def _guarded(self, slot: int) -> bool:
        return bool(self._pins[slot] or self._inflight[slot])

    def _reusable_holes(self, below: int | None = None) -> list[int]:
        valid = set(self._map.values())
        return sorted(
            slot
            for slot in self._vacated
            if (below is None or slot < below)
            and slot not in valid
            and slot not in self._shared
            and not self._guarded(slot)
        )

    # -- reads ----------------------------------------------------------------
    def snapshot(self) -> dict[int, int]:
        with self._mutex:
            self._check_open()
            return dict(self._map)

    def page_metadata(
        self, page_size: int, selected_tokens: Iterable[int]
    ) -> tuple[dict[str, int | bool], ...]:
        """Per physical page: mapped/selected counts and guard state (slide.py:119-156)."""
        if type(page_size) is not int or page_size < 1:
            raise ValueError("page_size must be a positive integer")
        selected = set(selected_tokens)
        with self._mutex:
            self._check_open()
            if any(type(token) is not int for token in selected) or not selected <= set(self._map):
                raise ValueError("selected tokens must have current logical mappings")
            mapped = Counter(slot // page_size for slot in self._map.values())
            chosen = Counter(self._map[token] // page_size for token in selected)
            shared = {slot // page_size for slot in self._shared}
            pinned = {slot // page_size for slot, n in self._pins.items() if n}
            inflight = {slot // page_size for slot, n in self._inflight.items() if n}
            blocked = shared | pinned | inflight
            return tuple(
                {
                    "page_id": page,
                    "mapped_tokens": mapped[page],
                    "selected_count": chosen[page],
                    "dirty": chosen[page] > 0,
                    "shared": page in shared,
                    "pinned": page in pinned,
                    "inflight": page in inflight,
                    "spill_eligible": page not in blocked,
                }
                for page in sorted(mapped)
            )

    # -- guards ---------------------------------------------------------------
    @contextmanager
    def pin_slots(self, slots: Iterable[int]) -> Iterator[None]:
        unique = set(slots)
        with self._mutex:
            self._check_open()
            if not unique <= set(self._map.values()):
                raise ValueError("only currently mapped slots can be pinned")
            if any(self._writes[slot] for slot in unique):
                raise RuntimeError("physical slots are being written")
            self._pins.update(unique)
        try:
            yield
        finally:
            with self._mutex:
                self._pins.subtract(unique)

    @contextmanager
    def pinned_mapping(self, tokens: Iterable[int]) -> Iterator[dict[int, int]]:
        """Atomically snapshot and pin the mappings of ``tokens`` for a gather."""
        tokens = tuple(tokens)
        with self._mutex:
            self._check_open()
            if any(type(token) is not int or token < 0 for token in tokens):
                raise ValueError("tokens must be nonnegative integer positions")
            snapshot = {token: self._map[token] for token in tokens}
            slots = set(snapshot.values())
            if any(self._writes[slot] for slot in slots):
                raise RuntimeError("physical slots are being written")
            self._pins.update(slots)
        try:
            yield snapshot
        finally:
            with self._mutex:
                self._pins.subtract(slots)

    @contextmanager
    def write_guard(
        self, slots: Iterable[int], *, optional_slots: Iterable[int] = ()
    ) -> Iterator[frozenset[int]]:
        """Reserve physical writes against readers and reclamation (slide.py:193-241).

        Required slots must be unshared, unpinned and not in flight or nothing
        is reserved; optional slots are dropped individually when blocked.  The
        map mutex is not held inside the body.
        """
        required_list, optional_list = tuple(slots), tuple(optional_slots)
        for slot in required_list + optional_list:
            if type(slot) is not int or slot < 0:
                raise ValueError("write slots must be nonnegative integers")
        required, optional = set(required_list), set(optional_list)
        with self._mutex:
            self._check_open()
            if required & self._shared:
                raise ValueError("required write slots cannot be shared")
            if any(self._guarded(slot) for slot in required):
                raise RuntimeError("required write slots are pinned or in-flight")
            available = frozenset(
                slot for slot in optional if slot not in self._shared and not self._guarded(slot)
            )
            guarded = required | available
            generation = self._generation
            self._writes.update(guarded)
            self._inflight.update(guarded)
        try:
            yield available
            with self._mutex:
                if self._closed or generation != self._generation:
                    raise StaleCompletionError("write completed for a retired layer")
        finally:
            with self._mutex:
                self._writes.subtract(guarded)
                self._inflight.subtract(guarded)

    # -- selected promotion -----------------------------------------------------
    def promote_selected(
        self,
        updates: Mapping[int, bytes],
        writer: Callable[[list[SlotWrite]], Future | None],
        *,
        load_future: Future | None = None,
        allow_inplace: bool = False,
    ) -> Future[dict[int, int]]:
        """Write selected tokens and publish their new slots after completion (slide.py:243-372)."""
        result: Future[dict[int, int]] = Future()
        result.set_running_or_notify_cancel()
        updates = dict(updates)
        coalesce_slot_writes({i: data for i, data in enumerate(updates.values())})
        with self._mutex:
            self._check_open()
            if not updates:
                result.set_result(dict(self._map))
                return result
            if not set(updates) <= set(self._map):
                raise KeyError("selected tokens must already have source slots")
            if self._pending_tokens & set(updates):
                raise RuntimeError("selected tokens already have an in-flight write")
            load_pending = load_future is not None and not load_future.done()
            if load_future is not None and not load_pending:
                load_future.result()  # a failed load cannot justify overwriting
            generation = self._generation
            source = {token: self._map[token] for token in updates}
            multiplicity = Counter(self._map.values())
            destinations: dict[int, int] = {}
            allocated: set[int] = set()
            try:
                for token, old_slot in source.items():
                    copy = (
                        not allow_inplace
                        or load_pending
                        or old_slot in self._shared
                        or self._guarded(old_slot)
                        or multiplicity[old_slot] > 1
                    )
                    target = self._fresh_slot() if copy else old_slot
                    destinations[token] = target
                    if target != old_slot:
                        allocated.add(target)
            except BaseException:
                self._unused |= allocated
                raise
            self._pending_tokens |= set(updates)
            guarded = set(source.values()) | set(destinations.values())
            self._inflight.update(guarded)
            writing = set(destinations.values())
            self._writes.update(writing)
            if load_pending:
                loading = set(source.values())
                self._inflight.update(loading)

                def load_finished(_: Future) -> None:
                    with self._mutex:
                        self._inflight.subtract(loading)

                load_future.add_done_callback(load_finished)

        runs = coalesce_slot_writes({destinations[t]: data for t, data in updates.items()})

        def finish(write_future: Future | None = None, failure: BaseException | None = None) -> None:
            error: BaseException | None = None
            published: dict[int, int] | None = None
            try:
                if failure is not None:
                    raise failure
                if write_future is not None:
                    write_future.result()
                with self._mutex:
                    if self._closed or generation != self._generation:
                        raise StaleCompletionError("selected write completed for a retired layer")
                    for token, old_slot in source.items():
                        if self._map[token] != old_slot:
                            raise StaleCompletionError("source mapping changed before publication")
                    self._map.update(destinations)
                    live = set(self._map.values())
                    for old_slot in source.values():
                        if old_slot not in live and old_slot not in self._shared:
                            self._vacated.add(old_slot)
                    published = dict(self._map)
            except BaseException as exc:
                with self._mutex:
                    self._unused |= allocated
                error = exc
            finally:
                with self._mutex:
                    self._writes.subtract(writing)
                    self._inflight.subtract(guarded)
                    self._pending_tokens -= set(updates)
            if error is not None:
                result.set_exception(error)
            else:
                result.set_result(published)

        try:
            written = writer(runs)
            if written is None:
                finish()
            elif isinstance(written, Future):
                written.add_done_callback(finish)
            else:
                raise TypeError("writer must return a concurrent Future or None")
        except BaseException as exc:
            finish(failure=exc)
        return result

    # -- decode -----------------------------------------------------------------
    def _check_new_token(self, token: int) -> None:
        if (
            type(token) is not int
            or token < 0
            or token in self._map
            or token in self._pending_tokens
        ):
            raise ValueError("decode token must be a new nonnegative position")

    def allocate_decode(self, token: int) -> int:
        with self._mutex:
            self._check_open()
            self._check_new_token(token)
            holes = self._reusable_holes()
            if holes:
                slot = holes[0]
                self._vacated.discard(slot)
            else:
                slot = self._fresh_slot()
            self._map[token] = slot
            return slot

    def _decode_destination(self, token: int, physical_slot: int, *, reuse_vacated: bool) -> int:
        """Validate and choose a native destination (mutex held)."""
        self._check_open()
        self._check_new_token(token)
        if type(physical_slot) is not int or not 0 <= physical_slot < self.allocation_floor:
            raise ValueError("native decode slot must be below allocation_floor")
        if (
            physical_slot in self._map.values()
            or physical_slot in self._shared
            or self._guarded(physical_slot)
        ):
            raise CacheCapacityError("native decode slot is valid or guarded")
        if reuse_vacated:
            holes = self._reusable_holes(below=self.allocation_floor)
            if holes:
                return holes[0]
        return physical_slot

    def bind_decode(self, token: int, physical_slot: int, *, reuse_vacated: bool = False) -> int:
        """Bind a caller-owned native slot below the allocation floor (slide.py:441-459)."""
        with self._mutex:
            chosen = self._decode_destination(token, physical_slot, reuse_vacated=reuse_vacated)
            self._vacated.discard(chosen)
            self._map[token] = chosen
            return chosen

    @contextmanager
    def decode_write_guard(
        self, token: int, physical_slot: int, *, reuse_vacated: bool = False
    ) -> Iterator[int]:
        """Reserve decode and mirror destinations; publish after the body (slide.py:461-504)."""
        with self._mutex:
            chosen = self._decode_destination(token, physical_slot, reuse_vacated=reuse_vacated)
            guarded = {chosen, physical_slot}
            generation = self._generation
            self._vacated.discard(chosen)
            self._pending_tokens.add(token)
            self._writes.update(guarded)
            self._inflight.update(guarded)
        try:
            yield chosen
            with self._mutex:
                if self._closed or generation != self._generation:
                    raise StaleCompletionError("decode write completed for a retired layer")
                self._map[token] = chosen
        except BaseException:
            with self._mutex:
                if not self._closed:
                    self.invalidate()
            raise
        finally:
            with self._mutex:
                self._writes.subtract(guarded)
                self._inflight.subtract(guarded)
                self._pending_tokens.discard(token)

    def invalidate(self) -> None:
        with self._mutex:
            self._generation += 1
            self._closed = True

    def stats(self) -> dict[str, int]:
        with self._mutex:
            return {
                "mapped_tokens": len(self._map),
                "vacated_slots": len(self._vacated),
                "shared_slots": len(self._shared),
                "pinned_slots": sum(1 for n in self._pins.values() if n > 0),
                "inflight_slots": sum(1 for n in self._inflight.values() if n > 0),
                "generation": self._generation,
            }
