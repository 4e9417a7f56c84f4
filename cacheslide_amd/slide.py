"""Per-layer SLIDE slot redirection with completion-ordered publication.

Host metadata counterpart of src/cacheslide_vllm/slide.py:20-520 with the same
allocation order, guard rules and exceptions.  It owns no device memory; the
bytes behind the slots are moved by the slot kernels (see paged.py).

Slot allocation order (``_fresh_slot``, slide.py:103-112): the lowest slot
returned to the unused pool first, otherwise the next never-used slot.
Decode reuse (slide.py:374-459) takes the lowest vacated slot that is not
mapped, shared, pinned or in flight.

State is kept per slot: a count of tokens mapped to it, and one guard record
(pins, in-flight reservations, writes) per guarded slot.  Returned slots and
vacated holes sit in min-heaps, so choosing a slot costs O(log n) instead of
a scan of the whole map; a hole that is guarded right now is skipped and
stays a hole.
"""

from __future__ import annotations

import heapq
import threading
from collections import Counter
from collections.abc import Callable, Iterable, Iterator, Mapping
from concurrent.futures import Future
from contextlib import contextmanager
from dataclasses import dataclass, field

from .errors import CacheCapacityError, StaleCompletionError


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


class _SlotHeap:
    """Min-heap of distinct slots; removal is lazy (stale heap entries are skipped)."""

    def __init__(self) -> None:
        self._heap: list[int] = []
        self._members: set[int] = set()

    def __len__(self) -> int:
        return len(self._members)

    def __contains__(self, slot: int) -> bool:
        return slot in self._members

    def add(self, slot: int) -> None:
        if slot not in self._members:
            self._members.add(slot)
            heapq.heappush(self._heap, slot)

    def discard(self, slot: int) -> None:
        self._members.discard(slot)

    def take_lowest(self) -> int | None:
        while self._heap:
            slot = heapq.heappop(self._heap)
            if slot in self._members:
                self._members.remove(slot)
                return slot
        return None

    def lowest(self, usable: Callable[[int], bool], below: int | None = None) -> int | None:
        """Lowest member (under ``below``) that ``usable`` accepts; it stays a member."""
        passed: list[int] = []
        found = None
        while self._heap:
            slot = self._heap[0]
            if slot not in self._members:
                heapq.heappop(self._heap)
                continue
            if below is not None and slot >= below:
                break
            if usable(slot):
                found = slot
                break
            passed.append(heapq.heappop(self._heap))
        for slot in passed:
            heapq.heappush(self._heap, slot)
        return found


_PINS, _FLIGHT, _WRITES = 0, 1, 2


@dataclass
class _Promotion:
    """One promote_selected call between reservation and publication."""

    generation: int
    tokens: frozenset[int]
    source: dict[int, int]  # token -> slot it is read from
    target: dict[int, int]  # token -> slot it is written to
    fresh: set[int] = field(default_factory=set)  # targets taken from the fresh pool
    flight: set[int] = field(default_factory=set)  # slots reserved until completion
    writes: set[int] = field(default_factory=set)  # slots that reject new readers


class LayerSlotMap:
    """Thread-safe token -> slot map for one request and one model layer
    (slide.py:54-520): completion-ordered publication of selected writes,
    copy-on-write unless an in-place write is safe, decode reuse of holes."""

    def __init__(
        self,
        initial_slots: Mapping[int, int],
        *,
        shared_slots: Iterable[int] = (),
        max_slots: int | None = None,
        allocation_floor: int = 0,
    ):
        mapping = dict(initial_slots)
        for token, slot in mapping.items():
            if type(token) is not int or token < 0 or type(slot) is not int or slot < 0:
                raise ValueError("tokens and slots must be nonnegative integers")
        refs = Counter(mapping.values())
        shared = frozenset(shared_slots)
        if any(slot not in refs for slot in shared):
            raise ValueError("shared slots must be present in the initial mapping")
        if type(allocation_floor) is not int or allocation_floor < 0:
            raise ValueError("allocation_floor must be a nonnegative integer")
        next_slot = max(allocation_floor, max(refs, default=-1) + 1)
        if max_slots is not None and (type(max_slots) is not int or max_slots < next_slot):
            raise ValueError("max_slots is smaller than the initial arena")
        self.allocation_floor = allocation_floor
        self.max_slots = max_slots
        self._lock = threading.RLock()
        self._map = mapping
        self._refs = refs  # slot -> number of tokens mapped to it
        self._shared = shared
        self._guards: dict[int, list[int]] = {}  # slot -> [pins, in-flight, writes]
        self._pending: set[int] = set()  # tokens with a write in flight
        self._next_slot = next_slot
        self._returned = _SlotHeap()  # reserved fresh slots given back unused
        self._holes = _SlotHeap()  # vacated sources, reusable by decode
        self._generation = 0
        self._closed = False

    # -- per-slot state (lock held) ---------------------------------------------
    def _open(self) -> None:
        if self._closed:
            raise StaleCompletionError("layer slot map is retired")

    def _count(self, slot: int, kind: int) -> int:
        record = self._guards.get(slot)
        return record[kind] if record else 0

    def _guard(self, slots: Iterable[int], kind: int, delta: int) -> None:
        for slot in slots:
            record = self._guards.setdefault(slot, [0, 0, 0])
            record[kind] += delta
            if not any(record):
                del self._guards[slot]

    def _blocked(self, slot: int) -> bool:
        """Pinned or reserved: no new writer and no reclamation."""
        record = self._guards.get(slot)
        return bool(record and (record[_PINS] or record[_FLIGHT]))

    def _reclaimable(self, slot: int) -> bool:
        return not self._refs[slot] and slot not in self._shared and not self._blocked(slot)

    def _remap(self, token: int, slot: int) -> None:
        old = self._map.get(token)
        if old is not None:
            self._refs[old] -= 1
            if not self._refs[old]:
                del self._refs[old]
        self._map[token] = slot
        self._refs[slot] += 1

    def _fresh_slot(self) -> int:
        slot = self._returned.take_lowest()
        if slot is not None:
            return slot
        if self.max_slots is not None and self._next_slot >= self.max_slots:
            raise CacheCapacityError("sidecar slot arena is full")
        self._next_slot += 1
        return self._next_slot - 1

    # -- reads ----------------------------------------------------------------
    def snapshot(self) -> dict[int, int]:
        with self._lock:
            self._open()
            return dict(self._map)

    def page_metadata(
        self, page_size: int, selected_tokens: Iterable[int]
    ) -> tuple[dict[str, int | bool], ...]:
        """Per physical page: mapped and selected token counts and the guard state
        that makes it ineligible to spill (slide.py:119-156)."""
        if type(page_size) is not int or page_size < 1:
            raise ValueError("page_size must be a positive integer")
        selected = set(selected_tokens)
        with self._lock:
            self._open()
            if any(type(token) is not int or token not in self._map for token in selected):
                raise ValueError("selected tokens must have current logical mappings")
            pages: dict[int, list[int]] = {}  # page -> [mapped tokens, selected tokens]
            for token, slot in self._map.items():
                entry = pages.setdefault(slot // page_size, [0, 0])
                entry[0] += 1
                entry[1] += token in selected
            shared = {slot // page_size for slot in self._shared}
            pinned = {slot // page_size for slot, g in self._guards.items() if g[_PINS]}
            flying = {slot // page_size for slot, g in self._guards.items() if g[_FLIGHT]}
            out = []
            for page in sorted(pages):
                mapped, chosen = pages[page]
                out.append({
                    "page_id": page,
                    "mapped_tokens": mapped,
                    "selected_count": chosen,
                    "dirty": chosen > 0,
                    "shared": page in shared,
                    "pinned": page in pinned,
                    "inflight": page in flying,
                    "spill_eligible": not (page in shared or page in pinned or page in flying),
                })
            return tuple(out)

    # -- guards ---------------------------------------------------------------
    def _pin(self, slots: set[int]) -> None:
        if any(self._count(slot, _WRITES) for slot in slots):
            raise RuntimeError("physical slots are being written")
        self._guard(slots, _PINS, +1)

    def _unpin(self, slots: set[int]) -> None:
        with self._lock:
            self._guard(slots, _PINS, -1)

    @contextmanager
    def pin_slots(self, slots: Iterable[int]) -> Iterator[None]:
        """Keep mapped slots from being written or reclaimed during a read."""
        wanted = set(slots)
        with self._lock:
            self._open()
            if any(slot not in self._refs for slot in wanted):
                raise ValueError("only currently mapped slots can be pinned")
            self._pin(wanted)
        try:
            yield
        finally:
            self._unpin(wanted)

    @contextmanager
    def pinned_mapping(self, tokens: Iterable[int]) -> Iterator[dict[int, int]]:
        """Snapshot and pin the slots of ``tokens`` in one step, for a gather."""
        tokens = tuple(tokens)
        with self._lock:
            self._open()
            if any(type(token) is not int or token < 0 for token in tokens):
                raise ValueError("tokens must be nonnegative integer positions")
            view = {token: self._map[token] for token in tokens}
            wanted = set(view.values())
            self._pin(wanted)
        try:
            yield view
        finally:
            self._unpin(wanted)

    def _reserve_writes(self, slots: set[int]) -> None:
        self._guard(slots, _WRITES, +1)
        self._guard(slots, _FLIGHT, +1)

    def _release_writes(self, slots: set[int]) -> None:
        with self._lock:
            self._guard(slots, _WRITES, -1)
            self._guard(slots, _FLIGHT, -1)

    @contextmanager
    def write_guard(
        self, slots: Iterable[int], *, optional_slots: Iterable[int] = ()
    ) -> Iterator[frozenset[int]]:
        """Reserve physical writes against readers and reclamation (slide.py:193-241).

        Every required slot must be unshared, unpinned and not in flight, or
        nothing is reserved; each optional slot is dropped when it is not.  The
        lock is not held inside the body.
        """
        required, optional = tuple(slots), tuple(optional_slots)
        if any(type(slot) is not int or slot < 0 for slot in required + optional):
            raise ValueError("write slots must be nonnegative integers")
        with self._lock:
            self._open()
            if any(slot in self._shared for slot in required):
                raise ValueError("required write slots cannot be shared")
            if any(self._blocked(slot) for slot in required):
                raise RuntimeError("required write slots are pinned or in-flight")
            mirrors = frozenset(
                slot for slot in set(optional) if slot not in self._shared and not self._blocked(slot)
            )
            held = set(required) | mirrors
            generation = self._generation
            self._reserve_writes(held)
        try:
            yield mirrors
            with self._lock:
                if self._closed or generation != self._generation:
                    raise StaleCompletionError("write completed for a retired layer")
        finally:
            self._release_writes(held)

    # -- selected promotion -----------------------------------------------------
    def _must_copy(self, slot: int, allow_inplace: bool, load_pending: bool) -> bool:
        return (
            not allow_inplace
            or load_pending
            or slot in self._shared
            or self._blocked(slot)
            or self._refs[slot] > 1
        )

    def _reserve_promotion(
        self, updates: dict[int, bytes], load_future: Future | None, allow_inplace: bool
    ) -> _Promotion | None:
        """Choose targets and take the guards (lock held); None for no updates."""
        self._open()
        if not updates:
            return None
        if any(token not in self._map for token in updates):
            raise KeyError("selected tokens must already have source slots")
        if any(token in self._pending for token in updates):
            raise RuntimeError("selected tokens already have an in-flight write")
        load_pending = load_future is not None and not load_future.done()
        if load_future is not None and not load_pending:
            load_future.result()  # a failed or cancelled load raises here: no overwrite
        job = _Promotion(self._generation, frozenset(updates),
                         {token: self._map[token] for token in updates}, {})
        try:
            for token, slot in job.source.items():
                if self._must_copy(slot, allow_inplace, load_pending):
                    target = self._fresh_slot()
                    job.fresh.add(target)
                else:
                    target = slot
                job.target[token] = target
        except BaseException:
            for slot in job.fresh:
                self._returned.add(slot)
            raise
        self._pending |= job.tokens
        job.writes = set(job.target.values())
        job.flight = set(job.source.values()) | job.writes
        self._guard(job.flight, _FLIGHT, +1)
        self._guard(job.writes, _WRITES, +1)
        if load_pending:
            # The sources stay reserved until their load lands, however the write ends.
            loading = set(job.source.values())
            self._guard(loading, _FLIGHT, +1)

            def load_landed(_: Future) -> None:
                with self._lock:
                    self._guard(loading, _FLIGHT, -1)

            load_future.add_done_callback(load_landed)
        return job

    def _complete_promotion(self, job: _Promotion, outcome: Future, error: BaseException | None) -> None:
        """Publish the targets, or give the fresh slots back; release the guards."""
        published = None
        try:
            if error is not None:
                raise error
            with self._lock:
                if self._closed or job.generation != self._generation:
                    raise StaleCompletionError("selected write completed for a retired layer")
                if any(self._map[token] != slot for token, slot in job.source.items()):
                    raise StaleCompletionError("source mapping changed before publication")
                for token, slot in job.target.items():
                    self._remap(token, slot)
                for slot in set(job.source.values()):
                    if slot not in self._refs and slot not in self._shared:
                        self._holes.add(slot)
                published = dict(self._map)
        except BaseException as exc:
            error = exc
            with self._lock:
                for slot in job.fresh:
                    self._returned.add(slot)
        finally:
            with self._lock:
                self._guard(job.writes, _WRITES, -1)
                self._guard(job.flight, _FLIGHT, -1)
                self._pending -= job.tokens
        if error is not None:
            outcome.set_exception(error)
        else:
            outcome.set_result(published)

    def promote_selected(
        self,
        updates: Mapping[int, bytes],
        writer: Callable[[list[SlotWrite]], Future | None],
        *,
        load_future: Future | None = None,
        allow_inplace: bool = False,
    ) -> Future[dict[int, int]]:
        """Write selected tokens and publish their slots after the write completes
        (slide.py:243-372).  The future holds the published map, or the error."""
        outcome: Future[dict[int, int]] = Future()
        outcome.set_running_or_notify_cancel()
        updates = dict(updates)
        coalesce_slot_writes(dict(enumerate(updates.values())))  # record checks, before any reservation
        with self._lock:
            job = self._reserve_promotion(updates, load_future, allow_inplace)
            if job is None:
                outcome.set_result(dict(self._map))
                return outcome
        runs = coalesce_slot_writes({job.target[token]: data for token, data in updates.items()})

        def written(done: Future) -> None:
            try:
                done.result()
            except BaseException as exc:
                self._complete_promotion(job, outcome, exc)
            else:
                self._complete_promotion(job, outcome, None)

        try:
            pending = writer(runs)
            if pending is None:
                self._complete_promotion(job, outcome, None)
            elif isinstance(pending, Future):
                pending.add_done_callback(written)
            else:
                raise TypeError("writer must return a concurrent Future or None")
        except BaseException as exc:
            self._complete_promotion(job, outcome, exc)
        return outcome

    # -- decode -----------------------------------------------------------------
    def _check_new_token(self, token: int) -> None:
        if type(token) is not int or token < 0 or token in self._map or token in self._pending:
            raise ValueError("decode token must be a new nonnegative position")

    def allocate_decode(self, token: int) -> int:
        """Map a new token to the lowest reusable hole, else a fresh slot."""
        with self._lock:
            self._open()
            self._check_new_token(token)
            slot = self._holes.lowest(self._reclaimable)
            if slot is not None:
                self._holes.discard(slot)
            else:
                slot = self._fresh_slot()
            self._remap(token, slot)
            return slot

    def _decode_destination(self, token: int, physical_slot: int, *, reuse_vacated: bool) -> int:
        """Validate a native slot and choose the destination (lock held)."""
        self._open()
        self._check_new_token(token)
        if type(physical_slot) is not int or not 0 <= physical_slot < self.allocation_floor:
            raise ValueError("native decode slot must be below allocation_floor")
        if physical_slot in self._refs or physical_slot in self._shared or self._blocked(physical_slot):
            raise CacheCapacityError("native decode slot is valid or guarded")
        if reuse_vacated:
            hole = self._holes.lowest(self._reclaimable, below=self.allocation_floor)
            if hole is not None:
                return hole
        return physical_slot

    def bind_decode(self, token: int, physical_slot: int, *, reuse_vacated: bool = False) -> int:
        """Bind a caller-owned native slot below the allocation floor (slide.py:441-459)."""
        with self._lock:
            chosen = self._decode_destination(token, physical_slot, reuse_vacated=reuse_vacated)
            self._holes.discard(chosen)
            self._remap(token, chosen)
            return chosen

    @contextmanager
    def decode_write_guard(
        self, token: int, physical_slot: int, *, reuse_vacated: bool = False
    ) -> Iterator[int]:
        """Reserve the decode destination and its canonical mirror, publish the
        token after the body; a failed body retires the map (slide.py:461-504)."""
        with self._lock:
            chosen = self._decode_destination(token, physical_slot, reuse_vacated=reuse_vacated)
            held = {chosen, physical_slot}
            generation = self._generation
            self._holes.discard(chosen)
            self._pending.add(token)
            self._reserve_writes(held)
        try:
            yield chosen
            with self._lock:
                if self._closed or generation != self._generation:
                    raise StaleCompletionError("decode write completed for a retired layer")
                self._remap(token, chosen)
        except BaseException:
            with self._lock:
                if not self._closed:
                    self.invalidate()
            raise
        finally:
            self._release_writes(held)
            with self._lock:
                self._pending.discard(token)

    def invalidate(self) -> None:
        """Retire the map: late completions cannot publish into it."""
        with self._lock:
            self._generation += 1
            self._closed = True

    def stats(self) -> dict[str, int]:
        with self._lock:
            return {
                "mapped_tokens": len(self._map),
                "vacated_slots": len(self._holes),
                "shared_slots": len(self._shared),
                "pinned_slots": sum(1 for g in self._guards.values() if g[_PINS] > 0),
                "inflight_slots": sum(1 for g in self._guards.values() if g[_FLIGHT] > 0),
                "generation": self._generation,
            }
