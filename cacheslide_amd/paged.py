"""Request-local SLIDE indirection over the packed paged KV cache.

Counterpart of src/cacheslide_vllm/paged.py:21-581 (``NativePagedKV``).  The
native cache is [block, KV head, block offset, 2 * head dimension]; only slots
named by the caller's block table are written, and selected KV beyond the
native pool goes to a bounded sidecar allocated on first use.  The public
methods keep the reference's names, argument meaning, order of checks and
exceptions; the records move through the slot kernels (``cs_slot_scatter`` /
``cs_slot_gather``, arbitrary strides, bit-exact for every dtype).

Completion.  A write becomes publishable when the device has executed it, not
when it was enqueued (paged.py:35-54).  Synchronous paths record an event on
the current stream and wait on it in the calling thread.  The one asynchronous
path -- a selected-token promotion, whose mapping is published by
``LayerSlotMap`` once the write lands -- hands its event to a single watcher
thread that resolves the futures in submission order.  Callbacks attached to
those futures run on the watcher thread and must not wait on another
completion.

``mover`` selects who moves the bytes.  The default is the HIP library and
requires device tensors; tests inject a host mover with the same two methods
to exercise the metadata rules without a GPU.
"""

from __future__ import annotations

import queue
import threading
from collections.abc import Iterable, Sequence
from concurrent.futures import Future
from contextlib import contextmanager

import numpy as np
import torch

from . import _hip
from ._hip import call, ptr, vref
from .slide import LayerSlotMap, SlotWrite


def _indices(value: Sequence[int] | torch.Tensor, name: str) -> list[int]:
    """Distinct nonnegative token positions as a host list (token metadata only)."""
    if isinstance(value, torch.Tensor):
        if value.ndim != 1 or value.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"{name} must be an integer vector")
        value = value.detach().cpu().tolist()
    out = list(value)
    if any(type(item) is not int or item < 0 for item in out):
        raise ValueError(f"{name} must contain nonnegative integer positions")
    if len(set(out)) != len(out):
        raise ValueError(f"{name} must contain distinct positions")
    return out


class _CompletionWatcher:
    """One daemon thread resolves futures as their device events complete."""

    def __init__(self) -> None:
        self._jobs: queue.SimpleQueue = queue.SimpleQueue()
        self._lock = threading.Lock()
        self._thread: threading.Thread | None = None

    def submit(self, event) -> Future:
        done: Future = Future()
        done.set_running_or_notify_cancel()
        with self._lock:
            if self._thread is None or not self._thread.is_alive():
                self._thread = threading.Thread(target=self._run, name="cacheslide-kv-completion",
                                                daemon=True)
                self._thread.start()
        self._jobs.put((event, done))
        return done

    def _run(self) -> None:
        while True:
            event, done = self._jobs.get()
            try:
                event.synchronize()
            except BaseException as error:  # the device reported a failure
                done.set_exception(error)
            else:
                done.set_result(None)


_WATCHER = _CompletionWatcher()


def _completion_future(device: torch.device) -> Future:
    """Future resolved when the work enqueued so far on the current stream of
    ``device`` has executed (immediately for host tensors)."""
    if device.type != "cuda":
        done: Future = Future()
        done.set_running_or_notify_cancel()
        done.set_result(None)
        return done
    event = torch.cuda.Event()
    event.record(torch.cuda.current_stream(device))
    return _WATCHER.submit(event)


def _wait_device(device: torch.device) -> None:
    """Block the calling thread until the current stream's enqueued work has executed."""
    if device.type == "cuda":
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(device))
        event.synchronize()


class HipSlotMover:
    """Moves token records between dense [n, H, D] rows and paged slots on the device."""

    def scatter(self, cache, side_k, side_v, slots: list[int], key, value, rows=None) -> None:
        device = _hip.require_device(cache, key, value)
        slot_t = torch.tensor(slots, dtype=torch.long, device=device)
        row_t = None if rows is None else torch.tensor(rows, dtype=torch.long, device=device)
        call("cs_slot_scatter", vref(cache), vref(side_k), vref(side_v), ptr(slot_t), ptr(row_t),
             len(slots), vref(key), vref(value), _hip.stream_of(device))

    def gather(self, cache, side_k, side_v, slots: list[int], key, value) -> None:
        device = _hip.require_device(cache, key, value)
        slot_t = torch.tensor(slots, dtype=torch.long, device=device)
        call("cs_slot_gather", vref(cache), vref(side_k), vref(side_v), ptr(slot_t), ptr(None),
             len(slots), vref(key), vref(value), _hip.stream_of(device))


_DEFAULT_MOVER = HipSlotMover()
_FLOAT_TYPES = (torch.float16, torch.bfloat16, torch.float32, torch.float64)


class NativePagedKV:
    """One request/layer's native slots plus a selected-token sidecar (paged.py:57-581).

    The block table may end in -1 entries (blocks not yet owned); decode that
    crosses into a new block needs the grown table first (``update_block_table``).
    Nothing here allocates or frees native blocks.
    """

    def __init__(
        self,
        cache: torch.Tensor,
        block_table: Sequence[int] | torch.Tensor,
        prompt_length: int,
        max_selected: int,
        *,
        request_id: str = "",
        layer_index: int = 0,
        shared_slots: Iterable[int] = (),
        mover=None,
    ):
        layout_ok = (
            isinstance(cache, torch.Tensor)
            and cache.ndim == 4
            and min(cache.shape) >= 1
            and cache.shape[-1] % 2 == 0
            and cache.dtype in _FLOAT_TYPES
            and cache.device.type in ("cpu", "cuda")
        )
        if not layout_ok:
            raise ValueError("cache must be floating [blocks,KV heads,block size,2*D]")
        if mover is None:
            mover = _DEFAULT_MOVER
            _hip.require_device(cache)
        for name, number, least in (("prompt_length", prompt_length, 1),
                                    ("max_selected", max_selected, 0),
                                    ("layer_index", layer_index, 0)):
            if type(number) is not int or number < least:
                kind = "positive" if least else "nonnegative"
                raise ValueError(f"{name} must be a {kind} integer")
        self.cache = cache
        self.prompt_length = prompt_length
        self.request_id = request_id
        self.layer_index = layer_index
        self.max_selected = max_selected
        blocks, self.kv_heads, self.block_size, width = cache.shape
        self.head_dim = width // 2
        self.native_total_slots = blocks * self.block_size
        self._mover = mover
        self._mutex = threading.RLock()
        self._block_table = self._parse_table(block_table)
        self._canonical = {t: self._slot_in(self._block_table, t) for t in range(prompt_length)}
        self._canonical_slots = set(self._canonical.values())
        if len(self._canonical_slots) != prompt_length:
            raise ValueError("active logical blocks must name distinct native slots")
        self._shared = frozenset(shared_slots)
        self.slot_map = LayerSlotMap(
            self._canonical,
            shared_slots=self._shared,
            allocation_floor=self.native_total_slots,
            max_slots=self.native_total_slots + max_selected,
        )
        self._side: tuple[torch.Tensor, torch.Tensor] | None = None  # sidecar K, V
        self._baseline: set[int] = set()  # tokens whose baseline write has executed
        self._selected: set[int] = set()
        self._loads: list[Future] = []
        self._promotions: list[Future] = []
        self._decoded = False
        self._counts = {"hole_reuse": 0, "native_bind": 0, "mirror": 0, "ready_inplace": 0}

    # -- block table ------------------------------------------------------------
    def _parse_table(self, block_table) -> tuple[int, ...]:
        if isinstance(block_table, torch.Tensor):
            if block_table.ndim != 1 or block_table.dtype not in (torch.int32, torch.int64):
                raise ValueError("block_table must be a one-dimensional integer row")
            block_table = block_table.detach().cpu().tolist()
        row = tuple(block_table)
        blocks = self.cache.shape[0]
        if not row or not all(type(b) is int and -1 <= b < blocks for b in row):
            raise ValueError("block_table contains invalid native block IDs")
        return row

    def _slot_in(self, row: tuple[int, ...], token: int) -> int:
        index, offset = divmod(token, self.block_size)
        block = row[index] if index < len(row) else -1
        if block < 0:
            raise ValueError("logical token has no caller-owned native block")
        return block * self.block_size + offset

    def update_block_table(self, block_table: Sequence[int] | torch.Tensor) -> None:
        """Accept newly owned blocks; existing canonical slots must not move."""
        row = self._parse_table(block_table)
        with self._mutex:
            self.slot_map.snapshot()  # raises once the map is retired
            for token, slot in self._canonical.items():
                if self._slot_in(row, token) != slot:
                    raise ValueError("block-table update moved an existing native token")
            self._block_table = row

    def canonical_slot(self, token: int) -> int:
        if type(token) is not int or token < 0:
            raise ValueError("token must be a nonnegative integer")
        with self._mutex:
            self.slot_map.snapshot()
            return self._slot_in(self._block_table, token)

    # -- checks -------------------------------------------------------------------
    def _records(self, count: int, key: torch.Tensor, value: torch.Tensor) -> None:
        want = (count, self.kv_heads, self.head_dim)
        for tensor in (key, value):
            if not (isinstance(tensor, torch.Tensor) and tensor.shape == want
                    and tensor.device == self.cache.device and tensor.dtype == self.cache.dtype):
                raise ValueError("K/V must match cache device/dtype and [token,KV head,D]")

    def _settled_loads(self, *, pending_ok: bool = False) -> None:
        """Loads must have finished (or may still run when ``pending_ok``); a failed one raises."""
        for load in self._loads:
            if load.done():
                load.result()
            elif not pending_ok:
                raise RuntimeError("source KV load must complete before baseline/mirror writes")

    def _settled_promotions(self) -> None:
        for promotion in self._promotions:
            if not promotion.done():
                raise RuntimeError("selected writes must complete before updating them")
            promotion.result()

    # -- moving records -------------------------------------------------------------
    def _sidecar(self) -> tuple[torch.Tensor, torch.Tensor]:
        if self._side is None:
            shape = (self.max_selected, self.kv_heads, self.head_dim)
            self._side = (self.cache.new_empty(shape), self.cache.new_empty(shape))
        return self._side

    def _scatter(self, slots: list[int], key, value, rows: list[int] | None = None) -> None:
        """Enqueue rows of key/value (all, or ``rows``) into their slots, native or sidecar."""
        if not slots:
            return
        side_k, side_v = self._side if self._side is not None else (None, None)
        if max(slots) >= self.native_total_slots:
            side_k, side_v = self._sidecar()
        self._mover.scatter(self.cache, side_k, side_v, slots, key, value, rows)

    def _guarded_write(self, slots: list[int], key, value, *, mirrors=None) -> int:
        """Write under a write guard and wait for the device; a failure retires the map
        (the copies are not transactional).  ``mirrors`` = (candidate slots, rows):
        the ones the guard grants get a second copy.  Returns the mirror count."""
        slots_opt, rows_opt = mirrors if mirrors is not None else ((), ())
        with self.slot_map.write_guard(slots, optional_slots=slots_opt) as granted:
            take = [i for i, slot in enumerate(slots_opt) if slot in granted]
            try:
                self._scatter(slots, key, value)
                if take:
                    self._scatter([slots_opt[i] for i in take], key, value, [rows_opt[i] for i in take])
                _wait_device(self.cache.device)
            except BaseException:
                self.slot_map.invalidate()
                raise
        return len(take)

    # -- writes -------------------------------------------------------------------
    def write(self, logical_positions, key: torch.Tensor, value: torch.Tensor) -> None:
        """Baseline KV into the original native slots, whatever the redirection (paged.py:242-272)."""
        positions = _indices(logical_positions, "logical_positions")
        self._records(len(positions), key, value)
        with self._mutex:
            self.slot_map.snapshot()
            self._settled_loads()
            if self._decoded:
                raise RuntimeError("baseline writes cannot overwrite slots after decode")
            if not all(token in self._canonical for token in positions):
                raise KeyError("baseline writes require existing logical tokens")
            slots = [self._canonical[token] for token in positions]
            if not self._shared.isdisjoint(slots):
                raise ValueError("baseline writes cannot mutate shared native slots")
            self._guarded_write(slots, key, value)
            # only an executed device write (not a finished host read) makes the baseline ready
            self._baseline.update(positions)

    load_baseline = write

    def write_prefill(self, key: torch.Tensor, value: torch.Tensor) -> None:
        self.write(range(self.prompt_length), key, value)

    def promote_selected(self, logical_positions, key: torch.Tensor, value: torch.Tensor, *,
                         load_future: Future | None = None) -> Future:
        """Stage selected KV in fresh slots while the source load may still run;
        the new slots are published when the write has executed (paged.py:279-328)."""
        positions = _indices(logical_positions, "logical_positions")
        self._records(len(positions), key, value)
        if load_future is not None and not isinstance(load_future, Future):
            raise TypeError("load_future must be a concurrent Future")
        with self._mutex:
            if self._decoded:
                raise RuntimeError("selected promotion must precede decode")
            if not self._selected.isdisjoint(positions):
                raise ValueError("already staged tokens must use update_selected")
            if load_future is not None and load_future.done():
                load_future.result()

            def writer(runs: list[SlotWrite]) -> Future:
                # each 8-byte record is the source row of its slot
                slots = [slot for run in runs for slot in range(run.start_slot, run.start_slot + run.slot_count)]
                rows = np.frombuffer(b"".join(run.payload for run in runs), dtype="<i8").tolist()
                self._scatter(slots, key, value, rows)
                return _completion_future(self.cache.device)

            records = {token: row.to_bytes(8, "little") for row, token in enumerate(positions)}
            promotion = self.slot_map.promote_selected(records, writer, load_future=load_future,
                                                       allow_inplace=False)
            self._selected.update(positions)
            self._promotions.append(promotion)
            if load_future is not None and load_future not in self._loads:
                self._loads.append(load_future)
            return promotion

    stage_selected = promote_selected

    def write_selected_ready(self, logical_positions, key: torch.Tensor,
                             value: torch.Tensor) -> dict[int, int]:
        """Load-first branch: overwrite the original native slots, no sidecar and
        no holes; needs every baseline write executed (paged.py:332-374)."""
        positions = _indices(logical_positions, "logical_positions")
        self._records(len(positions), key, value)
        with self._mutex:
            current = self.slot_map.snapshot()
            self._settled_loads()
            self._settled_promotions()
            if self._decoded:
                raise RuntimeError("ready selected writes must precede decode")
            if len(self._baseline) != self.prompt_length:
                raise RuntimeError("native baseline device writes must complete first")
            if not all(token in self._canonical for token in positions):
                raise ValueError("ready selected tokens require original native slots")
            moved = any(current[token] != self._canonical[token] for token in positions)
            if moved or not self._selected.isdisjoint(positions):
                raise ValueError("already selected tokens must use update_selected")
            self._guarded_write([self._canonical[token] for token in positions], key, value)
            self._selected.update(positions)
            self._counts["ready_inplace"] += len(positions)
            return self.slot_map.snapshot()

    def update_selected(self, logical_positions, key: torch.Tensor, value: torch.Tensor) -> None:
        """Fused rows to their current slots, plus a mirror into the canonical slot
        wherever no reader pins it (paged.py:376-431)."""
        positions = _indices(logical_positions, "logical_positions")
        self._records(len(positions), key, value)
        with self._mutex:
            self._settled_loads()
            self._settled_promotions()
            if self._decoded:
                raise RuntimeError("selected updates must precede decode hole reuse")
            current = self.slot_map.snapshot()
            if not all(token in current for token in positions):
                raise ValueError("updated rows must already have logical mappings")
            slots = [current[token] for token in positions]
            if not self._shared.isdisjoint(slots):
                raise ValueError("updated rows cannot mutate shared native slots")
            mirror_slots, mirror_rows = [], []
            for row, token in enumerate(positions):
                home = self._canonical[token]
                if home != current[token] and home not in self._shared:
                    mirror_slots.append(home)
                    mirror_rows.append(row)
            self._counts["mirror"] += self._guarded_write(slots, key, value,
                                                          mirrors=(mirror_slots, mirror_rows))

    # -- reads -----------------------------------------------------------------------
    def gather(self, logical_positions) -> tuple[torch.Tensor, torch.Tensor]:
        """Logical K/V in caller order, read under pins of their slots (paged.py:433-472)."""
        positions = _indices(logical_positions, "logical_positions")
        with self._mutex, self.slot_map.pinned_mapping(positions) as current:
            self._settled_loads(pending_ok=True)
            shape = (len(positions), self.kv_heads, self.head_dim)
            key, value = self.cache.new_empty(shape), self.cache.new_empty(shape)
            if positions:
                side_k, side_v = self._side if self._side is not None else (None, None)
                self._mover.gather(self.cache, side_k, side_v, [current[t] for t in positions],
                                   key, value)
            _wait_device(self.cache.device)  # the pins hold until the reads have executed
            return key, value

    def logical_length(self) -> int:
        """Number of logical tokens (prompt plus decoded), i.e. the next decode token."""
        with self._mutex:
            return len(self._canonical)

    @contextmanager
    def device_slots(self, logical_positions):
        """The slots ``gather`` would read for the positions, for a kernel that
        reads the arena in place: yields (int64 device slots, sidecar K, sidecar V)
        -- the sidecar tensors are None before first use -- under pins of those
        slots, held until the reads enqueued inside the block have executed
        (the read half of paged.py:433-472)."""
        positions = _indices(logical_positions, "logical_positions")
        with self._mutex, self.slot_map.pinned_mapping(positions) as current:
            self._settled_loads(pending_ok=True)
            slots = torch.tensor([current[t] for t in positions], dtype=torch.long,
                                 device=self.cache.device)
            side_k, side_v = self._side if self._side is not None else (None, None)
            try:
                yield slots, side_k, side_v
            finally:
                _wait_device(self.cache.device)  # the pins hold until the reads have executed

    def decode(self, token: int, key: torch.Tensor, value: torch.Tensor,
               canonical_slot: int | None = None) -> int:
        """Append one token: the lowest eligible native hole, else the canonical
        slot; a hole write is mirrored into the canonical slot too (paged.py:474-524)."""
        if type(token) is not int or token < 0:
            raise ValueError("decode token must be a nonnegative integer")
        key = key.unsqueeze(0) if key.ndim == 2 else key
        value = value.unsqueeze(0) if value.ndim == 2 else value
        self._records(1, key, value)
        with self._mutex:
            self._settled_loads(pending_ok=True)
            self._settled_promotions()
            if token != len(self._canonical):
                raise ValueError("decode must append the next logical token")
            owned = self._slot_in(self._block_table, token)
            home = owned if canonical_slot is None else canonical_slot
            if type(home) is not int or home != owned:
                raise ValueError("decode canonical slot is not owned by its block table")
            if home in self._canonical_slots:
                raise ValueError("decode native slot aliases an existing canonical token")
            with self.slot_map.decode_write_guard(token, home, reuse_vacated=True) as chosen:
                targets = [chosen] if chosen == home else [chosen, home]
                self._scatter(targets, key, value, [0] * len(targets))
                _wait_device(self.cache.device)
            reused = chosen != home
            self._counts["hole_reuse"] += reused
            self._counts["mirror"] += reused
            self._counts["native_bind"] += not reused
            self._canonical[token] = home
            self._canonical_slots.add(home)
            self._decoded = True
            return chosen

    def snapshot(self) -> dict[int, int]:
        with self._mutex:
            return self.slot_map.snapshot()

    def page_metadata(self) -> tuple[dict[str, int | bool], ...]:
        """Mapped physical pages with their selected-token counts and guards."""
        with self._mutex:
            return self.slot_map.page_metadata(self.block_size, self._selected)

    def spill_order(self) -> tuple[int, ...]:
        """Advisory order of spillable pages: clean first, then most selected tokens
        first, then page id (paged.py:540-559); guarded pages are left out."""
        pages = [page for page in self.page_metadata() if page["spill_eligible"]]
        pages.sort(key=lambda page: (page["dirty"], -page["selected_count"], page["page_id"]))
        return tuple(page["page_id"] for page in pages)

    def stats(self) -> dict[str, int]:
        with self._mutex:
            return {
                **self.slot_map.stats(),
                "physical_hole_reuse": self._counts["hole_reuse"],
                "decode_native_bind": self._counts["native_bind"],
                "canonical_mirror_writes": self._counts["mirror"],
                "sidecar_capacity_slots": self.max_selected,
                "sidecar_allocated_slots": self.max_selected if self._side is not None else 0,
                "selected_ready_inplace_writes": self._counts["ready_inplace"],
                "native_pool_capacity_slots": self.native_total_slots,
                "native_pool_capacity_blocks": self.cache.shape[0],
                "native_pool_capacity_delta": 0,
                "native_pool_blocks_released": 0,
            }

    def invalidate(self) -> None:
        with self._mutex:
            self.slot_map.invalidate()
