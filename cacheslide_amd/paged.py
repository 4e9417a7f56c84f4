"""Request-local SLIDE indirection over the packed paged KV cache.

Counterpart of src/cacheslide_vllm/paged.py:21-581.  The native cache is
[block, KV head, block offset, 2 * head dimension]; only slots named by the
caller's block table are written; selected KV beyond the native pool goes to
a bounded sidecar.  Host metadata (slot maps, guards, futures, statistics)
follows the reference exactly; the bytes move through the slot kernels
(cs_slot_scatter / cs_slot_gather), which accept arbitrary strides and are
bit-exact for every dtype.

``mover`` selects who moves the bytes.  The default is the HIP library and
requires device tensors; a test may inject another mover object with the same
two methods to exercise the host logic without a GPU.
"""

from __future__ import annotations

import threading
from collections.abc import Iterable, Sequence
from concurrent.futures import Future

import torch

from . import _hip
from ._hip import call, ptr, vref
from .slide import LayerSlotMap, SlotWrite


def _indices(value: Sequence[int] | torch.Tensor, name: str) -> list[int]:
    if isinstance(value, torch.Tensor):
        if value.ndim != 1 or value.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"{name} must be an integer vector")
        value = value.detach().cpu().tolist()  # token metadata only; KV stays on device
    result = list(value)
    if any(type(item) is not int or item < 0 for item in result):
        raise ValueError(f"{name} must contain nonnegative integer positions")
    if len(set(result)) != len(result):
        raise ValueError(f"{name} must contain distinct positions")
    return result


def _completion_future(device: torch.device) -> Future:
    """Device completion (an event on the current stream), not host enqueue, publishes."""
    completed: Future = Future()
    completed.set_running_or_notify_cancel()
    if device.type != "cuda":
        completed.set_result(None)
        return completed
    event = torch.cuda.Event()
    event.record(torch.cuda.current_stream(device))

    def finish() -> None:
        try:
            event.synchronize()
        except BaseException as error:
            completed.set_exception(error)
        else:
            completed.set_result(None)

    threading.Thread(target=finish, name="cacheslide-kv-write", daemon=True).start()
    return completed


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


class NativePagedKV:
    """One request/layer's native slots plus a selected-token sidecar (paged.py:57-581)."""

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
        if (
            not isinstance(cache, torch.Tensor)
            or cache.ndim != 4
            or min(cache.shape) < 1
            or cache.shape[-1] % 2
            or cache.dtype not in (torch.float16, torch.bfloat16, torch.float32, torch.float64)
            or cache.device.type not in ("cpu", "cuda")
        ):
            raise ValueError("cache must be floating [blocks,KV heads,block size,2*D]")
        if mover is None:
            mover = _DEFAULT_MOVER
            _hip.require_device(cache)
        if type(prompt_length) is not int or prompt_length < 1:
            raise ValueError("prompt_length must be a positive integer")
        if type(max_selected) is not int or max_selected < 0:
            raise ValueError("max_selected must be a nonnegative integer")
        if type(layer_index) is not int or layer_index < 0:
            raise ValueError("layer_index must be a nonnegative integer")
        self.cache = cache
        self._mover = mover
        self.prompt_length = prompt_length
        self.request_id = request_id
        self.layer_index = layer_index
        self.block_size = cache.shape[2]
        self.kv_heads = cache.shape[1]
        self.head_dim = cache.shape[3] // 2
        self.native_total_slots = cache.shape[0] * self.block_size
        self.max_selected = max_selected
        self._mutex = threading.RLock()
        self._block_table = self._table(block_table)
        self._canonical = {token: self._canonical_slot(token) for token in range(prompt_length)}
        if len(set(self._canonical.values())) != prompt_length:
            raise ValueError("active logical blocks must name distinct native slots")
        self._shared = set(shared_slots)
        self.slot_map = LayerSlotMap(
            self._canonical,
            shared_slots=self._shared,
            allocation_floor=self.native_total_slots,
            max_slots=self.native_total_slots + max_selected,
        )
        self._side_key: torch.Tensor | None = None
        self._side_value: torch.Tensor | None = None
        self._baseline_ready: set[int] = set()
        self._loads: list[Future] = []
        self._promotions: list[Future] = []
        self._selected: set[int] = set()
        self._decoded = False
        self._hole_reuses = 0
        self._native_binds = 0
        self._canonical_mirrors = 0
        self._ready_inplace_writes = 0

    # -- block table ------------------------------------------------------------
    def _table(self, block_table) -> tuple[int, ...]:
        if isinstance(block_table, torch.Tensor):
            if block_table.ndim != 1 or block_table.dtype not in (torch.int32, torch.int64):
                raise ValueError("block_table must be a one-dimensional integer row")
            block_table = block_table.detach().cpu().tolist()
        row = tuple(block_table)
        if not row or any(
            type(block) is not int or not -1 <= block < self.cache.shape[0] for block in row
        ):
            raise ValueError("block_table contains invalid native block IDs")
        return row

    def _canonical_slot(self, token: int, row: tuple[int, ...] | None = None) -> int:
        row = self._block_table if row is None else row
        block_index, offset = divmod(token, self.block_size)
        if block_index >= len(row) or row[block_index] < 0:
            raise ValueError("logical token has no caller-owned native block")
        return row[block_index] * self.block_size + offset

    def update_block_table(self, block_table: Sequence[int] | torch.Tensor) -> None:
        """Accept newly owned blocks without moving existing canonical slots."""
        row = self._table(block_table)
        with self._mutex:
            self.slot_map.snapshot()
            if any(self._canonical_slot(t, row) != s for t, s in self._canonical.items()):
                raise ValueError("block-table update moved an existing native token")
            self._block_table = row

    def canonical_slot(self, token: int) -> int:
        if type(token) is not int or token < 0:
            raise ValueError("token must be a nonnegative integer")
        with self._mutex:
            self.slot_map.snapshot()
            return self._canonical_slot(token)

    # -- records ------------------------------------------------------------------
    def _records(self, positions: list[int], key: torch.Tensor, value: torch.Tensor):
        expected = (len(positions), self.kv_heads, self.head_dim)
        for tensor in (key, value):
            if (
                not isinstance(tensor, torch.Tensor)
                or tensor.shape != expected
                or tensor.device != self.cache.device
                or tensor.dtype != self.cache.dtype
            ):
                raise ValueError("K/V must match cache device/dtype and [token,KV head,D]")
        return key, value

    def _check_loads(self, *, allow_pending: bool = False) -> None:
        for loading in self._loads:
            if not loading.done():
                if allow_pending:
                    continue
                raise RuntimeError("source KV load must complete before baseline/mirror writes")
            loading.result()

    def _check_promotions(self) -> None:
        for promotion in self._promotions:
            if not promotion.done():
                raise RuntimeError("selected writes must complete before updating them")
            promotion.result()

    def _ensure_sidecar(self) -> None:
        if self._side_key is None:
            shape = (self.max_selected, self.kv_heads, self.head_dim)
            self._side_key = self.cache.new_empty(shape)
            self._side_value = self.cache.new_empty(shape)

    def _write_slots(self, slots: list[int], key: torch.Tensor, value: torch.Tensor,
                     rows: list[int] | None = None) -> None:
        """Scatter rows of key/value into their slots (native or sidecar)."""
        if any(s >= self.native_total_slots for s in slots):
            self._ensure_sidecar()
        self._mover.scatter(self.cache, self._side_key, self._side_value, slots, key, value, rows)

    # -- writes -------------------------------------------------------------------
    def write(self, logical_positions, key: torch.Tensor, value: torch.Tensor) -> None:
        """Load baseline KV into the original native slots (paged.py:242-272)."""
        positions = _indices(logical_positions, "logical_positions")
        self._records(positions, key, value)
        with self._mutex:
            self.slot_map.snapshot()
            self._check_loads()
            if self._decoded:
                raise RuntimeError("baseline writes cannot overwrite slots after decode")
            if any(token not in self._canonical for token in positions):
                raise KeyError("baseline writes require existing logical tokens")
            slots = [self._canonical[token] for token in positions]
            if self._shared.intersection(slots):
                raise ValueError("baseline writes cannot mutate shared native slots")
            with self.slot_map.write_guard(slots):
                try:
                    self._write_slots(slots, key, value)
                    _completion_future(self.cache.device).result()
                except BaseException:
                    self.slot_map.invalidate()
                    raise
            self._baseline_ready.update(positions)

    load_baseline = write

    def write_prefill(self, key: torch.Tensor, value: torch.Tensor) -> None:
        self.write(range(self.prompt_length), key, value)

    def promote_selected(self, logical_positions, key: torch.Tensor, value: torch.Tensor, *,
                         load_future: Future | None = None) -> Future:
        """Stage selected KV in fresh slots while a source load is outstanding (paged.py:279-328)."""
        positions = _indices(logical_positions, "logical_positions")
        self._records(positions, key, value)
        if load_future is not None and not isinstance(load_future, Future):
            raise TypeError("load_future must be a concurrent Future")
        with self._mutex:
            if self._decoded:
                raise RuntimeError("selected promotion must precede decode")
            if self._selected.intersection(positions):
                raise ValueError("already staged tokens must use update_selected")
            if load_future is not None and load_future.done():
                load_future.result()

            def writer(runs: list[SlotWrite]) -> Future:
                slots, rows = [], []
                for run in runs:
                    for i in range(run.slot_count):
                        slots.append(run.start_slot + i)
                        rows.append(int.from_bytes(run.payload[8 * i : 8 * i + 8], "little"))
                self._write_slots(slots, key, value, rows)
                return _completion_future(self.cache.device)

            # payloads carry row numbers; KV stays on the device
            updates = {token: row.to_bytes(8, "little") for row, token in enumerate(positions)}
            promotion = self.slot_map.promote_selected(
                updates, writer, load_future=load_future, allow_inplace=False
            )
            self._selected.update(positions)
            self._promotions.append(promotion)
            if load_future is not None and load_future not in self._loads:
                self._loads.append(load_future)
            return promotion

    stage_selected = promote_selected

    def write_selected_ready(self, logical_positions, key: torch.Tensor,
                             value: torch.Tensor) -> dict[int, int]:
        """Load-first branch: overwrite the original slots in place (paged.py:332-374)."""
        positions = _indices(logical_positions, "logical_positions")
        self._records(positions, key, value)
        with self._mutex:
            mapping = self.slot_map.snapshot()
            self._check_loads()
            self._check_promotions()
            if self._decoded:
                raise RuntimeError("ready selected writes must precede decode")
            if len(self._baseline_ready) != self.prompt_length:
                raise RuntimeError("native baseline device writes must complete first")
            if not set(positions) <= set(self._canonical):
                raise ValueError("ready selected tokens require original native slots")
            if self._selected.intersection(positions) or any(
                mapping[t] != self._canonical[t] for t in positions
            ):
                raise ValueError("already selected tokens must use update_selected")
            slots = [self._canonical[t] for t in positions]
            with self.slot_map.write_guard(slots):
                try:
                    self._write_slots(slots, key, value)
                    _completion_future(self.cache.device).result()
                except BaseException:
                    self.slot_map.invalidate()
                    raise
            self._selected.update(positions)
            self._ready_inplace_writes += len(positions)
            return self.slot_map.snapshot()

    def update_selected(self, logical_positions, key: torch.Tensor, value: torch.Tensor) -> None:
        """Write fused rows to their current slots and mirror them canonically (paged.py:376-431)."""
        positions = _indices(logical_positions, "logical_positions")
        self._records(positions, key, value)
        with self._mutex:
            self._check_loads()
            self._check_promotions()
            if self._decoded:
                raise RuntimeError("selected updates must precede decode hole reuse")
            mapping = self.slot_map.snapshot()
            if not set(positions) <= set(mapping):
                raise ValueError("updated rows must already have logical mappings")
            if any(mapping[t] in self._shared for t in positions):
                raise ValueError("updated rows cannot mutate shared native slots")
            candidates = [
                row
                for row, t in enumerate(positions)
                if self._canonical[t] not in self._shared and self._canonical[t] != mapping[t]
            ]
            slots = [mapping[t] for t in positions]
            with self.slot_map.write_guard(
                slots, optional_slots=[self._canonical[positions[r]] for r in candidates]
            ) as writable:
                mirror_rows = [r for r in candidates if self._canonical[positions[r]] in writable]
                try:
                    self._write_slots(slots, key, value)
                    if mirror_rows:
                        self._write_slots(
                            [self._canonical[positions[r]] for r in mirror_rows], key, value,
                            mirror_rows,
                        )
                    _completion_future(self.cache.device).result()
                except BaseException:
                    self.slot_map.invalidate()
                    raise
                self._canonical_mirrors += len(mirror_rows)

    # -- reads -----------------------------------------------------------------------
    def gather(self, logical_positions) -> tuple[torch.Tensor, torch.Tensor]:
        """Logical K/V in caller order, under atomic mapping pins (paged.py:433-472)."""
        positions = _indices(logical_positions, "logical_positions")
        with self._mutex, self.slot_map.pinned_mapping(positions) as mapping:
            self._check_loads(allow_pending=True)
            shape = (len(positions), self.kv_heads, self.head_dim)
            key, value = self.cache.new_empty(shape), self.cache.new_empty(shape)
            slots = [mapping[t] for t in positions]
            if slots:
                self._mover.gather(self.cache, self._side_key, self._side_value, slots, key, value)
            _completion_future(self.cache.device).result()
            return key, value

    def decode(self, token: int, key: torch.Tensor, value: torch.Tensor,
               canonical_slot: int | None = None) -> int:
        """Reuse an eligible native hole, else bind the canonical slot (paged.py:474-524)."""
        if type(token) is not int or token < 0:
            raise ValueError("decode token must be a nonnegative integer")
        if key.ndim == 2:
            key = key.unsqueeze(0)
        if value.ndim == 2:
            value = value.unsqueeze(0)
        self._records([token], key, value)
        with self._mutex:
            self._check_loads(allow_pending=True)
            self._check_promotions()
            if token != len(self._canonical):
                raise ValueError("decode must append the next logical token")
            expected = self._canonical_slot(token)
            if canonical_slot is None:
                canonical_slot = expected
            if type(canonical_slot) is not int or canonical_slot != expected:
                raise ValueError("decode canonical slot is not owned by its block table")
            if canonical_slot in self._canonical.values():
                raise ValueError("decode native slot aliases an existing canonical token")
            with self.slot_map.decode_write_guard(token, canonical_slot, reuse_vacated=True) as chosen:
                self._write_slots([chosen], key, value)
                if chosen != canonical_slot:
                    self._write_slots([canonical_slot], key, value)
                _completion_future(self.cache.device).result()
            reused = chosen != canonical_slot
            self._hole_reuses += int(reused)
            self._canonical_mirrors += int(reused)
            self._native_binds += int(not reused)
            self._canonical[token] = canonical_slot
            self._decoded = True
            return chosen

    def snapshot(self) -> dict[int, int]:
        with self._mutex:
            return self.slot_map.snapshot()

    def page_metadata(self) -> tuple[dict[str, int | bool], ...]:
        with self._mutex:
            return self.slot_map.page_metadata(self.block_size, self._selected)

    def spill_order(self) -> tuple[int, ...]:
        """Clean pages first, then by descending selected count (paged.py:540-559)."""
        eligible = [page for page in self.page_metadata() if page["spill_eligible"]]
        eligible.sort(key=lambda page: (page["dirty"], -page["selected_count"], page["page_id"]))
        return tuple(page["page_id"] for page in eligible)

    def stats(self) -> dict[str, int]:
        with self._mutex:
            return {
                **self.slot_map.stats(),
                "physical_hole_reuse": self._hole_reuses,
                "decode_native_bind": self._native_binds,
                "canonical_mirror_writes": self._canonical_mirrors,
                "sidecar_capacity_slots": self.max_selected,
                "sidecar_allocated_slots": self.max_selected if self._side_key is not None else 0,
                "selected_ready_inplace_writes": self._ready_inplace_writes,
                "native_pool_capacity_slots": self.native_total_slots,
                "native_pool_capacity_blocks": self.cache.shape[0],
                "native_pool_capacity_delta": 0,
                "native_pool_blocks_released": 0,
            }

    def invalidate(self) -> None:
        with self._mutex:
            self.slot_map.invalidate()
