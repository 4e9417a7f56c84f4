"""Row bookkeeping of the selective prefill (src/cacheslide_vllm/runtime.py:397-456).

``CacheSlideRuntime._prefill`` runs each layer on the rows of the tokens WCA
keeps active.  Between layers it carries the rows that continue, restores the
newly active ones from the layer's input snapshot of the fixed tokens, and
at the end places the last layer's rows into a zero-filled ``[n, H]`` output.
It does this with two length-n lookup tables, boolean-mask indexing and
``.item()`` reads (host syncs).  These functions do the same on the device
with one kernel each (``libcacheslide_hip`` ``cs_rows_*``):

* ``next_layer_rows`` -- runtime.py:408-432.  Continuing rows, restored rows,
  the restored-row count, and ``ReuseFailure("a mandatory dynamic row was
  lost")``.  With ``check=False`` nothing is read back; ``LayerRows.check()``
  raises later, e.g. once per forward.
* ``gather_rows`` -- the ``hidden[fixed]`` / ``residual[fixed]`` snapshots
  (runtime.py:420-431).
* ``scatter_rows`` -- ``output = zeros(n, H); output[previous] = hidden``
  (runtime.py:454-456).

Token lists are int64 and ascending and distinct, as the runtime's are (WCA
active indices, the plan's fixed indices).  The kernels check this and raise
ValueError otherwise.  Rows move bit for bit.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _hip
from ._hip import call, index_tensor, new_flags, ptr, read_flags, require_device, stream_of, vref


class ReuseFailure(RuntimeError):
    """Reuse cannot continue; the runtime falls back to full recomputation (runtime.py:34)."""


def _raise_row_flags(bits: int) -> None:
    if bits & _hip.FLAG_ROWS_UNSORTED:
        raise ValueError("row token lists must be ascending and distinct")
    if bits & _hip.FLAG_ROW_INDEX:
        raise ValueError("row index outside the source rows")
    if bits & _hip.FLAG_ROW_LOST:
        raise ReuseFailure("a mandatory dynamic row was lost")


def _rows_operand(x: Tensor, name: str) -> Tensor:
    if x.ndim != 2:
        raise ValueError(f"{name} must be [rows, H]")
    return x if x.stride(1) == 1 or x.shape[1] <= 1 else x.contiguous()


@dataclass
class LayerRows:
    """The next layer's rows plus the device-side restored count and flags."""

    hidden: Tensor
    residual: Tensor | None
    restored: Tensor  # int64 [1], rows restored from the snapshot
    flags: Tensor  # int32 [1]

    def check(self) -> int:
        """One readback: raise the recorded failure, else return the restored count."""
        bits = read_flags(self.flags)[0]
        _raise_row_flags(bits)
        return int(self.restored.item())


def next_layer_rows(
    hidden: Tensor,
    residual: Tensor | None,
    previous: Tensor,
    active: Tensor,
    fixed: Tensor,
    snapshot: Mapping[str, Tensor] | None = None,
    *,
    read_snapshot: Callable[[], Mapping[str, Tensor]] | None = None,
    check: bool = True,
) -> LayerRows:
    """Rows of the tokens ``active`` for the next layer (runtime.py:408-432).

    ``hidden``/``residual`` hold the rows of ``previous``, in its order.  A
    token of ``active`` not in ``previous`` is restored from ``snapshot``
    (``{"hidden", "residual"}`` rows of ``fixed``, in its order).  When only
    ``read_snapshot`` is given it is called, as in the reference, only if
    some row needs restoring (one count readback decides).
    """
    device = require_device(hidden, residual)
    hidden = _rows_operand(hidden, "hidden")
    residual = None if residual is None else _rows_operand(residual, "residual")
    previous = index_tensor(previous, device, "previous")
    active = index_tensor(active, device, "active")
    fixed = index_tensor(fixed, device, "fixed")
    stream = stream_of(device)
    if snapshot is None and read_snapshot is not None:
        missing = torch.zeros(1, dtype=torch.long, device=device)
        call("cs_rows_missing", ptr(previous), len(previous), ptr(active), len(active), ptr(missing), stream)
        if int(missing.item()):
            snapshot = read_snapshot()
    snap_h = snap_r = None
    if snapshot is not None:
        snap_h = _rows_operand(snapshot["hidden"], "snapshot hidden")
        require_device(snap_h)
        if residual is not None:
            snap_r = _rows_operand(snapshot["residual"], "snapshot residual")
            require_device(snap_r)
    for name, x in (("residual", residual), ("snapshot hidden", snap_h), ("snapshot residual", snap_r)):
        if x is not None and x.dtype != hidden.dtype:
            raise ValueError(f"{name} dtype differs from hidden")
    out_h = hidden.new_empty((len(active), hidden.shape[1]))
    out_r = None if residual is None else torch.empty_like(out_h)
    restored = torch.zeros(1, dtype=torch.long, device=device)
    flags = new_flags(device)
    call("cs_rows_remap", vref(hidden), vref(residual), vref(snap_h), vref(snap_r), vref(out_h), vref(out_r),
         ptr(previous), len(previous), ptr(active), len(active), ptr(fixed), len(fixed), ptr(restored),
         ptr(flags), stream)
    rows = LayerRows(out_h, out_r, restored, flags)
    if check:
        rows.check()
    return rows


def gather_rows(x: Tensor, index: Tensor) -> Tensor:
    """``x[index]`` for row snapshots (runtime.py:420-431)."""
    device = require_device(x)
    x = _rows_operand(x, "rows")
    index = index_tensor(index, device, "index")
    out = x.new_empty((len(index), x.shape[1]))
    flags = new_flags(device)
    call("cs_rows_gather", vref(x), ptr(index), len(index), vref(out), ptr(flags), stream_of(device))
    _raise_row_flags(read_flags(flags)[0])
    return out


def scatter_rows(rows: Tensor, tokens: Tensor, n: int) -> Tensor:
    """``output = zeros(n, H); output[tokens] = rows`` (runtime.py:454-456)."""
    device = require_device(rows)
    rows = _rows_operand(rows, "rows")
    tokens = index_tensor(tokens, device, "tokens")
    if len(tokens) != rows.shape[0]:
        raise ValueError("one row per token is required")
    out = rows.new_empty((n, rows.shape[1]))
    flags = new_flags(device)
    call("cs_rows_scatter", vref(rows), ptr(tokens), len(tokens), vref(out), ptr(flags), stream_of(device))
    _raise_row_flags(read_flags(flags)[0])
    return out
