"""CPU oracle for the selective prefill's row bookkeeping (test infrastructure only).

numpy restatement of src/cacheslide_vllm/runtime.py:408-432 (next layer's
hidden/residual rows: continuing rows through a length-n lookup table, newly
active rows restored from the fixed-token snapshot, a row in neither raises),
:420-431 (hidden[fixed] snapshots) and :454-456 (zero-filled [n, H] output with
the last layer's rows at their tokens).  The reference's own lookup-table form
is kept: it needs no ordering of the token lists, which is what the checks in
tests/test_oracle.py use to pin the kernels' binary searches.
"""

from __future__ import annotations

import numpy as np


class RowLost(Exception):
    """runtime.py:423-424: "a mandatory dynamic row was lost"."""


def next_layer_rows(hidden, residual, previous, active, fixed, snap_hidden, snap_residual, n):
    """(hidden', residual', restored rows) for the tokens `active` (runtime.py:408-432)."""
    previous, active, fixed = (np.asarray(x, dtype=np.int64) for x in (previous, active, fixed))
    lookup = np.full(n, -1, dtype=np.int64)
    lookup[previous] = np.arange(len(previous))
    rows = lookup[active]
    continuing = rows >= 0
    out_h = np.empty((len(active), hidden.shape[1]), dtype=hidden.dtype)
    out_h[continuing] = hidden[rows[continuing]]
    out_r = None
    if residual is not None:
        out_r = np.empty_like(out_h)
        out_r[continuing] = residual[rows[continuing]]
    if not continuing.all():
        ordinal = np.full(n, -1, dtype=np.int64)
        ordinal[fixed] = np.arange(len(fixed))
        restored = ordinal[active[~continuing]]
        if (restored < 0).any():
            raise RowLost("a mandatory dynamic row was lost")
        out_h[~continuing] = snap_hidden[restored]
        if out_r is not None:
            out_r[~continuing] = snap_residual[restored]
    return out_h, out_r, int((~continuing).sum())


def scatter_rows(rows, tokens, n):
    """runtime.py:454-456: zeros [n, H] with rows at their tokens."""
    out = np.zeros((n, rows.shape[1]), dtype=rows.dtype)
    out[np.asarray(tokens, dtype=np.int64)] = rows
    return out


def gather_rows(x, idx):
    """runtime.py:420-431: x[idx]."""
    return x[np.asarray(idx, dtype=np.int64)]
