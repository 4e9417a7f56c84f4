"""CPU oracle for SLIDE slot moves (test infrastructure only).

Byte-level restatement of src/cacheslide_vllm/paged.py:205-240 (scatter into
native slots / sidecar) and :433-472 (gather), of the relocation of whole
pages and single token records, and of the lowest-first free-slot order of
src/cacheslide_vllm/slide.py:103-112.  Arrays hold raw element bits (e.g.
uint16 for bf16), so every comparison is bit-exact.
"""

from __future__ import annotations

import numpy as np


def slot_scatter(cache, side_k, side_v, slots, key, value, rows=None) -> None:
    """cache [B, H, bs, 2D]; slot s < B*bs -> (s // bs, s % bs), else sidecar row s - B*bs."""
    blocks, _, bs, two_d = cache.shape
    d = two_d // 2
    native = blocks * bs
    for i, s in enumerate(slots):
        r = i if rows is None else rows[i]
        if s < native:
            cache[s // bs, :, s % bs, :d] = key[r]
            cache[s // bs, :, s % bs, d:] = value[r]
        else:
            side_k[s - native] = key[r]
            side_v[s - native] = value[r]


def slot_gather(cache, side_k, side_v, slots):
    blocks, heads, bs, two_d = cache.shape
    d = two_d // 2
    native = blocks * bs
    key = np.empty((len(slots), heads, d), dtype=cache.dtype)
    value = np.empty_like(key)
    for i, s in enumerate(slots):
        if s < native:
            key[i] = cache[s // bs, :, s % bs, :d]
            value[i] = cache[s // bs, :, s % bs, d:]
        else:
            key[i] = side_k[s - native]
            value[i] = side_v[s - native]
    return key, value


def slot_copy(cache, src, dst) -> None:
    """Stacked cache [L, B, H, bs, 2D]: copy token records src[i] -> dst[i] (all layers)."""
    bs = cache.shape[3]
    snapshot = cache.copy()
    for s, t in zip(src, dst):
        cache[:, t // bs, :, t % bs, :] = snapshot[:, s // bs, :, s % bs, :]


def page_copy(cache, src_blocks, dst_blocks) -> None:
    snapshot = cache.copy()
    for s, t in zip(src_blocks, dst_blocks):
        cache[:, t] = snapshot[:, s]


def acquire_lowest(free: np.ndarray, count: int):
    """Take the `count` lowest free slots (ascending), or None if too few."""
    idx = np.flatnonzero(free)
    if idx.size < count:
        return None
    taken = idx[:count]
    free[taken] = False
    return taken


def fresh_slot_sequence(unused: set[int], next_slot: int, count: int, max_slots=None):
    """Successive LayerSlotMap._fresh_slot results: min(unused) first, then next++."""
    pool = set(unused)
    out = []
    for _ in range(count):
        if pool:
            s = min(pool)
            pool.discard(s)
        else:
            if max_slots is not None and next_slot >= max_slots:
                raise RuntimeError("sidecar slot arena is full")
            s = next_slot
            next_slot += 1
        out.append(s)
    return out
