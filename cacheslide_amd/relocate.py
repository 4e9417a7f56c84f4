"""Batched SLIDE relocation on a stacked paged cache.

A relocation step moves reused chunks to new slots: copy whole pages (and
single token records for partial pages), rewrite the token -> slot map, and
return the source slots to the free pool.  The per-request reference path
does the same one arena at a time (src/cacheslide_vllm/slide.py:243-372 with
paged.py:205-240); these entry points run it for every layer and chunk of a
step in a handful of launches.  All moves are byte copies (bit-exact).

Cache views are [L, blocks, H, bs, 2D] (or a single layer [blocks, H, bs, 2D]).
Sources and destinations of one call must be disjoint (checked unless the
caller passes ``check=False``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _hip
from ._hip import call, ptr, vref
from .errors import CacheCapacityError


def _long(t: Tensor, device) -> Tensor:
    if t.device != device or t.dtype != torch.long or not t.is_contiguous():
        raise ValueError("index tensors must be contiguous int64 on the cache device")
    return t


def _disjoint(src: Tensor, dst: Tensor, what: str) -> None:
    """Sources and destinations of one launch must be disjoint and the
    destinations distinct: the moves run concurrently, so an overlap races."""
    if src.numel() == 0:
        return
    if bool(torch.isin(dst, src).any()) or torch.unique(dst).numel() != dst.numel():
        raise ValueError(f"{what}: destinations must be distinct and disjoint from the sources")


def copy_pages(cache: Tensor, src_blocks: Tensor, dst_blocks: Tensor, *, check: bool = True) -> None:
    """cache[..., dst_blocks[i], :, :, :] = cache[..., src_blocks[i], :, :, :] for every layer.

    With ``check`` the index vectors are checked for overlap first (one
    readback); callers that build them from disjoint pools may skip it.
    """
    device = _hip.require_device(cache)
    if src_blocks.shape != dst_blocks.shape or src_blocks.ndim != 1:
        raise ValueError("src_blocks and dst_blocks must be matching vectors")
    src, dst = _long(src_blocks, device), _long(dst_blocks, device)
    if check:
        _disjoint(src, dst, "copy_pages")
    call("cs_page_copy", vref(cache), ptr(src), ptr(dst), src.numel(), _hip.stream_of(device))


def copy_slots(cache: Tensor, src_slots: Tensor, dst_slots: Tensor, *, check: bool = True) -> None:
    """Copy token records (all layers, heads, K and V) from src_slots[i] to dst_slots[i]."""
    device = _hip.require_device(cache)
    if src_slots.shape != dst_slots.shape or src_slots.ndim != 1:
        raise ValueError("src_slots and dst_slots must be matching vectors")
    src, dst = _long(src_slots, device), _long(dst_slots, device)
    if check:
        _disjoint(src, dst, "copy_slots")
    call("cs_slot_copy", vref(cache), ptr(src), ptr(dst), src.numel(), _hip.stream_of(device))


def scatter_mapping(mapping: Tensor, tokens: Tensor, slots: Tensor) -> None:
    """mapping[tokens[i]] = slots[i] (tokens outside the map are ignored)."""
    device = _hip.require_device(mapping)
    if tokens.numel() != slots.numel():
        raise ValueError("tokens and slots must have the same length")
    call("cs_mapping_scatter", ptr(_long(mapping, device)), mapping.numel(),
         ptr(_long(tokens, device)), ptr(_long(slots, device)), tokens.numel(),
         _hip.stream_of(device))


def gather_mapping(mapping: Tensor, tokens: Tensor) -> Tensor:
    """mapping[tokens[i]] (-1 for tokens outside the map)."""
    device = _hip.require_device(mapping)
    out = torch.empty(tokens.numel(), dtype=torch.long, device=device)
    call("cs_mapping_gather", ptr(_long(mapping, device)), mapping.numel(),
         ptr(_long(tokens, device)), ptr(out), tokens.numel(), _hip.stream_of(device))
    return out


class SlotFreeList:
    """Device bitmap of free slots with lowest-first allocation.

    ``acquire`` hands out the lowest free slots in ascending order, which is the
    order of LayerSlotMap._fresh_slot (min of the returned pool, then the next
    never-used slot) when the never-used tail is marked free.
    """

    def __init__(self, nbits: int, device, *, free_from: int = 0):
        if nbits < 0 or not 0 <= free_from <= nbits:
            raise ValueError("invalid free-list size")
        self.nbits = nbits
        self.device = torch.device(device)
        words = (nbits + 31) // 32
        bits = torch.zeros(max(words, 1), dtype=torch.int64)
        for w in range(words):
            lo, hi = 32 * w, min(32 * w + 32, nbits)
            a, b = max(lo, free_from), hi
            if a < b:
                mask = ((1 << (b - a)) - 1) << (a - lo)
                bits[w] = mask
        self.bitmap = _pack_words(bits, self.device)
        self._status = torch.zeros(1, dtype=torch.int32, device=self.device)

    def release(self, slots: Tensor) -> None:
        if slots.ndim != 1:
            raise ValueError("slots must be a vector")
        call("cs_freelist_release", ptr(self.bitmap), self.nbits, ptr(_long(slots, self.device)),
             slots.numel(), _hip.stream_of(self.device))

    def acquire(self, count: int, out: Tensor | None = None, *, check: bool = True) -> Tensor:
        if type(count) is not int or count < 0:
            raise ValueError("count must be a nonnegative integer")
        if out is None:
            out = torch.empty(max(count, 1), dtype=torch.long, device=self.device)
        else:
            out = _long(out, self.device)
            if out.numel() < count:
                raise ValueError(f"out holds {out.numel()} slots, acquire needs {count}")
        call("cs_freelist_acquire", ptr(self.bitmap), self.nbits, count, ptr(out), ptr(self._status),
             _hip.stream_of(self.device))
        if check and int(self._status.item()) == _hip.CS_ECAPACITY:
            raise CacheCapacityError("sidecar slot arena is full")
        return out[:count]

    def free_mask(self) -> Tensor:
        """bool [nbits] view of the bitmap (host copy, for inspection)."""
        words = self.bitmap.cpu().view(torch.int32).tolist()
        return torch.tensor(
            [bool((words[s >> 5] >> (s & 31)) & 1) for s in range(self.nbits)], dtype=torch.bool
        )


def _pack_words(bits: Tensor, device) -> Tensor:
    """int64 holders of 32-bit words -> int32 device tensor with the same bit patterns."""
    values = [int(v) & 0xFFFFFFFF for v in bits.tolist()]
    signed = [v - (1 << 32) if v >= (1 << 31) else v for v in values]
    return torch.tensor(signed, dtype=torch.int32, device=device)
