"""Fused CCPE attention over the paged KV cache (bf16, head dim 128).

These entry points read K and V straight from the vLLM-layout paged cache
[blocks, kv_heads, block_size, 2 * 128] instead of first materialising the
logical K/V with ``NativePagedKV.gather`` (src/cacheslide_vllm/runtime.py:
499-507 and :573, followed by position.py:404-560), with default key
positions 0..nk-1.  Key j of a request is addressed either

* through a block table, at its canonical slot ``table[j // bs] * bs + j % bs``
  (paged.py:146-151) -- what a vLLM block table names; or
* through a per-token slot map -- the slot ``NativePagedKV.gather`` reads for
  token j, native or sidecar (paged.py:433-472).  After SLIDE relocation and
  decode hole reuse the canonical slot of a selected token may hold a decode
  token's K/V and the token itself lives in the sidecar (paged.py:474-524,
  slide.py:401-459), so only this form equals ``gather`` + ``cope_attention``
  on such an arena.  ``ccpe_decode_arena`` / ``ccpe_prefill_arena`` take the map
  from a ``NativePagedKV`` under the same pins ``gather`` takes.

* ``ccpe_prefill_paged``: many query rows per request (MFMA kernel).
* ``ccpe_decode_paged``: one new row per request at position nk-1 (split-K
  kernel with speculative saturation).
* ``ccpe_decode_shared``: the same decode when the requests' block tables
  start with runs of blocks that several requests share (reused chunks,
  ``SharedRuns``): each run is read once for the whole batch.
"""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from . import _hip
from ._hip import call, ptr


def _check_e(cope, device, max_positions: int = 256) -> Tensor:
    e = cope.position_embeddings.detach()
    if e.device != device:
        raise ValueError("query and learned embeddings must share a device")
    if e.dtype != torch.float32 or not e.is_contiguous() or e.shape[0] != 128:
        raise ValueError("the fused kernels need a contiguous float32 [128, P] CoPE table")
    if not 2 <= cope.max_positions <= max_positions:
        raise ValueError(f"this fused kernel supports 2 <= max_positions <= {max_positions}")
    return e


def _cache_source(cache: Tensor) -> _hip.CsKvSource:
    if cache.ndim != 4 or cache.dtype != torch.bfloat16 or cache.shape[3] != 256:
        raise ValueError("cache must be bf16 [blocks, kv_heads, block_size, 256]")
    if cache.stride(3) != 1:
        raise ValueError("cache records must be contiguous in the last dimension")
    src = _hip.CsKvSource()
    src.cache = cache.data_ptr()
    src.s_block, src.s_head, src.s_offset = cache.stride(0), cache.stride(1), cache.stride(2)
    src.block_size = cache.shape[2]
    src.num_blocks = cache.shape[0]
    return src


def _paged_source(cache: Tensor, block_table: Tensor) -> _hip.CsKvSource:
    src = _cache_source(cache)
    if block_table.ndim != 2 or block_table.dtype != torch.int32:
        raise ValueError("block_table must be int32 [batch, max_blocks]")
    if block_table.stride(1) != 1:
        raise ValueError("block_table rows must be contiguous")
    src.block_table = block_table.data_ptr()
    src.bt_stride = block_table.stride(0)
    src.bt_cols = block_table.shape[1]
    return src


def _slot_source(cache: Tensor, slots: Tensor, side_k: Tensor | None,
                 side_v: Tensor | None) -> _hip.CsKvSource:
    """Per-token slot map [B, >= nk] int64; slots past the native pool name sidecar rows."""
    src = _cache_source(cache)
    if slots.ndim != 2 or slots.dtype != torch.long or slots.stride(1) != 1:
        raise ValueError("slots must be int64 [batch, tokens] with contiguous rows")
    src.slots = slots.data_ptr()
    src.slots_stride = slots.stride(0)
    src.slots_cols = slots.shape[1]
    if (side_k is None) != (side_v is None):
        raise ValueError("side_k and side_v go together")
    if side_k is not None:
        for side in (side_k, side_v):
            if (side.ndim != 3 or side.dtype != torch.bfloat16 or side.shape[1:] != (cache.shape[1], 128)
                    or side.stride(2) != 1 or side.device != cache.device):
                raise ValueError("sidecar must be bf16 [rows, kv_heads, 128] on the cache device")
        if side_k.shape != side_v.shape or side_k.stride() != side_v.stride():
            raise ValueError("side_k and side_v must share shape and strides")
        if side_k.shape[0]:
            src.side_k, src.side_v = side_k.data_ptr(), side_v.data_ptr()
            src.side_s_row, src.side_s_head = side_k.stride(0), side_k.stride(1)
            src.side_rows = side_k.shape[0]
    return src


def _kv_source(cache: Tensor, block_table: Tensor | None, slots: Tensor | None,
               side_k: Tensor | None, side_v: Tensor | None) -> _hip.CsKvSource:
    if slots is not None:
        if block_table is not None:
            raise ValueError("give either block_table or slots, not both")
        return _slot_source(cache, slots, side_k, side_v)
    if block_table is None:
        raise ValueError("block_table or slots is required")
    if side_k is not None or side_v is not None:
        raise ValueError("sidecar rows are addressed through slots only")
    return _paged_source(cache, block_table)


def _prefill_dense(query: Tensor, key: Tensor, value: Tensor, e: Tensor,
                   query_positions: Tensor, ck) -> Tensor:
    """One request, dense K/V [nk, Hkv, 128]; used by cope_attention's fast path."""
    device = ck.device
    nq, hq = query.shape[0], query.shape[1]
    nk, hkv = key.shape[0], key.shape[1]
    out = torch.empty((1, nq, hq, 128), dtype=torch.bfloat16, device=device)
    nk_dev = torch.full((1,), nk, dtype=torch.int32, device=device)
    src = _hip.CsKvSource()
    src.k, src.v = key.data_ptr(), value.data_ptr()
    src.k_s_batch, src.k_s_tok, src.k_s_head = 0, key.stride(0), key.stride(1)
    src.v_s_batch, src.v_s_tok, src.v_s_head = 0, value.stride(0), value.stride(1)
    if key.stride(2) != 1 or value.stride(2) != 1 or query.stride(2) != 1:
        q_c, k_c, v_c = query.contiguous(), key.contiguous(), value.contiguous()
        return _prefill_dense(q_c, k_c, v_c, e, query_positions, ck)
    call(
        "cs_ccpe_prefill_bf16", ptr(query), 0, query.stride(0), query.stride(1),
        ptr(query_positions), 0, 1, nq, hq, hkv, ptr(nk_dev), src, ptr(e),
        e.shape[1], ptr(out), ck.flags_ptr, ck.stream,
    )
    return out[0]


def ccpe_prefill_paged(
    query: Tensor,
    cache: Tensor,
    block_table: Tensor | None,
    context_lens: Tensor,
    cope,
    query_positions: Tensor,
    *,
    slots: Tensor | None = None,
    side_k: Tensor | None = None,
    side_v: Tensor | None = None,
    check: bool = True,
) -> Tensor:
    """Batched CCPE prefill over the paged cache.

    query [B, nq, Hq, 128] bf16; cache bf16 [blocks, Hkv, bs, 256]; keys
    0..n-1 of request b (n = context_lens[b], int32 [B]) come through
    ``block_table`` (int32 [B, max_blocks]: block table[b, j // bs], offset
    j % bs) or through ``slots`` (int64 [B, >= n]: native slots and rows of
    ``side_k`` / ``side_v``); query_positions int64 [B, nq].  Returns
    [B, nq, Hq, 128] bf16.  With ``check`` the invalid-block flag is read back
    (one sync).
    """
    device = _hip.require_device(query, cache, context_lens, query_positions, block_table, slots)
    if query.ndim != 4 or query.dtype != torch.bfloat16 or query.shape[3] != 128 or query.stride(3) != 1:
        raise ValueError("query must be bf16 [batch, rows, heads, 128] with contiguous rows")
    b, nq, hq = query.shape[0], query.shape[1], query.shape[2]
    hkv = cache.shape[1]
    if hq % hkv:
        raise ValueError("query heads must be a multiple of KV heads for GQA")
    if context_lens.shape != (b,) or context_lens.dtype != torch.int32:
        raise ValueError("context_lens must be int32 [batch]")
    if query_positions.shape != (b, nq) or query_positions.dtype != torch.long or query_positions.stride(1) != 1:
        raise ValueError("query_positions must be int64 [batch, rows]")
    if slots is not None and slots.shape[0] != b:
        raise ValueError("slots must have one row per request")
    e = _check_e(cope, device, max_positions=128)
    src = _kv_source(cache, block_table, slots, side_k, side_v)
    flags = _hip.new_flags(device)
    out = torch.empty((b, nq, hq, 128), dtype=torch.bfloat16, device=device)
    call(
        "cs_ccpe_prefill_bf16", ptr(query), query.stride(0), query.stride(1), query.stride(2),
        ptr(query_positions), query_positions.stride(0), b, nq, hq, hkv, ptr(context_lens), src,
        ptr(e), cope.max_positions, ptr(out), ptr(flags), _hip.stream_of(device),
    )
    if check:
        raise_flags(flags)
    return out


def ccpe_prefill_arena(query: Tensor, arena, cope, query_positions: Tensor, *,
                       check: bool = True) -> Tensor:
    """``cope_attention(query, *arena.gather(range(n)), cope, query_positions)``
    for one request's arena (runtime.py:571-573 without policies), fused: the
    kernel reads the n logical tokens in place through the arena's slot map.

    query [nq, Hq, 128] bf16, query_positions int64 [nq] (< n); returns
    [nq, Hq, 128] bf16.
    """
    n = arena.logical_length()
    with arena.device_slots(range(n)) as (slots, side_k, side_v):
        lens = torch.full((1,), n, dtype=torch.int32, device=query.device)
        out = ccpe_prefill_paged(query.unsqueeze(0), arena.cache, None, lens, cope,
                                 query_positions.reshape(1, -1).contiguous(), slots=slots.unsqueeze(0),
                                 side_k=side_k, side_v=side_v, check=check)
    return out[0]


def decode_workspace_bytes(batch: int, heads: int, max_context: int, split: int) -> int:
    return int(_hip.load().cs_ccpe_decode_workspace_bytes(batch, heads, max_context, split))


def decode_workspace(batch: int, heads: int, max_context: int, split: int, device) -> Tensor:
    nbytes = decode_workspace_bytes(batch, heads, max_context, split)
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def ccpe_decode_paged(
    query: Tensor,
    cache: Tensor,
    block_table: Tensor | None,
    context_lens: Tensor,
    cope,
    *,
    slots: Tensor | None = None,
    side_k: Tensor | None = None,
    side_v: Tensor | None = None,
    max_context: int | None = None,
    split: int = 1024,
    workspace: Tensor | None = None,
    out: Tensor | None = None,
    flags: Tensor | None = None,
    check: bool = True,
) -> Tensor:
    """Batched CCPE decode: row b attends keys 0..context_lens[b]-1 at position context_lens[b]-1.

    query [B, Hq, 128] bf16; returns [B, Hq, 128] bf16.  Keys come through
    ``block_table`` (int32 [B, max_blocks]) or through ``slots`` (int64
    [B, >= max_context], native slots and rows of ``side_k`` / ``side_v``).
    ``max_context`` bounds context_lens (read back from the device when
    omitted); a larger context raises ValueError, as does an empty one
    (position.py:149-150).  ``split`` is the number of keys per split-K work
    item (multiple of 64, <= 1024).  ``workspace`` (uint8, device) must hold
    ``decode_workspace_bytes(B, Hq, max_context, split)`` bytes.  ``out``
    (bf16 [B, Hq, 128], contiguous) receives the rows when given.  ``flags``
    (from ``_hip.new_flags``) collects the error bits of this and earlier
    calls when given, for a caller that checks once (``raise_flags``) after a
    loop of calls with ``check=False``.
    """
    device = _hip.require_device(query, cache, context_lens, block_table, slots)
    if query.ndim != 3 or query.dtype != torch.bfloat16 or query.shape[2] != 128 or query.stride(2) != 1:
        raise ValueError("query must be bf16 [batch, heads, 128] with contiguous rows")
    b, hq = query.shape[0], query.shape[1]
    hkv = cache.shape[1]
    if hq % hkv or hq // hkv > 8:
        raise ValueError("decode supports GQA groups of at most 8 query heads per KV head")
    if context_lens.shape != (b,) or context_lens.dtype != torch.int32:
        raise ValueError("context_lens must be int32 [batch]")
    e = _check_e(cope, device)
    src = _kv_source(cache, block_table, slots, side_k, side_v)
    if max_context is None:
        max_context = max(int(context_lens.max().item()), 1) if b else 1
    if type(max_context) is not int or max_context < 1:
        raise ValueError("max_context must be a positive integer")
    if slots is not None and slots.shape[0] != b:
        raise ValueError("slots must have one row per request")
    if slots is not None and slots.shape[1] < max_context:
        raise ValueError("slots must cover max_context tokens per request")
    need = decode_workspace_bytes(b, hq, max_context, split)
    if workspace is None:
        workspace = decode_workspace(b, hq, max_context, split, device)
    elif workspace.device != device or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous tensor on the query device")
    have = workspace.numel() * workspace.element_size()
    if have < need:
        raise ValueError(f"decode workspace holds {have} bytes, the call needs {need}")
    if flags is None:
        flags = _hip.new_flags(device)
    elif flags.device != device or flags.dtype != torch.int32 or flags.numel() < 1:
        raise ValueError("flags must be an int32 tensor on the query device")
    if out is None:
        out = torch.empty((b, hq, 128), dtype=torch.bfloat16, device=device)
    elif (out.shape != (b, hq, 128) or out.dtype != torch.bfloat16 or out.device != device
          or not out.is_contiguous()):
        raise ValueError("out must be a contiguous bf16 [batch, heads, 128] tensor on the query device")
    call(
        "cs_ccpe_decode_bf16", ptr(query), query.stride(0), query.stride(1), b, hq, hkv,
        ptr(context_lens), max_context, src, ptr(e), cope.max_positions, split, ptr(workspace),
        have, ptr(out), ptr(flags), _hip.stream_of(device),
    )
    if check:
        raise_flags(flags)
    return out


def ccpe_decode_arena(query: Tensor, arena, cope, *, split: int = 1024, check: bool = True) -> Tensor:
    """The decode step of runtime.py:489-508 on one request's arena, fused:
    ``cope_attention(query, *arena.gather(range(n)), cope, [n - 1])`` with n the
    arena's logical length, read in place through the arena's slot map.

    query [Hq, 128] (or [1, Hq, 128]) bf16; returns [1, Hq, 128] bf16.
    """
    if query.ndim == 2:
        query = query.unsqueeze(0)
    n = arena.logical_length()
    with arena.device_slots(range(n)) as (slots, side_k, side_v):
        lens = torch.full((1,), n, dtype=torch.int32, device=query.device)
        return ccpe_decode_paged(query, arena.cache, None, lens, cope, slots=slots.unsqueeze(0),
                                 side_k=side_k, side_v=side_v, max_context=max(n, 1), split=split,
                                 check=check)


class SharedRuns:
    """Requests whose block tables start with runs of shared blocks.

    ``runs`` (int [R, run_blocks]) names the blocks of each shared run (a
    reused chunk), ``request_runs`` (int [B, S]) the run at each of request
    b's first S run slots, in key order: ``block_table[b, :S * run_blocks]``
    must be those runs' blocks one after the other (checked here, once).  A
    request holds a run at most once.  The last ``margin`` keys of every
    request's shared part (a multiple of the block size, at least one block)
    and its keys after it form its tail, computed with exact contextual
    positions; the rest of the shared part is read run by run for the whole
    batch with every position P-1, which holds when the tail's gate mass
    reaches P-1 and is checked on the device each call (``ccpe_decode_shared``
    runs the exact decode where it does not).  Each run is cut into
    ``pieces`` equal parts, the units of work of the shared read.
    """

    def __init__(self, block_table: Tensor, runs, request_runs, block_size: int, *, margin: int = 256,
                 pieces: int = 2):
        runs = torch.as_tensor(runs, dtype=torch.int32).cpu()
        request_runs = torch.as_tensor(request_runs, dtype=torch.int64).cpu()
        if runs.ndim != 2 or request_runs.ndim != 2 or runs.shape[1] < 1:
            raise ValueError("runs must be [R, run_blocks] and request_runs [B, S]")
        if block_table.ndim != 2 or block_table.dtype != torch.int32 or block_table.stride(1) != 1:
            raise ValueError("block_table must be int32 [batch, max_blocks] with contiguous rows")
        n_runs, run_blocks = runs.shape
        b, n_slots = request_runs.shape
        if b != block_table.shape[0]:
            raise ValueError("request_runs must have one row per request")
        if n_slots < 1 or bool((request_runs < 0).any()) or bool((request_runs >= n_runs).any()):
            raise ValueError("request_runs must name runs, at least one per request")
        if any(len(set(row.tolist())) != n_slots for row in request_runs):
            raise ValueError("a request holds a run at most once")
        if type(margin) is not int or margin < block_size or margin % block_size:
            raise ValueError("margin must be a positive multiple of the block size")
        if type(pieces) is not int or pieces < 1 or run_blocks % pieces:
            raise ValueError("pieces must divide the run's blocks")
        shared_blocks = n_slots * run_blocks
        run_keys = run_blocks * block_size
        if margin >= shared_blocks * block_size:
            raise ValueError("margin must leave keys of the shared part outside the tail")
        if shared_blocks > block_table.shape[1]:
            raise ValueError("block_table is shorter than the requests' shared parts")
        expect = runs[request_runs].reshape(b, shared_blocks)
        if not torch.equal(block_table[:, :shared_blocks].cpu(), expect):
            raise ValueError("block_table does not start with the requests' runs")
        piece_blocks = run_blocks // pieces
        piece_keys = piece_blocks * block_size
        device = block_table.device
        self.block_size = block_size
        self.head_items = n_runs * pieces
        self.head_blocks = piece_blocks
        self.head_table = runs.view(n_runs * pieces, piece_blocks).contiguous().to(device)
        self.head_nk = torch.full((self.head_items,), piece_keys, dtype=torch.int32, device=device)
        # request b sees keys [0, limit) of its slot s's run, limit = run_keys
        # except in the slots the tail reaches into
        tail_key = shared_blocks * block_size - margin        # first tail key of every request
        qpos = torch.full((self.head_items, b), -1, dtype=torch.int64)
        for slot in range(n_slots):
            limit = min(run_keys, max(tail_key - slot * run_keys, 0))
            for k in range(pieces):
                visible = min(max(limit - k * piece_keys, 0), piece_keys)
                items = request_runs[:, slot] * pieces + k
                qpos[items, torch.arange(b)] = visible - 1
        self.head_qpos = qpos.to(device)
        self.tail_block = tail_key // block_size              # first block of the tail
        self.tail_table = block_table[:, self.tail_block:]
        self.batch = b

    def tail_lens(self, context_lens: Tensor) -> tuple[Tensor, Tensor]:
        """Key counts of the tails (int32) and their query keys (int64)."""
        tail_nk = context_lens - self.tail_block * self.block_size
        return tail_nk, (tail_nk - 1).to(torch.int64)


def decode_shared_workspace(batch: int, heads: int, shared: SharedRuns, max_context: int, split: int,
                            device) -> Tensor:
    nbytes = int(_hip.load().cs_ccpe_decode_shared_workspace_bytes(batch, heads, shared.head_items, max_context,
                                                                      split))
    return torch.empty(max(nbytes, 256) + 256, dtype=torch.uint8, device=device)


def ccpe_decode_shared(
    query: Tensor,
    cache: Tensor,
    block_table: Tensor,
    context_lens: Tensor,
    cope,
    shared: SharedRuns,
    *,
    max_context: int,
    split: int = 1024,
    tail: tuple[Tensor, Tensor] | None = None,
    workspace: Tensor | None = None,
    out: Tensor | None = None,
    flags: Tensor | None = None,
    check: bool = True,
) -> Tensor:
    """``ccpe_decode_paged`` over ``block_table`` (same arguments and result)
    with the requests' shared runs (``shared``, built on this block table)
    read once for the batch.  Every request's context must extend past its
    shared part's tail start (``context_lens > shared.tail_block * block
    size``).  ``tail``: ``shared.tail_lens(context_lens)`` when the caller has
    it; ``workspace``: ``decode_shared_workspace(...)`` bytes."""
    device = _hip.require_device(query, cache, context_lens, block_table)
    if query.ndim != 3 or query.dtype != torch.bfloat16 or query.shape[2] != 128 or query.stride(2) != 1:
        raise ValueError("query must be bf16 [batch, heads, 128] with contiguous rows")
    b, hq = query.shape[0], query.shape[1]
    hkv = cache.shape[1]
    if hq % hkv or hq // hkv > 8:
        raise ValueError("decode supports GQA groups of at most 8 query heads per KV head")
    if context_lens.shape != (b,) or context_lens.dtype != torch.int32:
        raise ValueError("context_lens must be int32 [batch]")
    if shared.batch != b or shared.block_size != cache.shape[2]:
        raise ValueError("shared runs were built for another batch or block size")
    if type(max_context) is not int or max_context < 1:
        raise ValueError("max_context must be a positive integer")
    e = _check_e(cope, device)
    src = _paged_source(cache, block_table)
    tail_nk, tail_qpos = shared.tail_lens(context_lens) if tail is None else tail
    nbytes = int(_hip.load().cs_ccpe_decode_shared_workspace_bytes(b, hq, shared.head_items, max_context, split))
    if workspace is None:
        workspace = decode_shared_workspace(b, hq, shared, max_context, split, device)
    start = (-workspace.data_ptr()) % 256
    have = workspace.numel() * workspace.element_size() - start
    if workspace.device != device or have < nbytes:
        raise ValueError(f"decode workspace holds {have} bytes after alignment, the call needs {nbytes}")
    if flags is None:
        flags = _hip.new_flags(device)
    if out is None:
        out = torch.empty((b, hq, 128), dtype=torch.bfloat16, device=device)
    elif (out.shape != (b, hq, 128) or out.dtype != torch.bfloat16 or out.device != device
          or not out.is_contiguous()):
        raise ValueError("out must be a contiguous bf16 [batch, heads, 128] tensor on the query device")
    args = _hip.CsDecodeSharedArgs()
    args.q = query.data_ptr()
    args.q_s_batch, args.q_s_head = query.stride(0), query.stride(1)
    args.batch, args.hq, args.hkv = b, hq, hkv
    args.nk = context_lens.data_ptr()
    args.max_nk = max_context
    args.kv = ctypes.pointer(src)
    args.e = e.data_ptr()
    args.max_positions = cope.max_positions
    args.split = split
    args.head_table = shared.head_table.data_ptr()
    args.head_items, args.head_blocks = shared.head_items, shared.head_blocks
    args.head_nk = shared.head_nk.data_ptr()
    args.head_qpos = shared.head_qpos.data_ptr()
    args.tail_table = shared.tail_table.data_ptr()
    args.tail_stride = shared.tail_table.stride(0)
    args.tail_cols = shared.tail_table.shape[1]
    args.tail_nk = tail_nk.data_ptr()
    args.tail_qpos = tail_qpos.data_ptr()
    args.out = out.data_ptr()
    args.flags = flags.data_ptr()
    call("cs_ccpe_decode_shared_bf16", ctypes.byref(args), workspace.data_ptr() + start, have,
         _hip.stream_of(device))
    if check:
        raise_flags(flags)
    return out


def raise_flags(flags: Tensor) -> None:
    """Raise the error the fused decode / prefill calls recorded in ``flags``
    (reads them back, so it waits for those calls)."""
    value = _hip.read_flags(flags)[0]
    if value & _hip.FLAG_NO_KEY:
        raise ValueError("attention requires at least one key")
    if value & _hip.FLAG_CONTEXT_RANGE:
        raise ValueError("context_lens exceeds max_context")
    if value & _hip.FLAG_BLOCK_INVALID:
        raise ValueError("a block-table entry or slot names a record outside the cache")
