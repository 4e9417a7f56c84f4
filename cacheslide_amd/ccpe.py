"""Fused CCPE attention over the paged KV cache (bf16, head dim 128).

These entry points read K and V straight from the vLLM-layout paged cache
[blocks, kv_heads, block_size, 2 * 128] through a block table, instead of
first materialising the logical K/V with ``NativePagedKV.gather``
(src/cacheslide_vllm/runtime.py:573 and :505-507 followed by
position.py:404-560).  Results equal ``cope_attention`` on the gathered K/V
with default key positions 0..nk-1, within the bf16 tolerance.

* ``ccpe_prefill_paged``: many query rows per request (MFMA kernel).
* ``ccpe_decode_paged``: one new row per request at position nk-1 (split-K
  kernel with speculative saturation).
"""

from __future__ import annotations

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


def _paged_source(cache: Tensor, block_table: Tensor) -> _hip.CsKvSource:
    if cache.ndim != 4 or cache.dtype != torch.bfloat16 or cache.shape[3] != 256:
        raise ValueError("cache must be bf16 [blocks, kv_heads, block_size, 256]")
    if cache.stride(3) != 1:
        raise ValueError("cache records must be contiguous in the last dimension")
    if block_table.ndim != 2 or block_table.dtype != torch.int32:
        raise ValueError("block_table must be int32 [batch, max_blocks]")
    src = _hip.CsKvSource()
    src.cache = cache.data_ptr()
    src.s_block, src.s_head, src.s_offset = cache.stride(0), cache.stride(1), cache.stride(2)
    src.block_size = cache.shape[2]
    src.num_blocks = cache.shape[0]
    src.block_table = block_table.data_ptr()
    src.bt_stride = block_table.stride(0)
    src.bt_cols = block_table.shape[1]
    if block_table.stride(1) != 1:
        raise ValueError("block_table rows must be contiguous")
    return src


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
    block_table: Tensor,
    context_lens: Tensor,
    cope,
    query_positions: Tensor,
    *,
    check: bool = True,
) -> Tensor:
    """Batched CCPE prefill over the paged cache.

    query [B, nq, Hq, 128] bf16; cache bf16 [blocks, Hkv, bs, 256];
    block_table int32 [B, max_blocks]; context_lens int32 [B] (keys 0..n-1 of
    request b live at block_table[b, j // bs], offset j % bs);
    query_positions int64 [B, nq].  Returns [B, nq, Hq, 128] bf16.
    With ``check`` the nonfinite / invalid-block flags are read back (one sync).
    """
    device = _hip.require_device(query, cache, block_table, context_lens, query_positions)
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
    e = _check_e(cope, device, max_positions=128)
    src = _paged_source(cache, block_table)
    flags = _hip.new_flags(device)
    out = torch.empty((b, nq, hq, 128), dtype=torch.bfloat16, device=device)
    call(
        "cs_ccpe_prefill_bf16", ptr(query), query.stride(0), query.stride(1), query.stride(2),
        ptr(query_positions), query_positions.stride(0), b, nq, hq, hkv, ptr(context_lens), src,
        ptr(e), cope.max_positions, ptr(out), ptr(flags), _hip.stream_of(device),
    )
    if check:
        _raise_flags(flags)
    return out


def decode_workspace(batch: int, heads: int, max_context: int, split: int, device) -> Tensor:
    nbytes = int(_hip.load().cs_ccpe_decode_workspace_bytes(batch, heads, max_context, split))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def ccpe_decode_paged(
    query: Tensor,
    cache: Tensor,
    block_table: Tensor,
    context_lens: Tensor,
    cope,
    *,
    max_context: int | None = None,
    split: int = 1024,
    workspace: Tensor | None = None,
    check: bool = True,
) -> Tensor:
    """Batched CCPE decode: row b attends keys 0..context_lens[b]-1 at position context_lens[b]-1.

    query [B, Hq, 128] bf16; returns [B, Hq, 128] bf16.  ``max_context`` bounds
    context_lens (read back from the device when omitted); ``split`` is the
    number of keys per split-K work item (multiple of 64, <= 1024).
    """
    device = _hip.require_device(query, cache, block_table, context_lens)
    if query.ndim != 3 or query.dtype != torch.bfloat16 or query.shape[2] != 128 or query.stride(2) != 1:
        raise ValueError("query must be bf16 [batch, heads, 128] with contiguous rows")
    b, hq = query.shape[0], query.shape[1]
    hkv = cache.shape[1]
    if hq % hkv or hq // hkv > 8:
        raise ValueError("decode supports GQA groups of at most 8 query heads per KV head")
    if context_lens.shape != (b,) or context_lens.dtype != torch.int32:
        raise ValueError("context_lens must be int32 [batch]")
    e = _check_e(cope, device)
    src = _paged_source(cache, block_table)
    if max_context is None:
        max_context = int(context_lens.max().item()) if b else 1
    if workspace is None:
        workspace = decode_workspace(b, hq, max_context, split, device)
    flags = _hip.new_flags(device)
    out = torch.empty((b, hq, 128), dtype=torch.bfloat16, device=device)
    call(
        "cs_ccpe_decode_bf16", ptr(query), query.stride(0), query.stride(1), b, hq, hkv,
        ptr(context_lens), max_context, src, ptr(e), cope.max_positions, split, ptr(workspace),
        ptr(out), ptr(flags), _hip.stream_of(device),
    )
    if check:
        _raise_flags(flags)
    return out


def _raise_flags(flags: Tensor) -> None:
    value = _hip.read_flags(flags)[0]
    if value & _hip.FLAG_BLOCK_INVALID:
        raise ValueError("block_table names a block outside the cache")
