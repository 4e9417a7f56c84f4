"""Shared helpers for the GPU parity tests (seeded inputs, oracle conversion)."""

from __future__ import annotations

import numpy as np
import torch

# bf16 attention outputs: within 2e-2 absolute / 1e-2 relative of the fp32 oracle
BF16_ATOL, BF16_RTOL = 2e-2, 1e-2


def seeded(shape, seed: int, *, scale: float = 1.0, dtype=torch.float32) -> torch.Tensor:
    """CPU tensor ~ N(0, scale^2) from torch.Generator('cpu').manual_seed(seed), cast to dtype."""
    gen = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(shape, generator=gen, dtype=torch.float32) * scale).to(dtype)


def acc_np(t: torch.Tensor) -> np.ndarray:
    """A tensor's values in its accumulation dtype as numpy (bf16/f16 -> float32 exactly)."""
    t = t.detach().cpu()
    if t.dtype == torch.float64:
        return t.numpy()
    return t.float().numpy()


def assert_close_bf16(actual: torch.Tensor, expected: np.ndarray) -> None:
    torch.testing.assert_close(
        actual.detach().cpu().float(), torch.from_numpy(np.asarray(expected, np.float32)),
        atol=BF16_ATOL, rtol=BF16_RTOL,
    )


def tolerance(dtype: torch.dtype) -> dict:
    if dtype == torch.float64:
        return {"atol": 1e-10, "rtol": 1e-10}
    if dtype == torch.float32:
        # fp32 dot products in a different order, amplified by softmax
        return {"atol": 1e-4, "rtol": 1e-4}
    return {"atol": BF16_ATOL, "rtol": BF16_RTOL}


def paged_layout(n_tokens: list[int], kv_heads: int, block_size: int, head_dim: int, seed: int,
                 extra_blocks: int = 3):
    """Random block tables (seeded permutation) for requests of n_tokens each.

    Returns (num_blocks, block_table int32 [B, max_blocks] with -1 padding, per-request lists).
    """
    per = [(n + block_size - 1) // block_size for n in n_tokens]
    total = sum(per) + extra_blocks
    gen = torch.Generator("cpu").manual_seed(seed)
    perm = torch.randperm(total, generator=gen).tolist()
    width = max(per) if per else 1
    table = torch.full((len(n_tokens), width), -1, dtype=torch.int32)
    rows, cursor = [], 0
    for b, nb in enumerate(per):
        row = perm[cursor : cursor + nb]
        cursor += nb
        table[b, :nb] = torch.tensor(row, dtype=torch.int32)
        rows.append(row)
    return total, table, rows


def fill_paged(cache: torch.Tensor, rows: list[list[int]], keys: list[torch.Tensor],
               values: list[torch.Tensor]) -> None:
    """Host-side reference placement of dense K/V [n, H, D] into cache [blocks, H, bs, 2D]."""
    bs = cache.shape[2]
    d = cache.shape[3] // 2
    for row, k, v in zip(rows, keys, values):
        for t in range(k.shape[0]):
            blk, off = row[t // bs], t % bs
            cache[blk, :, off, :d] = k[t]
            cache[blk, :, off, d:] = v[t]


class HostMover:
    """Host stand-in for the slot kernels, for tests of the paged-arena rules
    without a GPU: native slot s is cache[s // bs, :, s % bs] (K in the first
    half of the record, V in the second), slot native + i is sidecar row i."""

    def scatter(self, cache, side_k, side_v, slots, key, value, rows=None):
        bs, native, d = cache.shape[2], cache.shape[0] * cache.shape[2], cache.shape[3] // 2
        for i, slot in enumerate(slots):
            r = i if rows is None else rows[i]
            if slot < native:
                cache[slot // bs, :, slot % bs, :d] = key[r]
                cache[slot // bs, :, slot % bs, d:] = value[r]
            else:
                side_k[slot - native] = key[r]
                side_v[slot - native] = value[r]

    def gather(self, cache, side_k, side_v, slots, key, value):
        bs, native, d = cache.shape[2], cache.shape[0] * cache.shape[2], cache.shape[3] // 2
        for i, slot in enumerate(slots):
            if slot < native:
                key[i] = cache[slot // bs, :, slot % bs, :d]
                value[i] = cache[slot // bs, :, slot % bs, d:]
            else:
                key[i] = side_k[slot - native]
                value[i] = side_v[slot - native]
