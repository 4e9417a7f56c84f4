"""Torch-on-CPU restatement of the reuse-attention path -- TEST INFRASTRUCTURE.

This is the timed CPU baseline of ``bench.py`` (and nothing else): the
reference's operations in the reference's order, in torch on the host, so the
CPU figure measures what the reference path costs on the same box.  It is
checked against the numpy oracle in ``tests/test_torch_cpu.py``.  Paths are
relative to the CacheSlide repository, ``src/cacheslide_vllm/``.

* ``cope_attention``: position.py:404-560 for the plain contextual case --
  per query chunk: GQA ``repeat_interleave``, fp32 einsum logits / sqrt(D),
  causal mask, sigmoid gates, flip-cumsum-flip (fp32 on the CPU accumulates in
  fp64), clamp, Q.E einsum with the floor / floor+1 gather and lerp, masked
  softmax, einsum P.V, cast to the value dtype.
* ``paged_gather``: NativePagedKV.gather by advanced indexing (paged.py:433-472).
* ``relocate``: page and slot moves by advanced indexing on the
  [blocks, kv heads, block size, 2 D] layout, the token -> slot map update and
  the returned source slots (slide.py:243-372 with paged.py:205-240).
* ``WCA``: wca.py:55-304 in float64 (deviation, weight, stable top-k, blend,
  cosine gate, commit).
"""

from __future__ import annotations

import math

import torch
from torch import Tensor


# ------------------------------------------------------------------ CCPE
def cope_attention(query: Tensor, key: Tensor, value: Tensor, table: Tensor, query_positions: Tensor,
                   *, query_chunk_size: int = 64) -> Tensor:
    """query [q, Hq, D], key/value [k, Hkv, D] (bf16 or fp32), table [D, P] fp32,
    query_positions int64 [q]; keys at positions 0..k-1."""
    acc = torch.float32
    nk, hq = key.shape[0], query.shape[1]
    group = hq // key.shape[1]
    npos = table.shape[1]
    key_positions = torch.arange(nk)
    keys = key.repeat_interleave(group, dim=1).to(acc)
    values = value.repeat_interleave(group, dim=1).to(acc)
    e = table.to(acc)
    outputs = []
    for start in range(0, query.shape[0], query_chunk_size):
        end = min(start + query_chunk_size, query.shape[0])
        q = query[start:end].to(acc)
        logits = torch.einsum("qhd,khd->hqk", q, keys) / math.sqrt(q.shape[-1])
        if not torch.isfinite(logits).all():                       # position.py:162-163
            raise ValueError("attention logits overflowed the accumulation dtype")
        allowed = (key_positions[None, :] <= query_positions[start:end, None]).unsqueeze(0)
        allowed = allowed.expand(hq, -1, -1)
        if not torch.isfinite(logits[allowed]).all():              # position.py:304-305
            raise ValueError("unmasked logits must be finite")
        gates = torch.sigmoid(logits.masked_fill(~allowed, float("-inf")))
        positions = gates.flip(-1).cumsum(-1).flip(-1).clamp(0, npos - 1)
        if not torch.isfinite(positions).all() or (positions < 0).any() or (positions > npos - 1).any():
            raise ValueError("positions must be bounded query-dependent [head,query,key]")
        qe = torch.einsum("qhd,dp->hqp", q, e)
        lower = positions.floor().long()
        upper = (lower + 1).clamp(max=npos - 1)
        frac = positions - lower.to(acc)
        low, high = qe.gather(-1, lower), qe.gather(-1, upper)
        logits = logits + (low + frac * (high - low))
        if not torch.isfinite(logits).all():                       # position.py:519-520
            raise ValueError("contextual attention logits are not finite")
        any_allowed = allowed.any(-1, keepdim=True)
        logits = logits.masked_fill(~allowed, float("-inf"))
        logits = torch.where(any_allowed, logits, torch.zeros_like(logits))
        probs = logits.softmax(-1).masked_fill(~allowed, 0)
        outputs.append(torch.einsum("hqk,khd->qhd", probs, values))
    return torch.cat(outputs).to(value.dtype)


def paged_gather(cache: Tensor, slots: Tensor) -> tuple[Tensor, Tensor]:
    """K/V rows [n, H, D] of native slots (block slot // bs, offset slot % bs)."""
    bs, d = cache.shape[2], cache.shape[3] // 2
    rec = cache[slots // bs, :, slots % bs]
    return rec[..., :d], rec[..., d:]


def decode_step(cache: Tensor, block_row: Tensor, n: int, query: Tensor, table: Tensor) -> Tensor:
    """The decode step of runtime.py:489-508: gather the n logical tokens of one
    request through its canonical slots, then cope_attention at position n-1."""
    bs = cache.shape[2]
    t = torch.arange(n)
    slots = block_row[t // bs].long() * bs + t % bs
    k, v = paged_gather(cache, slots)
    return cope_attention(query, k, v, table, torch.tensor([n - 1]))


# ------------------------------------------------------------------ SLIDE
def relocate(cache: Tensor, src_blocks: Tensor, dst_blocks: Tensor, src_slots: Tensor, dst_slots: Tensor,
             mapping: Tensor, tokens: Tensor, slots: Tensor) -> Tensor:
    """Whole pages, then single token records, then the map; returns the freed
    source slots (what the free list takes back)."""
    cache[dst_blocks] = cache[src_blocks]
    bs = cache.shape[2]
    cache[dst_slots // bs, :, dst_slots % bs] = cache[src_slots // bs, :, src_slots % bs]
    mapping[tokens] = slots
    return torch.cat([(src_blocks[:, None] * bs + torch.arange(bs)).reshape(-1), src_slots])


# ------------------------------------------------------------------ WCA
def squared_deviation(cached: Tensor, fresh: Tensor) -> Tensor:
    return (fresh.double() - cached.double()).square().sum((1, 2))


def adaptation_weight(cached: Tensor, fresh: Tensor, epsilon: float = 1e-8) -> Tensor:
    num = squared_deviation(cached, fresh)
    den = cached.double().square().sum((1, 2)) + epsilon
    return num / den


def mean_head_cosine(a: Tensor, b: Tensor, epsilon: float = 1e-8) -> Tensor:
    a, b = a.double(), b.double()
    a = a / a.abs().amax(-1, keepdim=True).clamp_min(epsilon)
    b = b / b.abs().amax(-1, keepdim=True).clamp_min(epsilon)
    a = torch.nn.functional.normalize(a, dim=-1)
    b = torch.nn.functional.normalize(b, dim=-1)
    return (a * b).sum(-1).clamp(-1, 1).mean(-1)


class WCA:
    """WCAState (wca.py:128-304): masks, weights and the stable top-k."""

    def __init__(self, cached: Tensor, fresh: Tensor, reused: Tensor, mandatory: Tensor, *,
                 fraction: float = 0.15, epsilon: float = 1e-8, gate_interval: int = 4,
                 threshold: float = 0.12):
        if not torch.isfinite(cached).all() or not torch.isfinite(fresh).all():
            raise ValueError("WCA inputs must be finite")
        self.eps, self.gate, self.threshold = epsilon, gate_interval, threshold
        err = squared_deviation(cached, fresh)
        self.mandatory = mandatory.clone()
        self.initial = err
        self.candidate = reused & (err > 0)
        self.budget = min(math.ceil(fraction * int(reused.sum())), int(self.candidate.sum()))
        self.selected = torch.zeros_like(self.candidate)
        self.removed = torch.zeros_like(self.candidate)
        self.alpha = adaptation_weight(cached, fresh, epsilon)
        self.last_layer = 1
        self.promote()

    @property
    def active(self) -> Tensor:
        return torch.nonzero(self.selected | self.mandatory).flatten()

    def promote(self) -> Tensor:
        available = torch.nonzero(self.candidate & ~self.selected & ~self.removed).flatten()
        slots = max(0, self.budget - int(self.selected.sum()))
        order = torch.argsort(-self.initial[available], stable=True)
        promoted = available[order[:slots]]
        self.selected[promoted] = True
        return promoted

    def update(self, layer: int, cached_k: Tensor, cached_v: Tensor, fresh_k: Tensor, fresh_v: Tensor):
        if not torch.isfinite(cached_k).all() or not torch.isfinite(cached_v).all():
            raise ValueError("cached K/V must be finite")
        idx = self.active
        old_k, old_v = cached_k[idx], cached_v[idx]
        if not torch.isfinite(fresh_k).all() or not torch.isfinite(fresh_v).all():
            raise ValueError("recomputed K/V must be finite")
        nxt = adaptation_weight(old_k, fresh_k, self.eps)
        used = torch.where(self.mandatory[idx], torch.ones_like(nxt), self.alpha[idx])
        w = used[:, None, None]
        fused_k = (w * fresh_k.double() + (1 - w) * old_k.double()).to(cached_k.dtype)
        fused_v = (w * fresh_v.double() + (1 - w) * old_v.double()).to(cached_v.dtype)
        if not torch.isfinite(fused_k).all() or not torch.isfinite(fused_v).all():
            raise ValueError("weighted K/V overflowed the cache dtype")
        removed = idx[:0]
        if layer % self.gate == 0:
            cosine = mean_head_cosine(fresh_k, old_k, self.eps)
            removed = idx[self.selected[idx] & (cosine < self.threshold)]
        self.alpha[idx] = nxt
        self.selected[removed] = False
        self.candidate[removed] = False
        self.removed[removed] = True
        promoted = self.promote()
        self.last_layer = layer
        return idx, fused_k, fused_v, removed, promoted
