"""A Mistral-shaped CoPE decoder stepping one token per request over paged KV
caches: the caller of the fused decode in end-to-end runs.

Each layer follows the order of the reference's decoder layer
(src/cacheslide_vllm/reference.py:177-193, vLLM's Llama layer with a learned
CoPE table in place of rotary embeddings): RMSNorm with a fused residual, one
q/k/v projection, the new token's K/V written to its paged slot
(``cs_slot_scatter``, the paged.py:205-240 write), CCPE attention of the new
row over every key of its request (``cs_ccpe_decode_bf16``, the decode call of
runtime.py:489-508), the output projection, RMSNorm and a SiLU-gated MLP.  A
final norm and the LM head give the next-token logits.  Greedy decoding takes
their argmax on the device, so a generation loop never waits for the host;
error flags of every attention call collect in one tensor that is checked
once at the end.

All layers share one block table (one paged cache tensor per layer, the vLLM
layout [blocks, KV heads, block_size, 2 x 128]).  Weights are bf16 from
``torch.Generator`` seeds; the projections are plain library GEMMs.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _hip
from .ccpe import (SharedRuns, ccpe_decode_paged, ccpe_decode_shared, decode_shared_workspace, decode_workspace,
                   raise_flags)
from .position import CoPE

HEAD_DIM = 128


@dataclass(frozen=True)
class DecoderShape:
    layers: int = 32
    hidden: int = 4096
    heads: int = 32
    kv_heads: int = 8
    ffn: int = 14336
    vocab: int = 32000
    npos: int = 64
    eps: float = 1e-5

    def __post_init__(self):
        if self.hidden != self.heads * HEAD_DIM:
            raise ValueError("hidden must be heads x 128")
        if self.heads % self.kv_heads or self.heads // self.kv_heads > 8:
            raise ValueError("GQA groups of at most 8 query heads per KV head")

    @property
    def parameters(self) -> int:
        qkv = (self.heads + 2 * self.kv_heads) * HEAD_DIM * self.hidden
        per_layer = qkv + self.hidden * self.hidden + 3 * self.ffn * self.hidden + 2 * self.hidden
        return self.layers * per_layer + 2 * self.vocab * self.hidden + self.hidden


MISTRAL_7B = DecoderShape()


@dataclass
class _Layer:
    qkv: Tensor       # [(Hq + 2 Hkv) x 128, hidden]
    o: Tensor         # [hidden, hidden]
    gate_up: Tensor   # [2 ffn, hidden]: gate rows, then up rows
    down: Tensor      # [hidden, ffn]
    in_norm: Tensor
    post_norm: Tensor
    cope: CoPE


class PagedDecoder:
    """Random-init decoder of ``shape``: weights N(0, std) in ``dtype``, norm
    weights 1, CoPE tables N(0, std) in fp32."""

    def __init__(self, shape: DecoderShape, device, *, seed: int = 0, std: float = 0.02,
                 dtype: torch.dtype = torch.bfloat16):
        self.shape, self.device, self.dtype = shape, torch.device(device), dtype
        gen = torch.Generator(device=self.device).manual_seed(seed)

        def normal(*dims, dt=dtype):
            t = torch.empty(dims, dtype=dt, device=self.device)
            return t.normal_(0.0, std, generator=gen)

        s = shape
        self.embed = normal(s.vocab, s.hidden)
        self.layers: list[_Layer] = []
        for _ in range(s.layers):
            cope = CoPE(HEAD_DIM, s.npos, device=self.device)
            with torch.no_grad():
                cope.position_embeddings.copy_(normal(HEAD_DIM, s.npos, dt=torch.float32))
            self.layers.append(_Layer(
                qkv=normal((s.heads + 2 * s.kv_heads) * HEAD_DIM, s.hidden),
                o=normal(s.hidden, s.hidden),
                gate_up=normal(2 * s.ffn, s.hidden),
                down=normal(s.hidden, s.ffn),
                in_norm=torch.ones(s.hidden, dtype=dtype, device=self.device),
                post_norm=torch.ones(s.hidden, dtype=dtype, device=self.device),
                cope=cope,
            ))
        self.norm = torch.ones(s.hidden, dtype=dtype, device=self.device)
        self.lm_head = normal(s.vocab, s.hidden)

    def new_caches(self, num_blocks: int, block_size: int) -> list[Tensor]:
        """One paged cache per layer, [blocks, KV heads, block_size, 2 x 128]."""
        return [torch.empty((num_blocks, self.shape.kv_heads, block_size, 2 * HEAD_DIM), dtype=self.dtype,
                            device=self.device) for _ in range(self.shape.layers)]

    def _rms(self, x: Tensor, weight: Tensor) -> Tensor:
        return F.rms_norm(x, (self.shape.hidden,), weight, self.shape.eps)

    def step(self, ids: Tensor, positions: Tensor, caches: list[Tensor], block_table: Tensor, *,
             max_context: int, workspace: Tensor, flags: Tensor, split: int = 1024,
             attn_out: Tensor | None = None, shared: SharedRuns | None = None) -> Tensor:
        """One token per request: ``ids`` [B] at ``positions`` [B] (int64, the
        request's key count before this token) -> logits [B, vocab].  Writes the
        token's K/V to slot ``block_table[b, p // bs] * bs + p % bs`` of every
        layer's cache; ``max_context`` bounds positions + 1.  With ``shared``
        (runs of blocks the requests share, built on ``block_table``) the
        attention reads each run once for the batch (``ccpe_decode_shared``,
        whose ``workspace`` this then is)."""
        s = self.shape
        b = ids.shape[0]
        bs = caches[0].shape[2]
        slots = block_table.gather(1, (positions // bs).unsqueeze(1)).squeeze(1).long() * bs + positions % bs
        context = (positions + 1).to(torch.int32)
        if attn_out is None:
            attn_out = torch.empty((b, s.heads, HEAD_DIM), dtype=self.dtype, device=self.device)
        stream = _hip.stream_of(self.device)
        lib = _hip.load()
        tail = shared.tail_lens(context) if shared is not None else None
        q_end, k_end = s.heads * HEAD_DIM, (s.heads + s.kv_heads) * HEAD_DIM
        x, residual = self.embed[ids], None
        for layer, cache in zip(self.layers, caches):
            if residual is None:
                residual = x
            else:
                residual = x + residual
            h = self._rms(residual, layer.in_norm)
            qkv = h @ layer.qkv.T
            q = qkv[:, :q_end].view(b, s.heads, HEAD_DIM)
            k = qkv[:, q_end:k_end].view(b, s.kv_heads, HEAD_DIM)
            v = qkv[:, k_end:].view(b, s.kv_heads, HEAD_DIM)
            status = lib.cs_slot_scatter(_hip.vref(cache), _hip.vref(None), _hip.vref(None), _hip.ptr(slots),
                                         _hip.ptr(None), b, _hip.vref(k), _hip.vref(v), stream)
            if status:
                _hip.check(status, "cs_slot_scatter")
            if shared is not None:
                ccpe_decode_shared(q, cache, block_table, context, layer.cope, shared, max_context=max_context,
                                   split=split, tail=tail, workspace=workspace, out=attn_out, flags=flags,
                                   check=False)
            else:
                ccpe_decode_paged(q, cache, block_table, context, layer.cope, max_context=max_context,
                                  split=split, workspace=workspace, out=attn_out, flags=flags, check=False)
            residual = attn_out.view(b, s.hidden) @ layer.o.T + residual
            h = self._rms(residual, layer.post_norm)
            gate, up = (h @ layer.gate_up.T).split(s.ffn, dim=-1)
            x = (F.silu(gate) * up) @ layer.down.T
        return self._rms(x + residual, self.norm) @ self.lm_head.T

    def generate(self, first_ids: Tensor, lengths: Tensor, caches: list[Tensor], block_table: Tensor,
                 steps: int, *, max_context: int, split: int = 1024, check: bool = True,
                 shared: SharedRuns | None = None) -> Tensor:
        """Greedy decoding of ``steps`` tokens per request after contexts of
        ``lengths`` keys -> token ids [steps, B] (on the device); ``shared`` as
        in ``step``."""
        b = first_ids.shape[0]
        if shared is not None:
            workspace = decode_shared_workspace(b, self.shape.heads, shared, max_context, split, self.device)
        else:
            workspace = decode_workspace(b, self.shape.heads, max_context, split, self.device)
        flags = _hip.new_flags(self.device)
        attn_out = torch.empty((b, self.shape.heads, HEAD_DIM), dtype=self.dtype, device=self.device)
        out = torch.empty((steps, b), dtype=torch.long, device=self.device)
        ids, positions = first_ids, lengths.to(torch.long).clone()
        for t in range(steps):
            logits = self.step(ids, positions, caches, block_table, max_context=max_context,
                               workspace=workspace, flags=flags, split=split, attn_out=attn_out, shared=shared)
            ids = logits.argmax(dim=-1)
            out[t] = ids
            positions += 1
        if check:
            raise_flags(flags)
        return out
