"""A tiny random CoPE decoder: the caller's model in the end-to-end runs.

Llama-shaped like the reference's CPU smoke model (src/cacheslide_vllm/
reference.py:35-200): RMSNorm with a fused residual, q/k/v and o projections,
a SiLU-gated MLP, a final norm and an LM head, with a learned CoPE table per
layer and the attention computed by a pluggable handler
``handler(layer, positions, q, k, v, cope)``.  The workload: 2 layers (more
for deeper checks),
d_model 64, 4 query and 4 KV heads x 16, MLP 256, vocab 512, CoPE P = 64,
float32 weights ~ N(0, 0.02) from one seed.  The same weights run on the CPU
(oracle runs) and on the device.
"""

from __future__ import annotations

import torch
from torch import Tensor

LAYERS, HIDDEN, HEADS, KV_HEADS, HEAD_DIM, MLP, VOCAB, NPOS = 2, 64, 4, 4, 16, 256, 512, 64
EPS = 1e-6


class TinyCope:
    """What the handlers need of a CoPE module: the table and its size."""

    def __init__(self, table: Tensor):
        self.position_embeddings = table
        self.max_positions = table.shape[1]
        self.head_dim = table.shape[0]


def weights(seed: int = 92, layers: int = LAYERS) -> dict[str, Tensor]:
    g = torch.Generator().manual_seed(seed)
    w = lambda *shape: torch.randn(shape, generator=g) * 0.02  # noqa: E731
    out = {"embed": w(VOCAB, HIDDEN), "norm": 1 + w(HIDDEN), "lm_head": w(VOCAB, HIDDEN)}
    for i in range(layers):
        out[f"{i}.qkv"] = w((HEADS + 2 * KV_HEADS) * HEAD_DIM, HIDDEN)
        out[f"{i}.o"] = w(HIDDEN, HEADS * HEAD_DIM)
        out[f"{i}.gate_up"] = w(2 * MLP, HIDDEN)
        out[f"{i}.down"] = w(HIDDEN, MLP)
        out[f"{i}.in_norm"] = 1 + w(HIDDEN)
        out[f"{i}.post_norm"] = 1 + w(HIDDEN)
        out[f"{i}.cope"] = w(HEAD_DIM, NPOS)
    return out


def rms_norm(x: Tensor, weight: Tensor, residual: Tensor | None = None):
    """reference.py:45-61: normalise (hidden + residual), return it and the sum."""
    combined = x if residual is None else x + residual
    normalized = combined * torch.rsqrt(combined.square().mean(-1, keepdim=True) + EPS) * weight
    return normalized if residual is None else (normalized, combined)


class Layer:
    def __init__(self, model: "TinyDecoder", index: int):
        self.model, self.index = model, index

    def __call__(self, positions: Tensor, hidden: Tensor, residual: Tensor | None):
        """reference.py:170-186 (vLLM-style fused residual)."""
        w, i = self.model.w, self.index
        if residual is None:
            residual = hidden
            hidden = rms_norm(hidden, w[f"{i}.in_norm"])
        else:
            hidden, residual = rms_norm(hidden, w[f"{i}.in_norm"], residual)
        qkv = hidden @ w[f"{i}.qkv"].T
        q, k, v = qkv.split((HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM, KV_HEADS * HEAD_DIM), dim=-1)
        q = q.reshape(-1, HEADS, HEAD_DIM).contiguous()
        k = k.reshape(-1, KV_HEADS, HEAD_DIM).contiguous()
        v = v.reshape(-1, KV_HEADS, HEAD_DIM).contiguous()
        attention = self.model.handler(i, positions, q, k, v, self.model.copes[i])
        hidden = attention.reshape(hidden.shape[0], HEADS * HEAD_DIM) @ w[f"{i}.o"].T
        hidden, residual = rms_norm(hidden, w[f"{i}.post_norm"], residual)
        gate, up = (hidden @ w[f"{i}.gate_up"].T).chunk(2, dim=-1)
        return (torch.nn.functional.silu(gate) * up) @ w[f"{i}.down"].T, residual


class TinyDecoder:
    """``cope_factory(table)`` builds each layer's CoPE module (on the device,
    the package's ``CoPE`` holding the table; on the CPU, ``TinyCope``)."""

    def __init__(self, device, handler, seed: int = 92, cope_factory=TinyCope, layers: int = LAYERS):
        self.w = {name: t.to(device) for name, t in weights(seed, layers).items()}
        self.device = torch.device(device)
        self.handler = handler
        self.layers = [Layer(self, i) for i in range(layers)]
        self.copes = [cope_factory(self.w[f"{i}.cope"]) for i in range(layers)]

    def embed(self, ids: Tensor) -> Tensor:
        return self.w["embed"][ids.to(self.device)]

    def norm(self, hidden: Tensor, residual: Tensor | None):
        if residual is None:
            return rms_norm(hidden, self.w["norm"]), None
        return rms_norm(hidden, self.w["norm"], residual)

    def logits(self, hidden: Tensor) -> Tensor:
        return hidden @ self.w["lm_head"].T

    def forward(self, ids: Tensor, observer=None) -> Tensor:
        """Full dense forward (every row, every layer) -> final hidden rows."""
        positions = torch.arange(len(ids), device=self.device)
        hidden, residual = self.embed(ids), None
        for layer in self.layers:
            hidden, residual = layer(positions, hidden, residual)
        return self.norm(hidden, residual)[0]
