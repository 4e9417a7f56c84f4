"""Shared driver of the tiny end-to-end runs: request plans and the generation
loop the reference's CPU smoke uses (src/cacheslide_vllm/workflow_smoke.py:
117-324), run against either runtime (this package's or the oracle's)."""

from __future__ import annotations

from dataclasses import replace

import numpy as np
import torch

from cacheslide_amd.contracts import RequestPlan

VOCAB = 512


def tiny_plan(dynamic: int = 32, *, seed: int = 11) -> RequestPlan:
    """Reused chunk A (32 ids), a recomputed chunk (``dynamic`` ids), reused
    chunk B (32 ids) and the recomputed query token, ids uniform in [0, 512).
    A and B are the same for every ``dynamic``; the recomputed chunk differs."""
    rng = np.random.default_rng(seed)
    a, b = rng.integers(0, VOCAB, 32).tolist(), rng.integers(0, VOCAB, 32).tolist()
    query = rng.integers(0, VOCAB, 1).tolist()
    dyn = np.random.default_rng(seed + dynamic).integers(0, VOCAB, dynamic).tolist()
    tokens = a + dyn + b + query
    split = 32 + dynamic
    return RequestPlan.parse(
        {"version": 1, "operation": "recompute", "namespace": "tiny-e2e", "task_id": "synthetic",
         "chunks": [{"id": "A", "role": "reuse", "start": 0, "end": 32},
                    {"id": "dynamic", "role": "recompute", "start": 32, "end": split},
                    {"id": "B", "role": "reuse", "start": split, "end": split + 32},
                    {"id": "query", "role": "recompute", "start": split + 32, "end": len(tokens)}]},
        tokens,
    )


RECEIPT_KEYS = ("cache_hit", "fallback", "position_policy_fallback", "layer_rows", "restored_rows",
                "decode_tokens", "computed_token_layers", "dense_token_layers")


def invoke(runtime, model, plan: RequestPlan, operation: str, request_id: str, decode_steps: int = 5):
    """Prefill, the first greedy token, then ``decode_steps`` greedy decode
    steps; returns (first-token logits on the CPU, generated ids, receipts)."""
    request = replace(plan, operation=operation)
    device = model.device
    ids = torch.tensor(request.token_ids)
    n = len(ids)
    hidden = runtime.run(model, model.embed(ids), torch.arange(n, device=device), request_id, request)
    first = model.logits(hidden)[-1].detach().cpu().clone()
    generated = [int(first.argmax())]
    for offset in range(decode_steps):
        hidden = runtime.run(model, model.embed(torch.tensor([generated[-1]])),
                             torch.tensor([n + offset], device=device), request_id, request)
        logits = model.logits(hidden)[-1]
        assert bool(torch.isfinite(logits).all())
        generated.append(int(logits.argmax()))
    receipts = {key: runtime.last_metrics.get(key) for key in RECEIPT_KEYS}
    if hasattr(runtime, "release"):
        runtime.release(request_id)
    return first, generated, receipts
