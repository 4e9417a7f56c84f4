"""Shared driver of the tiny end-to-end runs: request plans and the generation
loop the reference's CPU smoke uses (src/cacheslide_vllm/workflow_smoke.py:
117-324), run against either runtime (this package's or the oracle's)."""

from __future__ import annotations

import hashlib
from dataclasses import replace

import numpy as np
import torch

from cacheslide_amd import CoPE, NativePagedKV, PageStore, cope_attention
from cacheslide_amd.contracts import RequestPlan
from cacheslide_amd.policy import WCAConfig
from cacheslide_amd.profiles import ProfileBundle, calibrate_from_forward
from cacheslide_amd.selective import RuntimeOptions, SelectiveRuntime
from tests._tiny_decoder import HEAD_DIM, HEADS, HIDDEN, KV_HEADS, NPOS, TinyDecoder

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


IDENTITY = hashlib.sha256(b"tiny-e2e").hexdigest()
BLOCK = 4


def cope_factory(device):
    def make(table):
        cope = CoPE(HEAD_DIM, NPOS, device=device)
        with torch.no_grad():
            cope.position_embeddings.copy_(table)
        return cope
    return make


class BlockPool:
    """Paged caches per layer ([blocks, KV heads, 4, 2 x 16], a strided view
    like the reference smoke's) and one reversed block table for every arena."""

    def __init__(self, layers: int, capacity: int, device):
        blocks = (capacity + BLOCK - 1) // BLOCK
        self.row = list(reversed(range(blocks)))
        self.caches = [torch.full((blocks, KV_HEADS, BLOCK, 4 * HEAD_DIM), -999.0, device=device)[..., ::2]
                       for _ in range(layers)]

    def __call__(self, layer, prompt_length, max_selected, *, existing=None):
        if existing is not None:
            existing.update_block_table(self.row)
            return existing
        return NativePagedKV(self.caches[layer], self.row, prompt_length, max_selected,
                             request_id="tiny", layer_index=layer)


def calibrated_profiles(device, plan, layers, tmp_path):
    model = TinyDecoder(device, None, cope_factory=cope_factory(device), layers=layers)

    def forward(p, observer):
        def handler(layer, positions, q, k, v, cope):
            observer(layer, q, k, cope)
            return cope_attention(q, k, v, cope, positions, key_positions=positions, query_chunk_size=64)
        model.handler = handler
        model.forward(torch.tensor(p.token_ids))

    path = calibrate_from_forward(forward, [plan], tmp_path / "profiles", adapter_identity=IDENTITY,
                                  num_layers=layers, query_heads=HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM,
                                  max_positions=NPOS)
    return ProfileBundle(path, IDENTITY, max_elements=1_000_000)


def device_runtimes(device, tmp_path, plan, layers, calibration_layer, paged=True, tag="a",
                    wca=WCAConfig()):
    store = PageStore(tmp_path / f"pages-{tag}", cpu_budget_bytes=1 << 26, disk_budget_bytes=1 << 28)
    profiles = calibrated_profiles(device, plan, layers, tmp_path / tag)
    pool = BlockPool(layers, len(plan.token_ids) + 64, device) if paged else None
    out = {}
    for mode in ("strict_contextual", "mixed_bias_override"):
        options = RuntimeOptions(calibration_layer=calibration_layer, wca=wca, ccpe_position_policy=mode)
        rt = SelectiveRuntime(layers=layers, kv_heads=KV_HEADS, head_dim=HEAD_DIM, hidden_size=HIDDEN,
                              store=store, profiles=profiles, identity=IDENTITY, checkpoint_id=IDENTITY,
                              options=options, arena_factory=pool)
        model = TinyDecoder(device, rt.attention, cope_factory=cope_factory(device), layers=layers)
        out[mode] = (rt, model)
    return store, out


def oracle_runtimes(plan, layers, calibration_layer, wca=WCAConfig()):
    from oracle.runtime import OracleRuntime

    out = {}
    shared = None
    for mode in ("strict_contextual", "mixed_bias_override"):
        rt = OracleRuntime(layers=layers, identity=IDENTITY,
                           options=RuntimeOptions(calibration_layer=calibration_layer, ccpe_position_policy=mode),
                           fraction=wca.correction_fraction, gate_interval=wca.gate_interval,
                           threshold=wca.convergence_threshold, mode=wca.convergence_mode)
        if shared is None:
            shared = rt
        else:
            rt.store, rt.profiles = shared.store, shared.profiles
        out[mode] = (rt, TinyDecoder("cpu", rt.attention, layers=layers))
    shared_rt, shared_model = out["strict_contextual"]
    shared_rt.calibrate(shared_model, plan)
    return out


CASES = [("populate", 32, "strict_contextual"), ("recompute", 32, "strict_contextual"),
         ("reuse", 32, "strict_contextual"), ("reuse", 40, "strict_contextual"),
         ("reuse", 40, "mixed_bias_override")]


def run_cases(runtimes, cases=CASES):
    results = []
    for i, (op, dyn, mode) in enumerate(cases):
        rt, model = runtimes[mode]
        results.append(invoke(rt, model, tiny_plan(dyn), op, f"req-{i}"))
    return results
