"""The oracle restatement of the runtime's call order, on the CPU: the
reference smoke's decisions for the tiny decoder (config-1 workload) --
population, same-context reuse, a shifted non-prefix chunk under strict CCPE
(fallback) and under mixed_bias_override (reuse) -- and the reference's own
logit checks of those cases (src/cacheslide_vllm/workflow_smoke.py:253-263,
302-306)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from oracle.runtime import OracleRuntime
from tests._e2e import invoke, tiny_plan
from tests._tiny_decoder import TinyDecoder

IDENTITY = "0" * 64


@dataclass(frozen=True)
class Opts:
    query_chunk_size: int = 64
    calibration_layer: int = 0
    selected_attention: str = "updated_and_self"
    ccpe_position_policy: str = "strict_contextual"


def oracle_setup(layers=2, calibration_layer=0):
    strict = OracleRuntime(layers=layers, identity=IDENTITY, options=Opts(calibration_layer=calibration_layer),
                           fraction=0.26)
    mixed = OracleRuntime(layers=layers, identity=IDENTITY,
                          options=Opts(calibration_layer=calibration_layer, ccpe_position_policy="mixed_bias_override"),
                          fraction=0.26)
    mixed.store, mixed.profiles = strict.store, strict.profiles
    model_s = TinyDecoder("cpu", strict.attention, layers=layers)
    model_m = TinyDecoder("cpu", mixed.attention, layers=layers)
    return strict, mixed, model_s, model_m


def test_tiny_decoder_smoke_decisions_on_the_oracle():
    strict, mixed, model_s, model_m = oracle_setup()
    plan, shifted = tiny_plan(32), tiny_plan(40)
    strict.calibrate(model_s, plan)
    _, _, pop = invoke(strict, model_s, plan, "populate", "p")
    assert not pop["cache_hit"] and pop["layer_rows"] == [97, 97]
    base, base_ids, _ = invoke(strict, model_s, plan, "recompute", "b")
    reuse, reuse_ids, rec = invoke(strict, model_s, plan, "reuse", "r")
    assert rec["cache_hit"] and not rec["fallback"]
    assert rec["computed_token_layers"] < rec["dense_token_layers"]
    torch.testing.assert_close(reuse, base, atol=3e-6, rtol=3e-6)     # workflow_smoke.py:302-306
    first, _, sh = invoke(strict, model_s, shifted, "reuse", "s")
    assert sh["position_policy_fallback"] and sh["fallback"] and not sh["cache_hit"]
    dense = model_s.logits(model_s.forward(torch.tensor(shifted.token_ids)))[-1]
    torch.testing.assert_close(first, dense, atol=3e-6, rtol=3e-6)    # workflow_smoke.py:253-263
    _, _, mx = invoke(mixed, model_m, shifted, "reuse", "m")
    assert mx["cache_hit"] and not mx["fallback"] and not mx["position_policy_fallback"]
