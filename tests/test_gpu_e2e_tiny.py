"""End to end on the tiny random decoder (2 layers, d_model 64, 4 heads x 16,
vocab 512, CoPE P = 64, fp32 weights ~ N(0, 0.02)): profiles calibrated from
the model's own forward (no adapter), population of the layer pages, then
same-context reuse, a shifted non-prefix chunk under strict CCPE (the
reference falls back to plain CoPE) and under mixed_bias_override (reused),
each followed by 5 greedy decode steps -- the reference's CPU smoke flow
(src/cacheslide_vllm/workflow_smoke.py:117-324) driving this package's
``SelectiveRuntime`` on the device, with SLIDE arenas on paged caches.

Checked against the oracle runtime (oracle/runtime.py) driven the same way on
the CPU: every decision (hit, fallback, strict-CCPE fallback, rows per layer,
restored rows) identical, first-token logits within 1e-4, the same greedy
tokens.  Also the reference's own checks: the reused logits equal the
recomputed ones and the strict fallback equals the dense forward
(workflow_smoke.py:253-263, 302-306); paged equals dense bit for bit
(tests/test_runtime_paged.py:62-181).
"""

from __future__ import annotations

import pytest
import torch

from cacheslide_amd.policy import WCAConfig
from tests._e2e import CASES, device_runtimes, oracle_runtimes, run_cases, tiny_plan

pytestmark = pytest.mark.gpu


def test_tiny_decoder_end_to_end_matches_oracle(device, tmp_path):
    plan = tiny_plan(32)
    store, ours = device_runtimes(device, tmp_path, plan, layers=2, calibration_layer=0)
    theirs = oracle_runtimes(plan, layers=2, calibration_layer=0)
    got, want = run_cases(ours), run_cases(theirs)
    for (op, dyn, mode), (g_first, g_ids, g_rec), (w_first, w_ids, w_rec) in zip(CASES, got, want):
        assert g_rec == w_rec, (op, dyn, mode, g_rec, w_rec)
        torch.testing.assert_close(g_first, w_first, atol=1e-4, rtol=1e-3)
        assert g_ids == w_ids, (op, dyn, mode)
    receipts = [r for _, _, r in got]
    assert not receipts[0]["cache_hit"]                                                  # populate
    assert receipts[2]["cache_hit"] and not receipts[2]["fallback"]                      # same context
    assert receipts[2]["computed_token_layers"] < receipts[2]["dense_token_layers"]
    assert receipts[3]["position_policy_fallback"] and not receipts[3]["cache_hit"]      # shifted, strict
    assert receipts[4]["cache_hit"] and not receipts[4]["position_policy_fallback"]      # shifted, mixed
    # the reference's own checks of these cases
    torch.testing.assert_close(got[2][0], got[1][0], atol=3e-6, rtol=3e-6)
    rt, model = ours["strict_contextual"]
    dense = model.logits(model.forward(torch.tensor(tiny_plan(40).token_ids)))[-1].cpu()
    torch.testing.assert_close(got[3][0], dense, atol=3e-6, rtol=3e-6)
    for rt, _ in ours.values():
        rt.close()
    store.close()


def test_paged_runtime_equals_dense_runtime_bit_for_bit(device, tmp_path):
    plan = tiny_plan(32)
    store_p, paged = device_runtimes(device, tmp_path, plan, layers=2, calibration_layer=0, tag="p")
    store_d, dense = device_runtimes(device, tmp_path, plan, layers=2, calibration_layer=0, paged=False, tag="d")
    for (op, dyn, mode), a, b in zip(CASES, run_cases(paged), run_cases(dense)):
        assert torch.equal(a[0], b[0]), (op, dyn, mode)
        assert a[1] == b[1] and a[2] == b[2]
    for rts in (paged, dense):
        for rt, _ in rts.values():
            rt.close()
    store_p.close()
    store_d.close()


def test_deeper_decoder_exercises_wca_rows_and_restores(device, tmp_path):
    """Six layers (the reference smoke's depth) with WCA calibrated at layer 1
    and the distance gate: after a shifted chunk the fixed tokens' layer-1 keys
    deviate, WCA selects rows, the gate of layer 3 removes converged rows and
    promotes others, and the promoted rows are restored from the layer-input
    snapshots before layer 4."""
    plan = tiny_plan(32)
    wca = WCAConfig(convergence_mode="distance_lt")
    cases = [("populate", 32, "strict_contextual"), ("reuse", 40, "mixed_bias_override"),
             ("reuse", 24, "mixed_bias_override")]
    store, ours = device_runtimes(device, tmp_path, plan, layers=6, calibration_layer=1, tag="w", wca=wca)
    theirs = oracle_runtimes(plan, layers=6, calibration_layer=1, wca=wca)
    got, want = run_cases(ours, cases), run_cases(theirs, cases)
    for case, (g_first, g_ids, g_rec), (w_first, w_ids, w_rec) in zip(cases, got, want):
        assert g_rec == w_rec, (case, g_rec, w_rec)
        torch.testing.assert_close(g_first, w_first, atol=1e-4, rtol=1e-3)
        assert g_ids == w_ids, case
    shifted = got[1][2]
    assert shifted["cache_hit"] and shifted["layer_rows"][2] < shifted["layer_rows"][0]
    assert shifted["restored_rows"] > 0
    for rt, _ in ours.values():
        rt.close()
    store.close()
