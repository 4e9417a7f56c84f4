"""CCPE calibration on the MI355X into the profile artifact format.

``calibrate_from_forward`` drives a seeded stand-in model forward; each layer's
device trace is projected onto the fixed tokens and calibrated on the device.
The loaded canonical table must equal the oracle's contextual positions of the
full context (position.py:295-307) at the fixed x fixed cells, renumbered to
ordinals (position.py:196-272), and identical samples keep that pattern
(position.py:594-699).
"""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from cacheslide_amd import CoPE, RequestPlan
from cacheslide_amd.profiles import ProfileBundle, calibrate_from_forward
from oracle import ccpe as orc

pytestmark = pytest.mark.gpu

ADAPTER = hashlib.sha256(b"trained adapter").hexdigest()
LAYERS, HQ, HKV, D, P = 3, 4, 2, 16, 8


def plan(tokens):
    doc = {"version": 1, "operation": "calibrate", "namespace": "ns", "task_id": "t",
           "chunks": [{"id": "sys", "role": "reuse", "start": 0, "end": 16},
                      {"id": "doc", "role": "reuse", "start": 16, "end": 30},
                      {"id": "q", "role": "recompute", "start": 30, "end": len(tokens)}]}
    return RequestPlan.parse(doc, tokens)


def layer_qk(p: RequestPlan, layer: int):
    """Seeded Q/K of a layer: a function of the full prompt, on the CPU."""
    seed = int(hashlib.sha256(repr((p.token_ids, layer)).encode()).hexdigest()[:8], 16)
    g = torch.Generator().manual_seed(seed)
    t = len(p.token_ids)
    return torch.randn(t, HQ, D, generator=g) * 2, torch.randn(t, HKV, D, generator=g) * 2


def test_calibrate_from_forward_matches_oracle_and_loads(device, tmp_path):
    cope = CoPE(D, P, device=device)
    base = list(range(100, 140))
    requests = [plan(base), plan(base), plan(base[:30] + [7] * 12)]   # two identical, one other query
    calls = []

    def forward(p, observer):
        calls.append(len(p.token_ids))
        for layer in range(LAYERS):
            q, k = layer_qk(p, layer)
            observer(layer, q.to(device), k.to(device), cope)

    out = calibrate_from_forward(forward, requests, tmp_path / "profiles", adapter_identity=ADAPTER,
                                 num_layers=LAYERS, query_heads=HQ, kv_heads=HKV, head_dim=D,
                                 max_positions=P, max_elements=10_000_000)
    assert calls == [40, 40, 42]
    bundle = ProfileBundle(out, ADAPTER, max_elements=10_000_000)
    fixed = np.arange(30)
    for layer in range(LAYERS):
        # the three requests share the fixed layout, so one profile key per layer;
        # the two identical requests give the modal pattern
        profile = bundle.get(requests[0], layer)
        assert profile.sample_count == 3
        q, k = layer_qk(requests[0], layer)
        n = len(requests[0].token_ids)
        lg = orc.logits(q.numpy().astype(np.float32), k.numpy().astype(np.float32))
        allowed = orc.allowed_mask(np.arange(n), np.arange(n), HQ)
        full = orc.contextual_positions(lg, allowed, P)
        expected = full[:, fixed][:, :, fixed]
        np.testing.assert_allclose(profile.canonical_positions.numpy(), expected, atol=1e-4, rtol=1e-5)
        assert torch.equal(profile.query_positions, torch.arange(30))


def test_calibration_rejects_bad_observers_and_budgets(device, tmp_path):
    cope = CoPE(D, P, device=device)
    p = plan(list(range(40)))
    kwargs = dict(adapter_identity=ADAPTER, num_layers=LAYERS, query_heads=HQ, kv_heads=HKV, head_dim=D,
                  max_positions=P, max_elements=10_000_000)

    def repeated(p_, observer):
        q, k = layer_qk(p_, 0)
        observer(0, q.to(device), k.to(device), cope)
        observer(0, q.to(device), k.to(device), cope)

    with pytest.raises(ValueError, match="invalid/repeated layer"):
        calibrate_from_forward(repeated, [p], tmp_path / "a", **kwargs)

    def partial(p_, observer):
        q, k = layer_qk(p_, 0)
        observer(0, q.to(device), k.to(device), cope)

    with pytest.raises(ValueError, match="did not observe every attention layer"):
        calibrate_from_forward(partial, [p], tmp_path / "b", **kwargs)

    def wrong_shape(p_, observer):
        q, k = layer_qk(p_, 0)
        observer(0, q[:, :2].to(device), k.to(device), cope)

    with pytest.raises(ValueError, match="Q/K layout mismatch"):
        calibrate_from_forward(wrong_shape, [p], tmp_path / "c", **kwargs)
    # 3 layers x 4 heads x (40^2 + 30^2) + 3 x (4 x 30^2 + 60) > 1000
    with pytest.raises(ValueError, match="source traces exceed max_elements budget"):
        calibrate_from_forward(repeated, [p], tmp_path / "d", **{**kwargs, "max_elements": 1000})
    with pytest.raises(ValueError, match="at least one request"):
        calibrate_from_forward(repeated, [], tmp_path / "e", **kwargs)
    assert not any((tmp_path / name).exists() for name in "abcde")
