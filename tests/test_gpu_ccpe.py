"""CCPE attention on the MI355X kernels vs the reference's known answers and the oracle.

Known answers are transcribed from tests/test_position.py and
tests/test_attention_policies.py of the reference (cited per test) and run
through this package's drop-in API on the device.  Seeded random cases compare
the generic kernel, the MFMA prefill kernel (dense and paged) and the split-K
decode kernel with oracle/ccpe.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd import (
    CCPEPositionError,
    CCPEProfile,
    CanonicalPositionPolicy,
    ChunkIdentity,
    CoPE,
    RequestPlan,
    SelectedAssociationPolicy,
    cope_attention,
    validate_contextual_path,
)
from cacheslide_amd.ccpe import ccpe_decode_paged, ccpe_prefill_paged
from oracle import ccpe as orc
from tests._helpers import acc_np, assert_close_bf16, fill_paged, paged_layout, seeded, tolerance

pytestmark = pytest.mark.gpu


def cope_on(device, head_dim, npos, dtype=torch.float32, table=None):
    cope = CoPE(head_dim, npos, device=device, dtype=dtype)
    if table is not None:
        with torch.no_grad():
            cope.position_embeddings.copy_(torch.as_tensor(table, dtype=dtype))
    return cope


# ------------------------------------------------------------ known answers
def test_gate_masking_reverse_cumsum_and_clamp(device):
    # tests/test_position.py:16-23
    cope = CoPE(2, 2, device=device)
    logits = torch.zeros(1, 3, 3, device=device)
    allowed = torch.ones(3, 3, dtype=torch.bool, device=device).tril().unsqueeze(0)
    logits[~allowed] = 1000
    positions = cope.contextual_positions(logits, allowed)
    expected = torch.tensor([[[0.5, 0, 0], [1, 0.5, 0], [1, 1, 0.5]]])
    torch.testing.assert_close(positions.cpu(), expected)


def test_interpolation_known_answer(device):
    # tests/test_position.py:26-35
    cope = cope_on(device, 1, 4, torch.float64, [[0, 2, 6, 10]])
    query = torch.tensor([[[2.0]]], dtype=torch.float64, device=device)
    positions = torch.tensor([[[0.25, 1.5, 3.0]]], dtype=torch.float64, device=device)
    bias = cope.positional_bias(query, positions)
    torch.testing.assert_close(bias.cpu(), torch.tensor([[[1, 8, 20]]], dtype=torch.float64))


def test_linear_table_bias_equals_position(device):
    # tests/test_position.py:48-62
    cope = cope_on(device, 1, 4, torch.float64, torch.arange(4.0)[None])
    query = torch.ones(1, 1, 1, dtype=torch.float64, device=device)
    positions = torch.tensor([[[1.0, 2.0, 3.0]]], dtype=torch.float64, device=device)
    torch.testing.assert_close(cope.positional_bias(query, positions), positions)


def test_two_causal_gates_give_position_one(device):
    # tests/test_position.py:65-77
    cope = cope_on(device, 1, 4, torch.float64, torch.arange(4.0)[None])
    query = torch.ones(1, 1, 1, dtype=torch.float64, device=device)
    key = torch.zeros(3, 1, 1, dtype=torch.float64, device=device)
    bias = cope(query, key, torch.tensor([1], device=device))
    assert bias[0, 0, 0].item() == 1


def test_gqa_chunking_arbitrary_rows_and_decode(device):
    # tests/test_position.py:99-115 against the textbook loop
    torch.manual_seed(3)
    e = torch.randn(3, 7, dtype=torch.float64)
    q = torch.randn(3, 4, 3, dtype=torch.float64)
    k = torch.randn(6, 2, 3, dtype=torch.float64)
    v = torch.randn(6, 2, 5, dtype=torch.float64)
    qpos, kpos = np.array([4, 1, 5]), np.arange(6)
    expected = orc.dense_reference(q.numpy(), k.numpy(), v.numpy(), e.numpy(), qpos, kpos, 7)
    cope = cope_on(device, 3, 7, torch.float64, e)
    actual, positions = cope_attention(
        q.to(device), k.to(device), v.to(device), cope, torch.tensor(qpos, device=device),
        query_chunk_size=1, return_positions=True,
    )
    np.testing.assert_allclose(actual.cpu().numpy(), expected, rtol=1e-10, atol=1e-10)
    assert positions.shape == (4, 3, 6)
    decode = cope_attention(q[-1:].to(device), k.to(device), v.to(device), cope,
                            torch.tensor([5], device=device))
    np.testing.assert_allclose(decode.cpu().numpy(), expected[-1:], rtol=1e-10, atol=1e-10)


def test_future_keys_values_do_not_change_earlier_output(device):
    # tests/test_position.py:118-128
    torch.manual_seed(8)
    cope = cope_on(device, 2, 6, table=torch.randn(2, 6))
    q, k, v = [torch.randn(4, 2, 2, device=device) for _ in range(3)]
    original = cope_attention(q, k, v, cope, torch.arange(4, device=device))
    k[2:] *= -100
    v[2:] += 100
    changed = cope_attention(q, k, v, cope, torch.arange(4, device=device))
    torch.testing.assert_close(changed[:2], original[:2])


def test_all_masked_rows_zero_and_errors(device):
    # tests/test_position.py:131-143
    cope = CoPE(2, 4, device=device)
    q, k, v = [torch.ones(2, 1, 2, device=device) for _ in range(3)]
    mask = torch.tensor([[False, False], [True, True]], device=device)
    output = cope_attention(q, k, v, cope, torch.arange(2, device=device), attention_mask=mask)
    assert output[0].abs().sum() == 0
    assert torch.isfinite(output).all()
    with pytest.raises(ValueError, match="query-dependent"):
        cope_attention(q, k, v, cope, torch.arange(2, device=device),
                       fixed_positions=torch.arange(2, device=device))
    with pytest.raises(ValueError, match="strictly increasing"):
        cope(q, k, torch.arange(2, device=device), torch.tensor([1, 0], device=device))
    with pytest.raises(ValueError, match="finite"):
        cope(q * torch.nan, k, torch.arange(2, device=device))


def test_association_visibility_preserves_gate_counts(device):
    # tests/test_position.py:146-171
    cope = CoPE(1, 8, device=device)
    q, k = torch.ones(1, 1, 1, device=device), torch.zeros(3, 1, 1, device=device)
    v = torch.tensor([1.0, 10.0, 100.0], device=device)[:, None, None]
    visibility = torch.tensor([[True, False, True]], device=device)
    output, trace = cope_attention(q, k, v, cope, torch.tensor([2], device=device),
                                   visibility_mask=visibility, return_positions=True)
    assert output.item() == 50.5
    torch.testing.assert_close(trace.cpu(), torch.tensor([[[1.5, 1.0, 0.5]]]))
    _, masked = cope_attention(q, k, v, cope, torch.tensor([2], device=device),
                               attention_mask=visibility, return_positions=True)
    assert masked[0, 0, 0] == 1


def test_contextual_path_accepts_genuine_ignores_future(device):
    # tests/test_position.py:174-187
    cope = CoPE(2, 3, device=device)
    q = torch.ones(3, 4, 2, device=device)
    k = torch.zeros(5, 2, 2, device=device)
    qpos, kpos = torch.tensor([4, 0, 2], device=device), torch.arange(5, device=device)
    trace = cope.position_trace(q, k, qpos, checkpoint_id="trained")
    positions = trace.positions.to(device)
    validate_contextual_path(positions, qpos, kpos)
    positions = positions.masked_fill(~trace.allowed_mask.to(device), 0.75)
    validate_contextual_path(positions, qpos, kpos)
    positions[0, 1, 0] = 1.1
    with pytest.raises(CCPEPositionError, match="available gates"):
        validate_contextual_path(positions, qpos, kpos)


def test_contextual_path_rejects_hybrid(device):
    # tests/test_position.py:190-209
    cope = CoPE(1, 16, device=device)
    old = cope.position_trace(torch.ones(3, 1, 1, device=device), torch.zeros(3, 1, 1, device=device),
                              torch.arange(3, device=device), checkpoint_id="trained")
    canonical = old.project(torch.tensor([0, 2]), torch.tensor([0, 2]))
    current = cope.position_trace(torch.ones(1, 1, 1, device=device), torch.zeros(5, 1, 1, device=device),
                                  torch.tensor([4], device=device), checkpoint_id="trained")
    hybrid = current.positions.clone()
    hybrid[:, 0, [0, 4]] = canonical.positions[:, 1]
    torch.testing.assert_close(hybrid, torch.tensor([[[1.5, 2, 1.5, 1, 0.5]]]))
    with pytest.raises(CCPEPositionError, match="nonincreasing"):
        validate_contextual_path(hybrid.to(device), torch.tensor([4], device=device),
                                 torch.arange(5, device=device))


def test_contextual_path_sparse_coordinates_and_masks(device):
    # tests/test_position.py:212-226
    d = device
    validate_contextual_path(torch.tensor([[[2.25, 0.5]]], device=d), torch.tensor([2], device=d),
                             torch.tensor([0, 2], device=d))
    with pytest.raises(CCPEPositionError, match="one gate per token"):
        validate_contextual_path(torch.tensor([[[2.75, 0.5]]], device=d), torch.tensor([2], device=d),
                                 torch.tensor([0, 2], device=d))
    validate_contextual_path(torch.tensor([[[1, 99, 0.5]]], device=d), torch.tensor([2], device=d),
                             torch.arange(3, device=d),
                             attention_mask=torch.tensor([[True, False, True]], device=d))


def test_contextual_path_binade_roundoff(device):
    # tests/test_position.py:229-237
    cope = CoPE(1, 256, device=device)
    logits = torch.tensor([100.0] * 128 + [-11.5], device=device)[None, None]
    positions = cope.contextual_positions(logits, torch.ones_like(logits, dtype=torch.bool))
    assert (positions[..., :-1] - positions[..., 1:]).max() > 1 + 1e-6
    validate_contextual_path(positions, torch.tensor([128], device=device), torch.arange(129, device=device))


@pytest.mark.parametrize("case", range(6))
def test_contextual_path_error_types(device, case):
    # tests/test_position.py:240-260
    d = device
    cases = [
        (torch.ones(1, 1, 2, dtype=torch.long, device=d), torch.tensor([1], device=d), torch.arange(2, device=d), {}),
        (torch.full((1, 1, 2), torch.nan, device=d), torch.tensor([1], device=d), torch.arange(2, device=d), {}),
        (torch.ones(1, 1, 2, device=d), torch.tensor([1.0], device=d), torch.arange(2, device=d), {}),
        (torch.ones(1, 1, 2, device=d), torch.tensor([1], device=d), torch.tensor([1, 0], device=d), {}),
        (torch.ones(1, 1, 2, device=d), torch.tensor([1], device=d), torch.arange(2, device=d), {"atol": -1}),
        (torch.ones(1, 1, 2, device=d), torch.tensor([1], device=d), torch.arange(2, device=d),
         {"attention_mask": torch.ones(1, 2, device=d)}),
    ]
    positions, qpos, kpos, kwargs = cases[case]
    with pytest.raises(CCPEPositionError):
        validate_contextual_path(positions, qpos, kpos, **kwargs)


def test_chunk_transforms_match_precomputed(device):
    # tests/test_position.py:263-322 (forward parity and callback order)
    torch.manual_seed(29)
    cope = cope_on(device, 2, 8, torch.float64, torch.randn(2, 8, dtype=torch.float64))
    q = torch.randn(3, 4, 2, dtype=torch.float64, device=device)
    k = torch.randn(5, 2, 2, dtype=torch.float64, device=device)
    v = torch.randn(5, 2, 3, dtype=torch.float64, device=device)
    qpos, kpos = torch.tensor([4, 1, 3], device=device), torch.arange(5, device=device)
    gate_mask = (kpos[None] != 0).expand(3, -1)
    trace = cope.position_trace(q, k, qpos, attention_mask=gate_mask, checkpoint_id="trained")
    tpos = trace.positions.to(device)
    visibility = (kpos[None] % 2 == 0) | (kpos[None] == qpos[:, None])
    expected = cope_attention(q, k, v, cope, qpos, attention_mask=gate_mask,
                              fixed_positions=tpos * 0.5, visibility_mask=visibility)
    events = []

    def transform(positions, queries, keys):
        events.append(("positions", queries.tolist()))
        assert positions.shape[1] <= 2
        torch.testing.assert_close(keys, kpos)
        indices = (queries[:, None] == qpos[None, :]).long().argmax(-1)
        torch.testing.assert_close(positions, tpos[:, indices])
        return positions * 0.5

    def visibility_transform(queries, keys):
        events.append(("visibility", queries.tolist()))
        return (keys[None] % 2 == 0) | (keys[None] == queries[:, None])

    actual, transformed = cope_attention(
        q, k, v, cope, qpos, attention_mask=gate_mask, positions_transform=transform,
        visibility_transform=visibility_transform, query_chunk_size=2, return_positions=True,
    )
    torch.testing.assert_close(actual, expected)
    torch.testing.assert_close(transformed, tpos * 0.5)
    assert events == [("positions", [4, 1]), ("visibility", [4, 1]), ("positions", [3]), ("visibility", [3])]


def test_transforms_reject_invalid_results(device):
    # tests/test_position.py:331-358
    cope = CoPE(1, 4, device=device)
    q, k, v = [torch.ones(2, 1, 1, device=device) for _ in range(3)]
    args = (q, k, v, cope, torch.arange(2, device=device))
    with pytest.raises(CCPEPositionError, match="mutually exclusive"):
        cope_attention(*args, fixed_positions=torch.ones(1, 2, 2, device=device),
                       positions_transform=lambda p, *_: p)
    with pytest.raises(ValueError, match="mutually exclusive"):
        cope_attention(*args, visibility_mask=torch.ones(2, 2, dtype=torch.bool, device=device),
                       visibility_transform=lambda *_: torch.ones(2, 2, dtype=torch.bool, device=device))
    for transform in (lambda p, *_: p[:, 0], lambda p, *_: p.double(), lambda p, *_: p * torch.nan,
                      lambda p, *_: p - 5, lambda *_: None):
        with pytest.raises(CCPEPositionError, match="positions_transform"):
            cope_attention(*args, positions_transform=transform)
    for transform in (lambda *_: None, lambda *_: torch.ones(2, 2, device=device)):
        with pytest.raises(ValueError, match="bool"):
            cope_attention(*args, visibility_transform=transform)


# ------------------------------------------------------------ policies
def plan_with_dynamic_length(length):
    # tests/test_attention_policies.py:18-42
    return RequestPlan.parse(
        {
            "version": 1, "namespace": "policy-test", "task_id": "two-fixed-chunks",
            "operation": "reuse",
            "chunks": [
                {"id": "A", "role": "reuse", "start": 0, "end": 1},
                {"id": "update", "role": "recompute", "start": 1, "end": 1 + length},
                {"id": "B", "role": "reuse", "start": 1 + length, "end": 2 + length},
            ],
        },
        [11, *([9] * length), 22],
    )


def calibrated_profile(device):
    # tests/test_attention_policies.py:45-60
    cope = CoPE(1, 16, device=device, dtype=torch.float64)
    original = plan_with_dynamic_length(1)
    trace = cope.position_trace(torch.ones(3, 2, 1, dtype=torch.float64, device=device),
                                torch.zeros(3, 1, 1, dtype=torch.float64, device=device),
                                torch.arange(3, device=device), checkpoint_id="trained-cope")
    fixed = torch.tensor(original.fixed_indices)
    profile = CCPEProfile.calibrate(
        [trace.project(fixed, fixed)], [ChunkIdentity(*e) for e in original.fixed_layout],
        trained_profile_version="task-profile-v1",
    )
    return cope, profile


def test_strict_policy_rejects_hybrid_and_mixed_overrides(device):
    # tests/test_attention_policies.py:63-92
    cope, profile = calibrated_profile(device)
    plan = plan_with_dynamic_length(3)
    query = torch.ones(1, 2, 1, dtype=torch.float64, device=device)
    key = torch.zeros(5, 1, 1, dtype=torch.float64, device=device)
    policy = CanonicalPositionPolicy(plan, profile, "trained-cope")
    with pytest.raises(CCPEPositionError, match="nonincreasing"):
        cope_attention(query, key, key, cope, torch.tensor([4], device=device), positions_transform=policy)
    mixed = CanonicalPositionPolicy(plan, profile, "trained-cope", mode="mixed_bias_override")
    output, trace = cope_attention(query, key, key, cope, torch.tensor([4], device=device),
                                   positions_transform=mixed, return_positions=True)
    expected = torch.tensor([[[1.5, 2, 1.5, 1, 0.5]]], dtype=torch.float64)
    torch.testing.assert_close(trace.cpu(), expected.expand(2, -1, -1))
    assert output.dtype == trace.dtype == torch.float64


def test_strict_policy_accepts_same_layout(device):
    # tests/test_attention_policies.py:95-104
    cope, profile = calibrated_profile(device)
    plan = plan_with_dynamic_length(1)
    q = torch.ones(3, 2, 1, dtype=torch.float64, device=device)
    k = torch.zeros(3, 1, 1, dtype=torch.float64, device=device)
    trace = cope.position_trace(q, k, torch.arange(3, device=device), checkpoint_id="trained-cope")
    policy = CanonicalPositionPolicy(plan, profile, "trained-cope")
    positions = trace.positions.to(device)
    actual = policy(positions, torch.arange(3, device=device), torch.arange(3, device=device))
    torch.testing.assert_close(actual, positions)
    # lowered form inside the kernel: same outputs as the precomputed positions
    out_policy = cope_attention(q, k, k, cope, torch.arange(3, device=device), positions_transform=policy)
    out_plain = cope_attention(q, k, k, cope, torch.arange(3, device=device))
    torch.testing.assert_close(out_policy, out_plain)


def test_canonical_policy_tiles_use_fixed_ordinals(device):
    # tests/test_attention_policies.py:107-128
    cope, profile = calibrated_profile(device)
    plan = plan_with_dynamic_length(3)
    trace = cope.position_trace(torch.ones(5, 2, 1, dtype=torch.float64, device=device),
                                torch.zeros(5, 1, 1, dtype=torch.float64, device=device),
                                torch.arange(5, device=device), checkpoint_id="trained-cope")
    policy = CanonicalPositionPolicy(plan, profile, "trained-cope", mode="mixed_bias_override")
    positions = trace.positions.to(device)
    original = positions.clone()
    full = policy(positions, torch.arange(5, device=device), torch.arange(5, device=device))
    qtile, ktile = torch.tensor([4, 1, 0], device=device), torch.tensor([0, 2, 4], device=device)
    tile = policy(positions[:, qtile][:, :, ktile], qtile, ktile)
    torch.testing.assert_close(tile, full[:, qtile][:, :, ktile])
    torch.testing.assert_close(positions, original)
    torch.testing.assert_close(full[:, 1:4], original[:, 1:4])
    dynamic_only = original[:, 1:2]
    assert policy(dynamic_only, torch.tensor([1], device=device), torch.arange(5, device=device)) is dynamic_only


def test_lowered_canonical_policy_matches_callable_form(device):
    # The lowered (fused) policy and the reference's per-chunk callable form agree.
    cope, profile = calibrated_profile(device)
    plan = plan_with_dynamic_length(1)
    torch.manual_seed(4)
    q = torch.randn(3, 2, 1, dtype=torch.float64, device=device)
    k = torch.randn(3, 1, 1, dtype=torch.float64, device=device)
    v = torch.randn(3, 1, 2, dtype=torch.float64, device=device)
    policy = CanonicalPositionPolicy(plan, profile, "trained-cope", mode="mixed_bias_override")
    fused, ftrace = cope_attention(q, k, v, cope, torch.arange(3, device=device),
                                   positions_transform=policy, return_positions=True)
    chunked, ctrace = cope_attention(q, k, v, cope, torch.arange(3, device=device),
                                     positions_transform=lambda p, a, b: policy(p, a, b),
                                     return_positions=True, query_chunk_size=1)
    torch.testing.assert_close(fused, chunked)
    torch.testing.assert_close(ftrace, ctrace)


def test_selected_association_tiles_and_causality(device):
    # tests/test_attention_policies.py:131-153
    policy = SelectedAssociationPolicy((0, 2, 4), torch.tensor([4, 2], device=device))
    queries, keys = torch.tensor([4, 1, 2], device=device), torch.arange(6, device=device)
    mask = policy(queries, keys)
    assert mask.dtype == torch.bool
    assert mask.tolist() == [
        [False, True, False, True, True, True],
        [True, True, True, True, True, True],
        [False, True, True, True, False, True],
    ]
    torch.testing.assert_close(policy(queries[1:], keys[2:]), mask[1:, 2:])
    cope = CoPE(1, 16, device=device, dtype=torch.float64)
    q = torch.ones(3, 1, 1, dtype=torch.float64, device=device)
    k = torch.zeros(6, 1, 1, dtype=torch.float64, device=device)
    v = torch.arange(6, dtype=torch.float64, device=device)[:, None, None]
    actual = cope_attention(q, k, v, cope, queries, visibility_transform=policy, query_chunk_size=1)
    torch.testing.assert_close(actual[:, 0, 0].cpu(), torch.tensor([8 / 3, 0.5, 1.5], dtype=torch.float64))


def test_wca_association_after_gates(device):
    # tests/test_attention_policies.py:156-190
    cope = cope_on(device, 1, 16, torch.float64, torch.arange(16.0)[None])
    q = torch.ones(1, 1, 1, dtype=torch.float64, device=device)
    k = torch.zeros(5, 1, 1, dtype=torch.float64, device=device)
    v = torch.tensor([1, 10, 100, 1000, 10000], dtype=torch.float64, device=device)[:, None, None]
    queries, keys = torch.tensor([4], device=device), torch.arange(5, device=device)
    association = SelectedAssociationPolicy((0, 2, 4), torch.tensor([4], device=device))
    output, positions = cope_attention(q, k, v, cope, queries, visibility_transform=association,
                                       return_positions=True)
    expected_positions = torch.tensor([[[2.5, 2, 1.5, 1, 0.5]]], dtype=torch.float64)
    torch.testing.assert_close(positions.cpu(), expected_positions)
    visible = association(queries, keys)[0].cpu()
    expected = expected_positions[0, 0, visible].softmax(0) @ v.cpu()[visible, 0, 0]
    torch.testing.assert_close(output[0, 0, 0].cpu(), expected)
    wrong, wrong_positions = cope_attention(q, k, v, cope, queries,
                                            attention_mask=association(queries, keys), return_positions=True)
    assert wrong_positions[0, 0, 1] == 1.5
    assert not torch.allclose(output, wrong)


# ------------------------------------------------------------ seeded vs oracle
CASES = ["causal", "sparse_rows", "attention_mask", "visibility", "fixed", "value_dim"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("case", CASES)
def test_generic_kernel_matches_oracle(device, dtype, case):
    seed = 100 + CASES.index(case)
    nq_all, nk, hq, hkv, d, dv, npos = 150, 150, 4, 2, 32, 32, 64
    if case == "value_dim":
        dv = 48
    q = seeded((nq_all, hq, d), seed, dtype=dtype)
    k = seeded((nk, hkv, d), seed + 1, dtype=dtype)
    v = seeded((nk, hkv, dv), seed + 2, dtype=dtype)
    e = seeded((d, npos), seed + 3, scale=0.5)
    qpos = np.arange(nq_all)
    if case == "sparse_rows":
        keep = np.sort(np.random.default_rng(seed).choice(nq_all, 40, replace=False))
        q, qpos = q[keep], qpos[keep][::-1].copy()  # any order
        q = q.flip(0)
    nq = q.shape[0]
    kwargs_np, kwargs_t = {}, {}
    if case == "attention_mask":
        m = np.random.default_rng(seed).random((nq, nk)) > 0.2
        kwargs_np["attention_mask"] = m
        kwargs_t["attention_mask"] = torch.from_numpy(m).to(device)
    if case == "visibility":
        m = np.random.default_rng(seed).random((hq, nq, nk)) > 0.3
        kwargs_np["visibility_mask"] = m
        kwargs_t["visibility_mask"] = torch.from_numpy(m).to(device)
    if case == "fixed":
        acc = torch.float64 if dtype == torch.float64 else torch.float32
        f = torch.rand((hq, nq, nk), generator=torch.Generator().manual_seed(seed), dtype=acc) * (npos - 1)
        kwargs_np["fixed_positions"] = f.numpy()
        kwargs_t["fixed_positions"] = f.to(device)
    expected, etrace = orc.cope_attention(acc_np(q), acc_np(k), acc_np(v), e.numpy().astype(acc_np(q).dtype),
                                          qpos, return_positions=True, **kwargs_np)
    cope = cope_on(device, d, npos, table=e)
    actual, trace = cope_attention(q.to(device), k.to(device), v.to(device), cope,
                                   torch.from_numpy(qpos).to(device), return_positions=True,
                                   query_chunk_size=64, **kwargs_t)
    if dtype == torch.bfloat16:
        assert_close_bf16(actual, expected)
    else:
        torch.testing.assert_close(actual.cpu(), torch.from_numpy(expected), **tolerance(dtype))
    ptol = {"atol": 1e-4, "rtol": 1e-5} if dtype != torch.float64 else {"atol": 1e-10, "rtol": 1e-10}
    torch.testing.assert_close(trace.cpu(), torch.from_numpy(etrace), **ptol)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 2), (4, 4), (16, 2)])
@pytest.mark.parametrize("n", [1, 130, 700])
def test_mfma_prefill_dense_matches_oracle(device, hq, hkv, n):
    """bf16, D = 128: cope_attention dispatches to the MFMA kernel."""
    seed = 7 * n + hq
    q = seeded((n, hq, 128), seed, dtype=torch.bfloat16)
    k = seeded((n, hkv, 128), seed + 1, dtype=torch.bfloat16)
    v = seeded((n, hkv, 128), seed + 2, dtype=torch.bfloat16)
    e = seeded((128, 64), seed + 3, scale=0.02)
    expected = orc.cope_attention(acc_np(q), acc_np(k), acc_np(v), e.numpy(), np.arange(n))
    cope = cope_on(device, 128, 64, table=e)
    actual = cope_attention(q.to(device), k.to(device), v.to(device), cope, torch.arange(n, device=device))
    assert_close_bf16(actual, expected)


@pytest.mark.parametrize("npos", [2, 3, 37, 127])
def test_mfma_prefill_odd_and_small_tables(device, npos):
    """Table lengths that are odd or tiny: P = 2, 3, 37 keep two 4-wave
    workgroups per CU, P = 127 takes the 8-wave layout; the QE rows are padded
    to an even length with an odd number of 32-bit words."""
    n, hq, hkv = 333, 8, 2
    q = seeded((n, hq, 128), 60 + npos, dtype=torch.bfloat16)
    k = seeded((n, hkv, 128), 61 + npos, dtype=torch.bfloat16)
    v = seeded((n, hkv, 128), 62 + npos, dtype=torch.bfloat16)
    e = seeded((128, npos), 63 + npos, scale=0.1)
    expected = orc.cope_attention(acc_np(q), acc_np(k), acc_np(v), e.numpy(), np.arange(n))
    cope = cope_on(device, 128, npos, table=e)
    actual = cope_attention(q.to(device), k.to(device), v.to(device), cope, torch.arange(n, device=device))
    assert_close_bf16(actual, expected)


@pytest.mark.parametrize("npos", [128, 256])
def test_prefill_large_table_and_sparse_rows(device, npos):
    # unsorted sparse query rows and a strong table; P = 128 runs the MFMA kernel
    # (4 position tiles), P = 256 exceeds its LDS budget and runs the generic kernel
    n, hq, hkv = 900, 4, 1
    q = seeded((n, hq, 128), 31, dtype=torch.bfloat16)
    k = seeded((n, hkv, 128), 32, dtype=torch.bfloat16)
    v = seeded((n, hkv, 128), 33, dtype=torch.bfloat16)
    e = seeded((128, npos), 34, scale=0.2)
    rows = np.random.default_rng(3).permutation(n)[:300]
    expected = orc.cope_attention(acc_np(q)[rows], acc_np(k), acc_np(v), e.numpy(), rows)
    cope = cope_on(device, 128, npos, table=e)
    actual = cope_attention(q[rows].to(device), k.to(device), v.to(device), cope,
                            torch.from_numpy(rows).to(device))
    assert_close_bf16(actual, expected)


def test_mfma_prefill_zero_table_is_sdpa(device):
    """Library reduction: E = 0 gives causal softmax attention (torch SDPA, fp32, CPU)."""
    n, hq, hkv = 333, 8, 2
    q = seeded((n, hq, 128), 41, dtype=torch.bfloat16)
    k = seeded((n, hkv, 128), 42, dtype=torch.bfloat16)
    v = seeded((n, hkv, 128), 43, dtype=torch.bfloat16)
    cope = CoPE(128, 64, device=device)
    actual = cope_attention(q.to(device), k.to(device), v.to(device), cope, torch.arange(n, device=device))
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.float().permute(1, 0, 2), k.float().repeat_interleave(4, 1).permute(1, 0, 2).contiguous(),
        v.float().repeat_interleave(4, 1).permute(1, 0, 2).contiguous(), is_causal=True,
    ).permute(1, 0, 2)
    assert_close_bf16(actual, ref.numpy())


def test_paged_prefill_matches_oracle(device):
    lens = [300, 64, 1000]
    hq, hkv, bs = 8, 2, 16
    nb, table, rows = paged_layout(lens, hkv, bs, 128, seed=5)
    cache = seeded((nb, hkv, bs, 256), 50, dtype=torch.bfloat16)
    keys = [seeded((n, hkv, 128), 60 + i, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    vals = [seeded((n, hkv, 128), 70 + i, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    fill_paged(cache, rows, keys, vals)
    e = seeded((128, 64), 80, scale=0.02)
    nq = 200
    qs = seeded((len(lens), nq, hq, 128), 81, dtype=torch.bfloat16)
    gen = np.random.default_rng(90)
    # request 1 is shorter than the row count: its rows repeat positions (each
    # row is independent in the fused entry point)
    qpos = np.stack([
        np.sort(gen.choice(lens[0], nq, replace=False)),
        np.arange(nq) // 4,
        np.sort(gen.choice(lens[2], nq, replace=False)),
    ]).astype(np.int64)
    cope = cope_on(device, 128, 64, table=e)
    out = ccpe_prefill_paged(qs.to(device), cache.to(device), table.to(device),
                             torch.tensor(lens, dtype=torch.int32, device=device), cope,
                             torch.from_numpy(qpos).to(device))
    for b in range(len(lens)):
        rows_out = [
            orc.cope_attention(acc_np(qs[b, r:r + 1]), acc_np(keys[b]), acc_np(vals[b]), e.numpy(),
                               qpos[b, r:r + 1])
            for r in range(nq)
        ]
        assert_close_bf16(out[b], np.concatenate(rows_out, axis=0))


@pytest.mark.parametrize("split", [64, 512])
def test_decode_matches_oracle(device, split):
    lens = [1, 63, 700, 2100]
    hq, hkv, bs = 8, 2, 16
    nb, table, rows = paged_layout(lens, hkv, bs, 128, seed=9)
    cache = seeded((nb, hkv, bs, 256), 51, dtype=torch.bfloat16)
    keys = [seeded((n, hkv, 128), 61 + i, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    vals = [seeded((n, hkv, 128), 71 + i, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    fill_paged(cache, rows, keys, vals)
    e = seeded((128, 64), 82, scale=0.02)
    q = seeded((len(lens), hq, 128), 83, dtype=torch.bfloat16)
    cope = cope_on(device, 128, 64, table=e)
    out = ccpe_decode_paged(q.to(device), cache.to(device), table.to(device),
                            torch.tensor(lens, dtype=torch.int32, device=device), cope, split=split)
    for b, n in enumerate(lens):
        expected = orc.cope_attention(acc_np(q[b:b + 1]), acc_np(keys[b]), acc_np(vals[b]), e.numpy(),
                                      np.array([n - 1]))
        assert_close_bf16(out[b:b + 1], expected)


@pytest.mark.parametrize("n, split", [(1500, 128), (17000, 64)])
def test_decode_unsaturated_splits_are_recomputed(device, n, split):
    """Keys anti-aligned with the query: gates ~0, positions never saturate, so
    every split's speculation fails and the exact fixup path produces the result
    (17000 keys in splits of 64: 265 recomputed splits, more than one chunk of
    the finishing workgroup's list)."""
    hq, hkv, bs = 4, 1, 16
    nb, table, rows = paged_layout([n], hkv, bs, 128, seed=11)
    q = seeded((1, hq, 128), 84, dtype=torch.bfloat16)
    base = q[0, 0].float()
    keys = [(-(base[None, None, :] * 2) + seeded((n, hkv, 128), 85, scale=0.1)).to(torch.bfloat16)]
    vals = [seeded((n, hkv, 128), 86, dtype=torch.bfloat16)]
    cache = torch.zeros((nb, hkv, bs, 256), dtype=torch.bfloat16)
    fill_paged(cache, rows, keys, vals)
    e = seeded((128, 64), 87, scale=0.3)
    cope = cope_on(device, 128, 64, table=e)
    qq = q.clone()
    qq[0, 1:] = q[0, 0]
    out = ccpe_decode_paged(qq.to(device), cache.to(device), table.to(device),
                            torch.tensor([n], dtype=torch.int32, device=device), cope, split=split)
    allowed = orc.allowed_mask(np.array([n - 1]), np.arange(n), hq)
    p = orc.contextual_positions(orc.logits(acc_np(qq), acc_np(keys[0])), allowed, 64)
    assert p.max() < 63  # never saturated: the fixup path is exercised
    expected = orc.cope_attention(acc_np(qq), acc_np(keys[0]), acc_np(vals[0]), e.numpy(), np.array([n - 1]))
    assert_close_bf16(out, expected)


@pytest.mark.parametrize("hq, hkv, bs", [(4, 4, 16), (8, 4, 32), (16, 2, 64), (32, 1, 16)])
def test_paged_prefill_group_and_block_sizes(device, hq, hkv, bs):
    """GQA groups 1, 2, 8 and 32 over block sizes 16-64, every row causal."""
    lens = [150, 520]
    nb, table, rows = paged_layout(lens, hkv, bs, 128, seed=hq + bs)
    cache = seeded((nb, hkv, bs, 256), 150 + hq, dtype=torch.bfloat16)
    keys = [seeded((n, hkv, 128), 160 + i + hq, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    vals = [seeded((n, hkv, 128), 170 + i + hq, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    fill_paged(cache, rows, keys, vals)
    e = seeded((128, 64), 180 + bs, scale=0.02)
    nq = 48
    qs = seeded((len(lens), nq, hq, 128), 181 + hq, dtype=torch.bfloat16)
    gen = np.random.default_rng(hq * 100 + bs)
    qpos = np.stack([np.sort(gen.choice(n, nq, replace=False)) for n in lens]).astype(np.int64)
    cope = cope_on(device, 128, 64, table=e)
    out = ccpe_prefill_paged(qs.to(device), cache.to(device), table.to(device),
                             torch.tensor(lens, dtype=torch.int32, device=device), cope,
                             torch.from_numpy(qpos).to(device))
    for b in range(len(lens)):
        expected = np.concatenate([
            orc.cope_attention(acc_np(qs[b, r:r + 1]), acc_np(keys[b]), acc_np(vals[b]), e.numpy(),
                               qpos[b, r:r + 1])
            for r in range(nq)], axis=0)
        assert_close_bf16(out[b], expected)


@pytest.mark.parametrize("hq, hkv, bs, split", [(4, 4, 16, 1024), (32, 8, 32, 1024), (64, 8, 64, 256)])
def test_decode_group_and_block_sizes(device, hq, hkv, bs, split):
    """GQA groups 1, 4 and 8 over block sizes 16-64, the default split included."""
    lens = [5, 1100, 2600]
    nb, table, rows = paged_layout(lens, hkv, bs, 128, seed=hq + split)
    cache = seeded((nb, hkv, bs, 256), 250 + hq, dtype=torch.bfloat16)
    keys = [seeded((n, hkv, 128), 260 + i + hq, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    vals = [seeded((n, hkv, 128), 270 + i + hq, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    fill_paged(cache, rows, keys, vals)
    e = seeded((128, 64), 280 + bs, scale=0.02)
    q = seeded((len(lens), hq, 128), 283 + hq, dtype=torch.bfloat16)
    cope = cope_on(device, 128, 64, table=e)
    out = ccpe_decode_paged(q.to(device), cache.to(device), table.to(device),
                            torch.tensor(lens, dtype=torch.int32, device=device), cope, split=split)
    for b, n in enumerate(lens):
        expected = orc.cope_attention(acc_np(q[b:b + 1]), acc_np(keys[b]), acc_np(vals[b]), e.numpy(),
                                      np.array([n - 1]))
        assert_close_bf16(out[b:b + 1], expected)


@pytest.mark.parametrize("hq, hkv, splits", [
    (8, 2, [16, 17, 32, 33]), (8, 2, [48, 49, 64, 65]), (16, 2, [31, 32, 33]), (2, 2, [1, 64, 65]),
])
def test_decode_finish_split_counts(device, hq, hkv, splits):
    """Split counts on both sides of each 16-split chunk of the finishing
    workgroup's register merge and of its limit (64 splits for GQA groups up
    to 4, 32 for a group of 8), past which the merge reads its partials in
    rounds.  Splits of 256 keys, the last one partly filled; the right-most
    split's gate mass reaches P-1 in every head, so no split is recomputed
    and the register merge (or, past its limit, the merge in rounds) forms
    every output row."""
    split, bs = 256, 16
    lens = [split * (s - 1) + 1 + (7 * s) % (split - 1) for s in splits]
    assert [(n + split - 1) // split for n in lens] == splits
    nb, table, rows = paged_layout(lens, hkv, bs, 128, seed=hq + len(lens))
    cache = seeded((nb, hkv, bs, 256), 290 + hq, dtype=torch.bfloat16)
    keys = [seeded((n, hkv, 128), 300 + i + hq, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    vals = [seeded((n, hkv, 128), 310 + i + hq, dtype=torch.bfloat16) for i, n in enumerate(lens)]
    fill_paged(cache, rows, keys, vals)
    e = seeded((128, 64), 320 + hq, scale=0.02)
    q = seeded((len(lens), hq, 128), 321 + hq, dtype=torch.bfloat16)
    cope = cope_on(device, 128, 64, table=e)
    out = ccpe_decode_paged(q.to(device), cache.to(device), table.to(device),
                            torch.tensor(lens, dtype=torch.int32, device=device), cope, split=split)
    for b, n in enumerate(lens):
        if n > split:  # split 0 saturates every head: no recomputation
            right = orc.sigmoid(orc.logits(acc_np(q[b:b + 1]), acc_np(keys[b][-split:]))).sum(axis=-1)
            assert right.min() >= 63
        expected = orc.cope_attention(acc_np(q[b:b + 1]), acc_np(keys[b]), acc_np(vals[b]), e.numpy(),
                                      np.array([n - 1]))
        assert_close_bf16(out[b:b + 1], expected)


def test_zero_query_tokens_give_an_empty_result(device):
    # position.py:117-150 requires one key and one head, not one query token
    cope = CoPE(16, 8, device=device)
    q = torch.zeros((0, 4, 16), device=device)
    k = torch.randn((5, 2, 16), device=device)
    v = torch.randn((5, 2, 16), device=device)
    out = cope_attention(q, k, v, cope, torch.zeros(0, dtype=torch.long, device=device))
    assert out.shape == (0, 4, 16)
