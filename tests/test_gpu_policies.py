"""The two attention policies on the device at realistic size, against the oracle.

``CacheSlideRuntime._attend`` (src/cacheslide_vllm/runtime.py:576-609) calls
``cope_attention`` on the active rows of a reuse prefill with a
``CanonicalPositionPolicy`` (attention.py:18-57) and a
``SelectedAssociationPolicy`` (attention.py:60-72).  The reference evaluates
them per query chunk: ``CCPEProfile.lookup`` for the chunk's fixed rows
(position.py:701-748), canonical substitution of the fixed x fixed cells,
then, in ``strict_contextual`` mode, ``validate_contextual_path``
(position.py:28-114), whose first failing check in the first failing chunk
raises.  Here the policies are lowered to kernel data; the decisions (accept,
or which error with which message, from which chunk) must be the oracle's, and
accepted outputs and traces must agree within the float tolerance.

Layout: 600 tokens = reused chunk A (200) + recomputed chunk (120) + reused
chunk B (280); 480 fixed tokens, a profile of 4 heads x 480 x 480 cells (the
1,000,000-element calibration budget), active rows as after WCA selection.
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
from oracle import ccpe as orc
from tests._helpers import seeded

pytestmark = pytest.mark.gpu

HQ, HKV, D, P = 4, 2, 64, 64


def make_plan(a: int, dyn: int, b: int) -> RequestPlan:
    n = a + dyn + b
    return RequestPlan.parse(
        {"version": 1, "namespace": "policy-scale", "task_id": "t", "operation": "reuse",
         "chunks": [{"id": "A", "role": "reuse", "start": 0, "end": a},
                    {"id": "update", "role": "recompute", "start": a, "end": a + dyn},
                    {"id": "B", "role": "reuse", "start": a + dyn, "end": n}]},
        [7 + (i % 97) for i in range(a)] + [3] * dyn + [11 + (i % 89) for i in range(b)],
    )


def profile_for(plan: RequestPlan, canonical: np.ndarray, ordinals: list[int]) -> CCPEProfile:
    fixed = len(plan.fixed_indices)
    return CCPEProfile(
        trained_profile_version="v1", checkpoint_id="ckpt",
        chunks=tuple(ChunkIdentity(*e) for e in plan.fixed_layout),
        query_positions=torch.tensor(ordinals, dtype=torch.long),
        key_positions=torch.arange(fixed, dtype=torch.long),
        canonical_positions=torch.from_numpy(np.ascontiguousarray(canonical)).float(),
        max_positions=P, histogram_bin_width=0.25, sample_count=1,
    )


def contextual(q: np.ndarray, k: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """Oracle contextual positions [H, rows, keys] of query rows at positions ``rows``."""
    allowed = orc.allowed_mask(rows, np.arange(k.shape[0]), HQ)
    return orc.contextual_positions(orc.logits(q[rows], k), allowed, P)


def oracle_run(q, k, v, e, rows, plan, canonical, ordinals, strict, selected, chunk):
    """The reference's per-chunk evaluation with the policies, on the oracle
    (no visibility transform when ``selected`` is None).  Returns ("ok", out,
    trace) or ("error", type, message)."""
    fixed = list(plan.fixed_indices)
    ordinal = {p: i for i, p in enumerate(fixed)}
    known = set(ordinals)

    def positions_transform(pos, qpos, kpos):
        frows = [int(p) for p in qpos if int(p) in ordinal]
        if frows and any(ordinal[p] not in known for p in frows):
            raise ValueError("CCPE profile has no contextual trace for these query positions")
        return orc.canonical_policy(pos, qpos, kpos, fixed, canonical, ordinals, strict)

    def visibility_transform(qpos, kpos):
        return orc.selected_visibility(qpos, kpos, fixed, selected)

    try:
        out, trace = orc.cope_attention(q[rows], k, v, e, rows, positions_transform=positions_transform,
                                        visibility_transform=visibility_transform if selected is not None else None,
                                        query_chunk_size=chunk, return_positions=True)
    except orc.PathError as err:
        return ("error", CCPEPositionError, orc.PATH_MESSAGES[err.kind])
    except ValueError as err:
        return ("error", ValueError, str(err))
    return ("ok", out, trace)


def device_run(q, k, v, e, rows, plan, profile, mode, selected, chunk, device):
    cope = CoPE(D, P, device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(torch.from_numpy(e))
    policy = CanonicalPositionPolicy(plan, profile, "ckpt", mode=mode)
    visibility = SelectedAssociationPolicy(plan.fixed_indices, torch.tensor(selected, device=device))
    try:
        out, trace = cope_attention(
            torch.from_numpy(q[rows]).to(device), torch.from_numpy(k).to(device),
            torch.from_numpy(v).to(device), cope, torch.from_numpy(rows).to(device),
            positions_transform=policy, visibility_transform=visibility, query_chunk_size=chunk,
            return_positions=True)
    except CCPEPositionError as err:
        return ("error", CCPEPositionError, str(err))
    except ValueError as err:
        return ("error", ValueError, str(err))
    return ("ok", out.cpu().numpy(), trace.cpu().numpy())


def scenario(seed: int, *, shift: int, drop_ordinals: int, perturb: float):
    """Inputs, plan and profile.  The profile is calibrated on the same fixed
    chunks with the recomputed chunk ``shift`` tokens longer (0: the current
    layout), ``drop_ordinals`` fixed ordinals get no trace, and ``perturb``
    adds noise to the canonical table."""
    a, dyn, b = 200, 120, 280
    plan = make_plan(a, dyn, b)
    n = a + dyn + b
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n, HQ, D)).astype(np.float32)
    k = rng.standard_normal((n, HKV, D)).astype(np.float32)
    v = rng.standard_normal((n, HKV, D)).astype(np.float32)
    e = (rng.standard_normal((D, P)) * 0.3).astype(np.float32)
    fixed = np.array(plan.fixed_indices)
    # calibration layout: A, a recomputed chunk of dyn + shift tokens, B
    cal_dyn = rng.standard_normal((dyn + shift, HQ, D)).astype(np.float32) if shift else q[a:a + dyn]
    cal_dyn_k = rng.standard_normal((dyn + shift, HKV, D)).astype(np.float32) if shift else k[a:a + dyn]
    cq = np.concatenate([q[:a], cal_dyn, q[a + dyn:]])
    ckk = np.concatenate([k[:a], cal_dyn_k, k[a + dyn:]])
    cal_fixed = np.concatenate([np.arange(a), np.arange(a + dyn + shift, n + shift)])
    cal = contextual(cq, ckk, cal_fixed)[:, :, cal_fixed]          # [H, F, F]
    if perturb:
        cal = np.clip(cal + rng.standard_normal(cal.shape).astype(np.float32) * perturb, 0, P - 1)
    # active rows: a WCA-like selection of fixed rows, every recomputed row, the last row
    sel = np.sort(rng.choice(fixed[:-1], 90, replace=False))
    # untraced ordinals are taken among the active fixed rows, so a chunk meets one
    ordinal_of = {int(pos): i for i, pos in enumerate(fixed)}
    dropped = {ordinal_of[int(pos)] for pos in rng.choice(sel, drop_ordinals, replace=False)} if drop_ordinals else set()
    ordinals = sorted(set(range(len(fixed))) - dropped)
    canonical = cal[:, ordinals]
    rows = np.unique(np.concatenate([sel, np.arange(a, a + dyn), [n - 1]]))
    rows = rows[rng.permutation(len(rows))]                          # any row order
    selected = sel[: len(sel) // 2]
    return q, k, v, e, rows, plan, canonical, ordinals, selected


def compare(expected, actual):
    assert expected[0] == actual[0], (expected[:1] + expected[1:] if expected[0] == "error" else "ok", actual)
    if expected[0] == "error":
        assert expected[1] is actual[1] and expected[2] == actual[2], (expected, actual)
        return
    np.testing.assert_allclose(actual[1], expected[1], atol=1e-4, rtol=1e-4)
    np.testing.assert_allclose(actual[2], expected[2], atol=1e-4, rtol=1e-5)


CASES = {
    # name: (seed, shift, drop_ordinals, perturb, mode, chunk)
    "same_layout_strict": (1, 0, 0, 0.0, "strict_contextual", 64),
    "shifted_strict": (2, 16, 0, 0.0, "strict_contextual", 64),
    "shifted_mixed": (3, 16, 0, 0.0, "mixed_bias_override", 64),
    "perturbed_strict": (4, 0, 0, 0.02, "strict_contextual", 48),
    "perturbed_mixed": (5, 0, 0, 0.5, "mixed_bias_override", 128),
    "untraced_ordinals_strict": (6, 0, 5, 0.0, "strict_contextual", 32),
    "untraced_ordinals_mixed": (7, 0, 5, 0.0, "mixed_bias_override", 32),
    "shift_one_strict": (8, 1, 0, 0.0, "strict_contextual", 64),
}


@pytest.mark.parametrize("name", list(CASES))
def test_policy_decisions_and_outputs_match_oracle(device, name):
    seed, shift, drop, perturb, mode, chunk = CASES[name]
    q, k, v, e, rows, plan, canonical, ordinals, selected = scenario(seed, shift=shift, drop_ordinals=drop,
                                                                     perturb=perturb)
    strict = mode == "strict_contextual"
    expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, strict, selected, chunk)
    profile = profile_for(plan, canonical, ordinals)
    actual = device_run(q, k, v, e, rows, plan, profile, mode, selected, chunk, device)
    compare(expected, actual)
    if name == "same_layout_strict":
        assert expected[0] == "ok"
    if name in ("shifted_strict", "perturbed_strict"):
        assert expected[0] == "error" and expected[1] is CCPEPositionError
    if name.startswith("untraced"):
        assert expected[0] == "error" and "no contextual trace" in expected[2]


def test_first_failing_chunk_decides(device):
    """Row chunks of one row each: chunk 0 a recomputed row (never validated),
    then a fixed row whose canonical path fails 'available', then a fixed row
    with an untraced ordinal.  The reference raises the first failing chunk's
    error, so the order of the rows decides which; an out-of-range canonical
    cell fails the transform bounds check in mixed mode."""
    q, k, v, e, _, plan, canonical, ordinals, selected = scenario(11, shift=0, drop_ordinals=0, perturb=0.0)
    fixed = list(plan.fixed_indices)
    bad_row, untraced_row = fixed[150], fixed[300]
    canonical = canonical.copy()
    canonical[:, 150, 150] = 60.0            # the row's own key: 1 gate available, 60 claimed
    keep = [i for i in range(canonical.shape[1]) if i != 300]
    canonical, ordinals = canonical[:, keep], [ordinals[i] for i in keep]
    profile = profile_for(plan, canonical, ordinals)
    untraced = "CCPE profile has no contextual trace for these query positions"
    for mode, order, want in (
        ("strict_contextual", [250, bad_row, untraced_row], orc.PATH_MESSAGES["available"]),
        ("strict_contextual", [250, untraced_row, bad_row], untraced),
        ("mixed_bias_override", [250, untraced_row, bad_row], untraced),
    ):
        rows = np.array(order)
        strict = mode == "strict_contextual"
        expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, strict, selected, 1)
        actual = device_run(q, k, v, e, rows, plan, profile, mode, selected, 1, device)
        compare(expected, actual)
        assert actual[0] == "error" and actual[2] == want, (mode, order, actual)
    # mixed mode: a canonical cell outside [0, P-1] fails the bounds check of its chunk
    canonical[:, 150, 10] = P + 3.0
    profile = profile_for(plan, canonical, ordinals)
    rows = np.array([250, bad_row, untraced_row])
    expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, False, selected, 1)
    actual = device_run(q, k, v, e, rows, plan, profile, "mixed_bias_override", selected, 1, device)
    compare(expected, actual)
    assert actual[0] == "error" and actual[2] == orc.PATH_MESSAGES["transform"]


def _ordered(x: np.float32) -> int:
    """float32 -> integer with the same order (adjacent floats differ by 1)."""
    bits = int(np.array(x, np.float32).view(np.uint32))
    return bits if bits < 0x80000000 else -(bits & 0x7FFFFFFF)


def _from_ordered(i: int) -> np.float32:
    bits = i if i >= 0 else (-i) | 0x80000000
    return np.array(bits, np.uint32).view(np.float32)[()]


def _decision(p: np.ndarray):
    try:
        orc.validate_contextual_path(p[None, None, :], np.array([11]), np.arange(12))
    except orc.PathError as err:
        return err.kind
    return None


def borderline_paths(seed: int) -> list[np.ndarray]:
    """Paths of query position 11 over keys 0..11 that sit within 3 ulps of
    the edge of one check of validate_contextual_path (position.py:98-114):
    one gate per token (gap), the available count, nonnegativity and
    nonincreasing order.  The edge is found by bisection over float32 values
    on the oracle; each check's tolerance includes the fp32 rounding slack."""
    rng = np.random.default_rng(seed)
    out = []

    def with_left(p, i, gates):
        # p[j] for j < i: nonincreasing small steps from p[i], inside the available counts
        acc = p[i]
        for j in range(i - 1, -1, -1):
            acc = np.float32(acc + gates[j])
            p[j] = acc
        return p

    for kind in ("gap", "available", "nonnegative", "nonincreasing"):
        right = np.flip(np.cumsum(np.flip(rng.uniform(0.05, 0.9, 5)))).astype(np.float32)
        small = rng.uniform(0.05, 0.2, 11).astype(np.float32)

        def build(x, kind=kind, right=right, small=small):
            p = np.zeros(12, np.float32)
            if kind == "gap":
                p[7:] = right
                p[6] = x
                return with_left(p, 6, small)
            if kind in ("available", "nonnegative"):
                p[11] = x
                return with_left(p, 11, small)
            p[11] = np.float32(0.5)           # nonincreasing between keys 10 and 11
            p[10] = x
            return with_left(p, 10, small)

        lo_hi = {"gap": (right[0] + 0.5, right[0] + 1.01), "available": (0.5, 1.01),
                 "nonnegative": (0.0, -1e-5), "nonincreasing": (0.5, 0.49)}[kind]
        good, bad = (_ordered(np.float32(v)) for v in lo_hi)
        assert _decision(build(_from_ordered(good))) != kind
        assert _decision(build(_from_ordered(bad))) == kind
        while abs(bad - good) > 1:
            mid = (good + bad) // 2
            if _decision(build(_from_ordered(mid))) == kind:
                bad = mid
            else:
                good = mid
        step = 1 if bad > good else -1
        out += [build(_from_ordered(bad + step * k)) for k in range(-3, 4)]
    return out


def test_validation_borderlines_match_oracle(device):
    """validate_contextual_path within 3 ulps of each check's edge, on the
    device: standalone, and fused into the strict canonical policy (the
    canonical row covers every causal key of the query)."""
    plan = make_plan(12, 1, 1)          # fixed keys 0..11 and 13, recomputed key 12
    cope = CoPE(8, P, device=device)
    q = torch.zeros((1, 1, 8), device=device)
    k = torch.zeros((14, 1, 8), device=device)
    seen = set()
    for seed in range(3):
        for p in borderline_paths(seed):
            want = _decision(p)
            seen.add(want)
            got = None
            try:
                validate_contextual_path(torch.from_numpy(p[None, None, :]).to(device),
                                         torch.tensor([11], device=device), torch.arange(12, device=device))
            except CCPEPositionError as err:
                got = str(err)
            assert got == (orc.PATH_MESSAGES[want] if want else None), (p.tolist(), want, got)
            # fused: the profile row of ordinal 11 is the path; cells past the
            # query are future keys (not validated) and must stay in bounds
            canonical = np.zeros((1, 13, 13), np.float32)
            canonical[0, 11, :12] = p
            profile = profile_for(plan, canonical, list(range(13)))
            policy = CanonicalPositionPolicy(plan, profile, "ckpt")
            fused = None
            try:
                cope_attention(q, k, k, cope, torch.tensor([11], device=device), positions_transform=policy)
            except CCPEPositionError as err:
                fused = str(err)
            if want is None and (p < 0).any():
                want_fused = orc.PATH_MESSAGES["transform"]    # passes validation, fails the bounds
            else:
                want_fused = orc.PATH_MESSAGES[want] if want else None
            assert fused == want_fused, (p.tolist(), want_fused, fused)
    assert {None, "gap", "available", "nonnegative", "nonincreasing"} <= seen
