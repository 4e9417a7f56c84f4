"""The reuse call of ``CacheSlideRuntime._attend`` (src/cacheslide_vllm/
runtime.py:576-609) on the MFMA policy path: bf16 Q/K/V with head dim 128,
dense keys at coordinates 0..n-1, a ``CanonicalPositionPolicy``
(attention.py:18-57) and a ``SelectedAssociationPolicy`` in updated_and_self
mode (attention.py:60-72) whose selected rows are every fixed query row.

Checked against the oracle's per-chunk evaluation of the two policies
(oracle/ccpe.py canonical_policy, selected_visibility, cope_attention): the
same decision (accept, or the same error type and message from the same
chunk) and, when accepted, outputs within the bf16 tolerance (2e-2 absolute,
1e-2 relative).  Each test also checks which kernel ran: the MFMA path (also
for fixed query rows that are not selected, whose canonical cells it reads
tile by tile), or the generic kernel when the plan holds more dynamic keys
beside fixed keys than the checker does.

Layout: reused chunk A, a recomputed chunk, reused chunk B (make_plan);
8 query heads over 2 KV heads; CoPE P = 64, table N(0, 0.1).  The profile is
calibrated on the oracle (contextual positions of the fixed x fixed cells of
a calibration layout: the same chunks, the recomputed chunk ``shift`` tokens
longer), optionally perturbed or missing some ordinals.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import cacheslide_amd.position as position_module
from cacheslide_amd import CanonicalPositionPolicy, CCPEPositionError, CoPE, SelectedAssociationPolicy, cope_attention
from oracle import ccpe as orc
from tests._helpers import assert_close_bf16
from tests.test_gpu_policies import make_plan, oracle_run, profile_for

pytestmark = pytest.mark.gpu

HQ, HKV, D, P = 8, 2, 128, 64


def bf16_normal(rng, shape, scale=1.0):
    x = torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(torch.bfloat16)
    return x.float().numpy()


def contextual(q, k, rows):
    allowed = orc.allowed_mask(rows, np.arange(k.shape[0]), HQ)
    return orc.contextual_positions(orc.logits(q[rows], k), allowed, P)


def scenario(seed, *, a, dyn, b, shift=0, perturb=0.0, drop=0, n_sel=60):
    plan = make_plan(a, dyn, b)
    n = a + dyn + b
    rng = np.random.default_rng(seed)
    q, k, v = bf16_normal(rng, (n, HQ, D)), bf16_normal(rng, (n, HKV, D)), bf16_normal(rng, (n, HKV, D))
    e = (rng.standard_normal((D, P)) * 0.1).astype(np.float32)
    fixed = np.array(plan.fixed_indices)
    cq = np.concatenate([q[:a], bf16_normal(rng, (dyn + shift, HQ, D)) if shift else q[a:a + dyn], q[a + dyn:]])
    ck = np.concatenate([k[:a], bf16_normal(rng, (dyn + shift, HKV, D)) if shift else k[a:a + dyn], k[a + dyn:]])
    cal_fixed = np.concatenate([np.arange(a), np.arange(a + dyn + shift, n + shift)])
    cal = contextual(cq, ck, cal_fixed)[:, :, cal_fixed]
    if perturb:
        cal = np.clip(cal + rng.standard_normal(cal.shape).astype(np.float32) * perturb, 0, P - 1)
    sel = np.sort(rng.choice(fixed, n_sel, replace=False))
    ordinal_of = {int(pos): i for i, pos in enumerate(fixed)}
    dropped = {ordinal_of[int(p)] for p in rng.choice(sel, drop, replace=False)} if drop else set()
    ordinals = sorted(set(range(len(fixed))) - dropped)
    rows = np.unique(np.concatenate([sel, np.arange(a, a + dyn)]))
    rows = rows[rng.permutation(len(rows))]
    return q, k, v, e, rows, plan, cal[:, ordinals], ordinals, sel


def device_run(q, k, v, e, rows, plan, profile, mode, selected, chunk, device, monkeypatch):
    """cope_attention on the device -> (decision, kernels called); no
    visibility transform when ``selected`` is None."""
    called = []
    real = position_module.call

    def spy(name, *args):
        called.append(name)
        return real(name, *args)

    monkeypatch.setattr(position_module, "call", spy)
    cope = CoPE(D, P, device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(torch.from_numpy(e))
    policy = CanonicalPositionPolicy(plan, profile, "ckpt", mode=mode) if profile is not None else None
    visibility = (SelectedAssociationPolicy(plan.fixed_indices, torch.tensor(selected, device=device))
                  if selected is not None else None)
    as_bf16 = lambda x: torch.from_numpy(x).to(device=device, dtype=torch.bfloat16)  # noqa: E731
    try:
        out = cope_attention(as_bf16(q[rows]), as_bf16(k), as_bf16(v), cope, torch.from_numpy(rows).to(device),
                             positions_transform=policy, visibility_transform=visibility, query_chunk_size=chunk)
        result = ("ok", out)
    except CCPEPositionError as err:
        result = ("error", CCPEPositionError, str(err))
    except ValueError as err:
        result = ("error", ValueError, str(err))
    monkeypatch.setattr(position_module, "call", real)
    return result, called


def compare(expected, actual):
    assert expected[0] == actual[0], (expected[:1] + expected[1:] if expected[0] == "error" else "ok", actual[:3])
    if expected[0] == "error":
        assert expected[1] is actual[1] and expected[2] == actual[2], (expected, actual)
        return
    assert_close_bf16(actual[1], expected[1])


BIG = dict(a=700, dyn=150, b=900, n_sel=60)
# 724 fixed tokens: the profile [8, 724, 724] holds 4193408 cells, at the
# reference's max_profile_elements budget of 4194304 (config.py:19)
BUDGET = dict(a=360, dyn=100, b=364, n_sel=80)
SMALL = dict(a=40, dyn=30, b=60, n_sel=50)   # positions never saturate: the boundary pairs decide

CASES = {
    # name: (layout, seed, shift, perturb, drop, mode, chunk, expected decision)
    "same_layout_strict": (BIG, 1, 0, 0.0, 0, "strict_contextual", 64, "ok"),
    "same_layout_mixed": (BIG, 2, 0, 0.0, 0, "mixed_bias_override", 64, "ok"),
    "shifted_strict": (BIG, 3, 24, 0.0, 0, "strict_contextual", 64, "ok"),
    "shifted_mixed": (BIG, 4, 24, 0.0, 0, "mixed_bias_override", 32, "ok"),
    "perturbed_strict": (BIG, 5, 0, 0.05, 0, "strict_contextual", 48, "error"),
    "perturbed_mixed": (BIG, 6, 0, 0.5, 0, "mixed_bias_override", 128, "ok"),
    "untraced_strict": (BIG, 7, 0, 0.0, 4, "strict_contextual", 32, "error"),
    # the fixed key before the recomputed chunk against its contextual neighbour:
    # the calibration chunk was longer (gap) or its gates summed lower (order)
    "boundary_gap_strict": (SMALL, 20, 8, 0.0, 0, "strict_contextual", 16, "error"),
    "boundary_order_strict": (SMALL, 20, 4, 0.0, 0, "strict_contextual", 16, "error"),
    "boundary_mixed": (SMALL, 20, 8, 0.0, 0, "mixed_bias_override", 16, "ok"),
    "budget_strict": (BUDGET, 30, 0, 0.0, 0, "strict_contextual", 64, "ok"),
    "budget_shifted_mixed": (BUDGET, 31, 16, 0.0, 0, "mixed_bias_override", 64, "ok"),
    "budget_perturbed_strict": (BUDGET, 32, 0, 0.05, 0, "strict_contextual", 64, "error"),
}


@pytest.mark.parametrize("name", list(CASES))
def test_mfma_policy_call_matches_oracle(device, monkeypatch, name):
    """BIG: a 700-token chunk, 150 recomputed tokens, a 900-token chunk, 60
    selected fixed rows and the recomputed rows; tiles of A's fixed keys are
    skipped once a selected row's positions saturate.  SMALL: 40 + 30 + 60."""
    layout, seed, shift, perturb, drop, mode, chunk, want = CASES[name]
    q, k, v, e, rows, plan, canonical, ordinals, sel = scenario(seed, shift=shift, perturb=perturb, drop=drop,
                                                                **layout)
    strict = mode == "strict_contextual"
    if layout is BUDGET:
        assert 0.99 * 4_194_304 < canonical.size <= 4_194_304
    expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, strict, sel, chunk)
    assert expected[0] == want, expected[:3] if expected[0] == "error" else "ok"
    actual, called = device_run(q, k, v, e, rows, plan, profile_for(plan, canonical, ordinals), mode, sel, chunk,
                                device, monkeypatch)
    compare(expected, actual)
    assert "cs_ccpe_attention" not in called, called


def test_selected_rows_without_profile(device, monkeypatch):
    """Visibility policy alone (a layer without a profile): the MFMA path."""
    q, k, v, e, rows, plan, _, _, sel = scenario(9, a=500, dyn=200, b=640)
    fixed = list(plan.fixed_indices)

    def visibility(qpos, kpos):
        return orc.selected_visibility(qpos, kpos, fixed, sel)

    want = orc.cope_attention(q[rows], k, v, e, rows, visibility_transform=visibility, query_chunk_size=64)
    actual, called = device_run(q, k, v, e, rows, plan, None, "strict_contextual", sel, 64, device, monkeypatch)
    assert actual[0] == "ok"
    assert_close_bf16(actual[1], want)
    assert "cs_ccpe_attention" not in called


def test_unselected_fixed_row_on_the_mfma_path(device, monkeypatch):
    """A fixed query row outside the selected set sees every fixed key with
    its canonical position, beside selected rows that see only their own
    fixed key: one MFMA call, the oracle's result."""
    q, k, v, e, rows, plan, canonical, ordinals, sel = scenario(10, a=300, dyn=100, b=400)
    partial = sel[1:]                       # sel[0] stays an active fixed row, now not selected
    expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, False, partial, 64)
    actual, called = device_run(q, k, v, e, rows, plan, profile_for(plan, canonical, ordinals),
                                "mixed_bias_override", partial, 64, device, monkeypatch)
    compare(expected, actual)
    assert "cs_ccpe_attention" not in called, called


MID = dict(a=300, dyn=100, b=400, n_sel=60)
# fixed/dynamic boundaries off the 4-key grid: key groups that are partly
# fixed, and chunk B's ordinals not a multiple of 4 (the key-by-key reads)
ODD = dict(a=301, dyn=99, b=403, n_sel=60)

CANON_CASES = {
    # name: (layout, seed, shift, perturb, drop, mode, chunk, rows, expected decision)
    # rows "all": the calibration-layer call, every row in order with no
    # selection yet (runtime.py:448-454); "active": selected_attention "all",
    # the active rows with no visibility transform
    "calibration_strict": (MID, 41, 0, 0.0, 0, "strict_contextual", 64, "all", "ok"),
    "calibration_shifted_mixed": (MID, 42, 24, 0.0, 0, "mixed_bias_override", 64, "all", "ok"),
    "calibration_perturbed_mixed": (MID, 43, 0, 0.5, 0, "mixed_bias_override", 128, "all", "ok"),
    "calibration_perturbed_strict": (MID, 44, 0, 0.05, 0, "strict_contextual", 64, "all", "error"),
    "all_attention_strict": (BIG, 45, 0, 0.0, 0, "strict_contextual", 48, "active", "ok"),
    "all_attention_shifted_mixed": (BIG, 46, 16, 0.0, 0, "mixed_bias_override", 64, "active", "ok"),
    "all_attention_untraced_strict": (BIG, 47, 0, 0.0, 4, "strict_contextual", 32, "active", "error"),
    "odd_boundaries_calibration_mixed": (ODD, 48, 0, 0.3, 0, "mixed_bias_override", 64, "all", "ok"),
    "odd_boundaries_strict": (ODD, 49, 0, 0.0, 0, "strict_contextual", 64, "all", "ok"),
    "odd_boundaries_shifted_strict": (ODD, 49, 8, 0.0, 0, "strict_contextual", 64, "all", "error"),
    "small_boundary_gap_strict": (SMALL, 20, 8, 0.0, 0, "strict_contextual", 16, "all", "error"),
    "small_boundary_mixed": (SMALL, 20, 8, 0.0, 0, "mixed_bias_override", 16, "all", "ok"),
    "budget_strict": (BUDGET, 50, 0, 0.0, 0, "strict_contextual", 64, "all", "ok"),
}


@pytest.mark.parametrize("name", list(CANON_CASES))
def test_canonical_only_call_matches_oracle(device, monkeypatch, name):
    """A CanonicalPositionPolicy with no SelectedAssociationPolicy on the MFMA
    path: every fixed row reads all its fixed x fixed cells from the profile,
    dynamic rows keep contextual positions."""
    layout, seed, shift, perturb, drop, mode, chunk, which, want = CANON_CASES[name]
    q, k, v, e, rows, plan, canonical, ordinals, _ = scenario(seed, shift=shift, perturb=perturb, drop=drop,
                                                              **layout)
    if which == "all":
        rows = np.arange(q.shape[0])
    strict = mode == "strict_contextual"
    expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, strict, None, chunk)
    assert expected[0] == want, expected[:3] if expected[0] == "error" else "ok"
    actual, called = device_run(q, k, v, e, rows, plan, profile_for(plan, canonical, ordinals), mode, None, chunk,
                                device, monkeypatch)
    compare(expected, actual)
    assert "cs_ccpe_attention" not in called, called


def test_canonical_only_strided_profile(device, monkeypatch):
    """A profile whose key stride is not 1 (a transposed view): every cell is
    read key by key."""
    q, k, v, e, _, plan, canonical, ordinals, _ = scenario(51, **MID)
    rows = np.arange(q.shape[0])
    expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, True, None, 64)
    profile = profile_for(plan, canonical, ordinals)
    swapped = profile.canonical_positions.transpose(1, 2).contiguous().transpose(1, 2)
    assert swapped.stride(2) != 1 and torch.equal(swapped, profile.canonical_positions)
    object.__setattr__(profile, "canonical_positions", swapped)
    actual, called = device_run(q, k, v, e, rows, plan, profile, "strict_contextual", None, 64, device, monkeypatch)
    compare(expected, actual)
    assert "cs_ccpe_attention" not in called, called


def test_policy_errors_in_chunk_order(device, monkeypatch):
    """One row per chunk: a recomputed row, a fixed row whose own canonical
    cell claims 60 positions with one key available, a fixed row with an
    out-of-range cell at a future key; strict mode raises the path error of
    the first failing chunk, mixed mode the bounds error, and reordering the
    rows reorders the decision."""
    q, k, v, e, _, plan, canonical, ordinals, sel = scenario(11, a=300, dyn=100, b=400)
    fixed = list(plan.fixed_indices)
    bad_self, bad_future = 250, 500           # ordinals of two fixed rows
    canonical = canonical.copy()
    canonical[:, bad_self, bad_self] = 60.0
    canonical[:, bad_future, 650] = P + 3.0   # key fixed[650] lies after row fixed[500]
    profile = profile_for(plan, canonical, ordinals)
    sel = np.unique(np.concatenate([sel, [fixed[bad_self], fixed[bad_future]]]))
    for mode, order in (("strict_contextual", [320, fixed[bad_self], fixed[bad_future]]),
                        ("strict_contextual", [320, fixed[bad_future], fixed[bad_self]]),
                        ("mixed_bias_override", [320, fixed[bad_self], fixed[bad_future]])):
        rows = np.array(order)
        expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, mode == "strict_contextual", sel, 1)
        actual, called = device_run(q, k, v, e, rows, plan, profile, mode, sel, 1, device, monkeypatch)
        compare(expected, actual)
        assert actual[0] == "error", (mode, order)
        assert "cs_ccpe_attention" not in called


def long_case(seed, *, low_gates=False, a=1200, dyn=160, b=1200):
    """A calibration-layer call with long key walks: all rows, a
    mixed_bias_override profile of one path per head (0.3 + 0.05 h per
    token).  With ``low_gates`` the logits sit near -2.8 (gates ~0.06), so
    contextual positions stay unsaturated for ~1000 keys."""
    plan = make_plan(a, dyn, b)
    n = a + dyn + b
    rng = np.random.default_rng(seed)
    if low_gates:
        q = bf16_normal(rng, (n, HQ, D), 0.05) + 0.5
        k = bf16_normal(rng, (n, HKV, D), 0.05) - 0.5
        q = torch.from_numpy(q).to(torch.bfloat16).float().numpy()
        k = torch.from_numpy(k).to(torch.bfloat16).float().numpy()
    else:
        q, k = bf16_normal(rng, (n, HQ, D)), bf16_normal(rng, (n, HKV, D))
    v = bf16_normal(rng, (n, HKV, D))
    e = (rng.standard_normal((D, P)) * 0.1).astype(np.float32)
    nf = len(plan.fixed_indices)
    rates = (0.3 + 0.05 * np.arange(HQ)).astype(np.float32)
    o = np.arange(nf, dtype=np.float32)
    canonical = np.clip((o[None, :, None] - o[None, None, :] + 1) * rates[:, None, None], 0, P - 1)
    canonical = np.where(o[None, None, :] > o[None, :, None], np.float32(0), canonical).astype(np.float32)
    return q, k, v, e, plan, canonical, list(range(nf))


@pytest.mark.parametrize("low_gates", [False, True])
def test_long_calibration_call_matches_generic_and_oracle(device, monkeypatch, low_gates):
    """A 2560-token calibration-layer call (2 x 1200 fixed + 160 recomputed,
    every row): the MFMA path equals the generic kernel on every row and the
    oracle on sampled rows, with saturating and with slowly rising positions."""
    q, k, v, e, plan, canonical, ordinals = long_case(60 + int(low_gates), low_gates=low_gates)
    n = q.shape[0]
    rows = np.arange(n)
    profile = profile_for(plan, canonical, ordinals)
    actual, called = device_run(q, k, v, e, rows, plan, profile, "mixed_bias_override", None, 64, device,
                                monkeypatch)
    assert actual[0] == "ok" and "cs_ccpe_attention" not in called, called
    cope = CoPE(D, P, device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(torch.from_numpy(e))
    as_bf16 = lambda x: torch.from_numpy(x).to(device=device, dtype=torch.bfloat16)  # noqa: E731
    policy = CanonicalPositionPolicy(plan, profile, "ckpt", mode="mixed_bias_override")
    ref = cope_attention(as_bf16(q), as_bf16(k), as_bf16(v), cope, torch.from_numpy(rows).to(device),
                         torch.arange(n, device=device), positions_transform=policy, query_chunk_size=64)
    assert_close_bf16(actual[1], ref.float().cpu().numpy())
    pick = np.array([0, 700, 1199, 1200, 1300, 1359, 1360, 1800, 2400, n - 1])
    fixed = np.array(plan.fixed_indices)
    ords = sorted({int(np.searchsorted(fixed, p)) for p in pick if p in set(fixed.tolist())})
    expected = oracle_run(q, k, v, e, pick, plan, canonical[:, ords], ords, False, None, 64)
    assert expected[0] == "ok"
    assert_close_bf16(actual[1][torch.from_numpy(pick).to(device)], expected[1])


def test_prepare_device_is_idempotent_and_made_at_first_use(device):
    """cs_prepare_device creates the device's helper stream once; later calls
    return CS_OK and change nothing, and the package has made the call by the
    time it validated a tensor of the device."""
    from cacheslide_amd import _hip

    _hip.require_device(torch.zeros(1, device=device))
    assert device.index in _hip._PREPARED
    lib = _hip.load()
    with torch.cuda.device(device):
        assert lib.cs_prepare_device() == _hip.CS_OK
        assert lib.cs_prepare_device() == _hip.CS_OK


@pytest.mark.parametrize("drop, want", [(0.5, "error"), ("ulp", "ok")])
def test_single_cell_drop_inside_a_fixed_block(device, monkeypatch, drop, want):
    """One canonical cell of a selected row, in the block of keys 0..255 (all
    fixed and far below the row, where every cell is P-1), set below its
    right-hand neighbour: by 0.5 it breaks 'nonincreasing'; by one ulp it
    stays within the pair tolerance (1e-6 plus the rounding terms) and
    passes.  The checker screens such blocks with plain bounds and takes its
    exact checks only where a cell misses them, so both decisions must equal
    the oracle's."""
    q, k, v, e, rows, plan, canonical, ordinals, sel = scenario(61, **BIG)
    canonical = canonical.copy()
    fixed = list(plan.fixed_indices)
    r = fixed.index(int(sel[-1]))            # a selected row in the second chunk
    h, c = 3, 100
    right = np.float32(canonical[h, r, c + 1])
    assert right == P - 1
    canonical[h, r, c] = right - np.float32(0.5) if drop != "ulp" else np.nextafter(right, np.float32(0))
    expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, True, sel, 64)
    assert expected[0] == want, expected[:3] if expected[0] == "error" else "ok"
    actual, called = device_run(q, k, v, e, rows, plan, profile_for(plan, canonical, ordinals), "strict_contextual",
                                sel, 64, device, monkeypatch)
    compare(expected, actual)
    assert "cs_ccpe_attention" not in called, called


# 600 fixed + 100 recomputed + 600 fixed: the 256-key blocks of both chunks
# hold consecutive ordinals at offsets that are multiples of 4, so their cells
# are read 16 bytes per lane and screened
EDGE = dict(a=600, dyn=100, b=600, n_sel=40)


@pytest.mark.parametrize("case, mode, want", [
    ("out_of_range", "strict_contextual", "error"),
    ("nan", "strict_contextual", "error"),
    ("negative_zero", "strict_contextual", "ok"),
    ("out_of_range", "mixed_bias_override", "error"),
    ("negative_zero", "mixed_bias_override", "ok"),
])
def test_screened_block_after_the_row(device, monkeypatch, case, mode, want):
    """One canonical cell of fixed row 100, at key 300: in the block of keys
    256..511, all fixed and all after the row, which only the bounds check
    covers.  P + 2 and NaN must raise the bounds error; -0.0 (the cell's
    calibrated value is 0) passes the reference's p >= 0 although its bit
    pattern is not that of a value in [+0, P-1], so the checker's screen
    sends the block to the exact checks, which must accept it."""
    q, k, v, e, rows, plan, canonical, ordinals, sel = scenario(62, **EDGE)
    canonical = canonical.copy()
    r, h, c = 100, 5, 300                    # ordinals = positions in chunk A
    assert canonical[h, r, c] == 0.0
    canonical[h, r, c] = {"out_of_range": np.float32(P + 2), "nan": np.float32(np.nan),
                          "negative_zero": np.float32(-0.0)}[case]
    sel = np.unique(np.concatenate([sel, [r]]))
    rows = np.unique(np.concatenate([rows, [r]]))
    strict = mode == "strict_contextual"
    expected = oracle_run(q, k, v, e, rows, plan, canonical, ordinals, strict, sel, 64)
    assert expected[0] == want, expected[:3] if expected[0] == "error" else "ok"
    actual, called = device_run(q, k, v, e, rows, plan, profile_for(plan, canonical, ordinals), mode, sel, 64,
                                device, monkeypatch)
    compare(expected, actual)
    assert "cs_ccpe_attention" not in called, called


@pytest.mark.parametrize("low_gates", [False, True])
def test_key_split_selected_call_matches_generic_and_oracle(device, monkeypatch, low_gates):
    """A call long enough for the key splits, on a layer without a profile
    (SelectedAssociationPolicy alone, so no checker runs beside the
    attention): 4800 fixed keys, 256 recomputed (the question rows), 32 more
    fixed; the rows are 200 selected fixed rows of the first chunk and the 256
    question rows.  The question rows walk every causal key, so their row
    blocks are split into parts over the keys.  With saturating positions the
    parts' states are merged; with low gates (positions still rising ~1000
    keys below the diagonal) part 0 ends unsaturated and the block is walked
    again unsplit.  Both must equal the generic kernel on every row and the
    oracle on sampled rows."""
    a, dyn, b = 4800, 256, 32
    q, k, v, e, plan, _, _ = long_case(70 + int(low_gates), low_gates=low_gates, a=a, dyn=dyn, b=b)
    n = q.shape[0]
    fixed = list(plan.fixed_indices)
    sel = np.sort(np.random.default_rng(71).choice(np.arange(a), 200, replace=False))
    rows = np.concatenate([sel, np.arange(a, a + dyn)])
    actual, called = device_run(q, k, v, e, rows, plan, None, "strict_contextual", sel, 64, device, monkeypatch)
    assert actual[0] == "ok" and "cs_ccpe_attention" not in called, (actual[:3], called)
    cope = CoPE(D, P, device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(torch.from_numpy(e))
    as_bf16 = lambda x: torch.from_numpy(x).to(device=device, dtype=torch.bfloat16)  # noqa: E731
    visibility = SelectedAssociationPolicy(plan.fixed_indices, torch.tensor(sel, device=device))
    ref = cope_attention(as_bf16(q[rows]), as_bf16(k), as_bf16(v), cope, torch.from_numpy(rows).to(device),
                         torch.arange(n, device=device), visibility_transform=visibility, query_chunk_size=64)
    assert_close_bf16(actual[1], ref.float().cpu().numpy())
    pick = np.array([0, 57, 123, 199, 200, 201, 300, 383, 455])  # indices into rows

    def oracle_visibility(qpos, kpos):
        return orc.selected_visibility(qpos, kpos, fixed, sel)

    want = orc.cope_attention(q[rows[pick]], k, v, e, rows[pick], visibility_transform=oracle_visibility,
                              query_chunk_size=64)
    assert_close_bf16(actual[1][torch.from_numpy(pick).to(device)], want)
