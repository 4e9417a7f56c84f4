"""WCA kernels on the MI355X vs the reference's known answers (tests/test_wca.py)
and the fp64 oracle (bit-exact deviations, weights, selections and blends)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd import (
    WCAConfig,
    WCANumericalError,
    WCAState,
    adaptation_weight,
    mean_head_cosine,
    squared_deviation,
)
from oracle import wca as orc
from tests._helpers import seeded

pytestmark = pytest.mark.gpu


def make_state(device, config=None):
    # tests/test_wca.py:14-20
    cached = torch.ones(6, 1, 2, device=device)
    fresh = torch.tensor([5, 4, 3, 2, 1, 100.0], device=device)[:, None, None].expand_as(cached).contiguous()
    reused = torch.tensor([True, True, True, True, True, False], device=device)
    state = WCAState.initialize(cached, fresh, reused, ~reused, config)
    return state, cached, fresh, reused, ~reused


def test_budget_and_selection(device):
    # tests/test_wca.py:23-32
    state, _, _, reused, mandatory = make_state(device)
    assert state.budget == 2
    assert state.selected_indices.tolist() == [0, 1]
    assert state.active_indices.tolist() == [0, 1, 5]
    assert state.candidate_mask.tolist() == [True, True, True, True, False, False]
    reused[:] = False
    assert state.reused_mask.sum() == 5


def test_zero_errors_and_ties(device):
    # tests/test_wca.py:35-43
    cached = torch.ones(7, 2, 3, device=device)
    mask = torch.ones(7, dtype=torch.bool, device=device)
    state = WCAState.initialize(cached, cached + 1, mask, ~mask)
    assert state.selected_indices.tolist() == [0, 1]
    assert torch.equal(squared_deviation(cached, cached + 1).cpu(), torch.full((7,), 6.0, dtype=torch.float64))
    empty = WCAState.initialize(cached, cached, mask, ~mask)
    assert empty.budget == 0 and empty.active_indices.numel() == 0


def test_weight_known_answers(device):
    # tests/test_wca.py:46-60
    cached = torch.zeros(1, 1, 2, dtype=torch.float16, device=device)
    fresh = torch.ones_like(cached)
    alpha = adaptation_weight(cached, fresh, epsilon=0.5)
    assert alpha.dtype == torch.float64 and alpha.item() == 4
    assert adaptation_weight(cached, fresh, epsilon=0.5, clamp=True).item() == 1
    assert adaptation_weight(cached, cached).item() == 0
    huge = torch.full((1, 1, 2), 1e30, device=device)
    assert adaptation_weight(huge, 2 * huge).item() == pytest.approx(1.0)
    with pytest.raises(WCANumericalError, match="overflow"):
        adaptation_weight(torch.zeros(1, 1, 1, dtype=torch.float64, device=device),
                          torch.full((1, 1, 1), 1e308, dtype=torch.float64, device=device))


@pytest.mark.parametrize("mode, expected_alpha", [("previous_layer", 4), ("same_layer", 1)])
def test_weight_order(device, mode, expected_alpha):
    # tests/test_wca.py:63-85
    cached = torch.ones(2, 1, 1, device=device)
    reused = torch.tensor([True, False], device=device)
    state = WCAState.initialize(cached, torch.tensor([3.0, 9.0], device=device)[:, None, None], reused,
                                ~reused, WCAConfig(correction_fraction=1, epsilon=1e-20, weight_update=mode))
    result = state.update(2, cached, cached * 2, torch.tensor([2.0, 7.0], device=device)[:, None, None],
                          torch.tensor([4.0, 8.0], device=device)[:, None, None])
    assert result.alpha.tolist() == pytest.approx([expected_alpha, 1])
    assert result.fused_k[:, 0, 0].tolist() == pytest.approx([1 + expected_alpha, 7])
    assert result.fused_v[:, 0, 0].tolist() == pytest.approx([2 + 2 * expected_alpha, 8])
    assert state.alpha[0].item() == pytest.approx(1)


def test_literal_gate(device):
    # tests/test_wca.py:88-101
    state, cached, _, _, _ = make_state(device, WCAConfig(gate_interval=2))
    rows = state.active_indices
    result = state.update(2, cached, cached, -cached[rows], cached[rows])
    assert result.removed_indices.tolist() == [0, 1]
    assert result.promoted_indices.tolist() == [2, 3]
    assert result.next_indices.tolist() == [2, 3, 5]
    assert not state.candidate_mask[:2].any()
    rows = state.active_indices
    state.update(3, cached, cached, -cached[rows], cached[rows])
    result = state.update(4, cached, cached, -cached[rows], cached[rows])
    assert result.removed_indices.tolist() == [2, 3]
    assert result.promoted_indices.numel() == 0
    assert result.next_indices.tolist() == [5]


def test_distance_gate(device):
    # tests/test_wca.py:104-114
    literal, cached, _, _, _ = make_state(device)
    distance, _, _, _, _ = make_state(device, WCAConfig(convergence_mode="distance_lt"))
    for layer in (2, 3, 4):
        for state in (literal, distance):
            rows = state.active_indices
            result = state.update(layer, cached, cached, cached[rows], cached[rows])
            if layer < 4:
                assert result.removed_indices.numel() == 0
    assert literal.selected_indices.tolist() == [0, 1]
    assert distance.selected_indices.tolist() == [2, 3]


def test_cosine_zero_heads(device):
    # tests/test_wca.py:117-120
    a = torch.tensor([[[1.0, 0], [0, 1]], [[0, 0], [0, 0]]], device=device)
    b = torch.tensor([[[1.0, 0], [0, -1]], [[1, 1], [1, 1]]], device=device)
    assert mean_head_cosine(a, b).tolist() == [0, 0]


def test_sparse_identity_validation(device):
    # tests/test_wca.py:123-134
    first, cached, _, _, _ = make_state(device, WCAConfig(gate_interval=2))
    second, _, _, _, _ = make_state(device, WCAConfig(gate_interval=2))
    rows = first.active_indices
    first.update(2, cached, cached, -cached[rows], cached[rows])
    assert second.selected_indices.tolist() == [0, 1]
    with pytest.raises(ValueError, match="computed_indices"):
        second.update(2, cached, cached, cached[rows], cached[rows], rows.flip(0))
    with pytest.raises(ValueError, match="computed_indices"):
        second.update(2, cached, cached, cached[rows], cached[rows], rows[:1])
    # the device-side mismatch left the state as it was
    assert second.selected_indices.tolist() == [0, 1] and second.last_layer == 1
    with pytest.raises(ValueError, match="consecutively"):
        second.update(3, cached, cached, cached[rows], cached[rows])
    with pytest.raises(ValueError, match="shape, dtype"):
        second.update(2, cached, cached, cached, cached)


def test_mandatory_rows_fresh(device):
    # tests/test_wca.py:137-144
    cached = torch.ones(3, 1, 1, device=device)
    reused = torch.tensor([True, True, False], device=device)
    mandatory = torch.tensor([False, True, True], device=device)
    state = WCAState.initialize(cached, cached + 2, reused, mandatory)
    result = state.update(2, cached, cached, cached * 2, cached * 3)
    assert result.fused_k[1:, 0, 0].tolist() == [2, 2]
    assert result.fused_v[1:, 0, 0].tolist() == [3, 3]


def test_invalid_masks_and_transactional_overflow(device):
    # tests/test_wca.py:147-168
    cached = torch.ones(1, 1, 1, device=device)
    with pytest.raises(ValueError, match="mandatory"):
        WCAState.initialize(cached, cached, torch.tensor([False], device=device),
                            torch.tensor([False], device=device))
    with pytest.raises(WCANumericalError, match="finite"):
        adaptation_weight(cached, cached * torch.nan)
    half = torch.zeros(1, 1, 1, dtype=torch.float16, device=device)
    state = WCAState.initialize(half, half + 1, torch.tensor([True], device=device),
                                torch.tensor([False], device=device))
    initial = {n: getattr(state, n).clone() for n in ("alpha", "candidate_mask", "selected_mask", "removed_mask")}
    with pytest.raises(WCANumericalError, match="overflow"):
        state.update(2, half, half, half + 1, half + 1)
    assert state.last_layer == 1
    assert state.selected_indices.tolist() == [0]
    for name, value in initial.items():
        assert torch.equal(getattr(state, name), value)


def test_float64_overflow_messages(device):
    # tests/test_wca.py:221-231
    zero = torch.zeros(1, 1, 1, dtype=torch.float64, device=device)
    huge = torch.full_like(zero, 1e308)
    with pytest.raises(WCANumericalError, match="deviation overflow"):
        squared_deviation(zero, huge)
    with pytest.raises(WCANumericalError, match="weight overflow"):
        adaptation_weight(huge, huge)
    with pytest.raises(WCANumericalError, match="weight overflow"):
        adaptation_weight(zero, zero + 1, epsilon=1e-320)


# ------------------------------------------------------------ seeded vs oracle
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_wca_trajectory_bit_exact_vs_oracle(device, dtype):
    """Eight layers of WCA on drifted bf16 KV: deviations, weights, selections,
    removals/promotions and fused K/V identical to the fp64 oracle."""
    T, H, D = 700, 8, 128
    name = "bfloat16" if dtype == torch.bfloat16 else "float32"
    fresh = seeded((T, H, D), 200, dtype=dtype)
    cached = (fresh.double() + seeded((T, H, D), 201, scale=0.05).double()).to(dtype)
    reused = torch.ones(T, dtype=torch.bool)
    reused[600:640] = False
    mandatory = ~reused
    mandatory[-1] = True
    cfg = dict(fraction=0.15, gate_interval=2, threshold=0.999)
    ost = orc.State(cached.double().numpy(), fresh.double().numpy(), reused.numpy(), mandatory.numpy(),
                    dtype=name, **cfg)
    dst = WCAState.initialize(cached.to(device), fresh.to(device), reused.to(device), mandatory.to(device),
                              WCAConfig(correction_fraction=0.15, gate_interval=2, convergence_threshold=0.999))
    np.testing.assert_array_equal(dst.initial_deviation.cpu().numpy(), ost.initial)
    np.testing.assert_array_equal(dst.alpha.cpu().numpy(), ost.alpha)
    assert dst.selected_indices.tolist() == np.flatnonzero(ost.selected).tolist()
    for layer in range(2, 10):
        ck = seeded((T, H, D), 300 + layer, dtype=dtype)
        cv = seeded((T, H, D), 400 + layer, dtype=dtype)
        idx = ost.active
        rk = (ck[idx].double() + seeded((len(idx), H, D), 500 + layer, scale=0.3).double()).to(dtype)
        rv = (cv[idx].double() + seeded((len(idx), H, D), 600 + layer, scale=0.3).double()).to(dtype)
        o_idx, ofk, ofv, oused, orem, oprom, onext = ost.update(
            layer, ck.double().numpy(), cv.double().numpy(), rk.double().numpy(), rv.double().numpy())
        res = dst.update(layer, ck.to(device), cv.to(device), rk.to(device), rv.to(device))
        assert res.indices.tolist() == o_idx.tolist()
        np.testing.assert_array_equal(res.alpha.cpu().numpy(), oused)
        np.testing.assert_array_equal(res.fused_k.double().cpu().numpy(), ofk)
        np.testing.assert_array_equal(res.fused_v.double().cpu().numpy(), ofv)
        assert res.removed_indices.tolist() == orem.tolist()
        assert res.promoted_indices.tolist() == oprom.tolist()
        assert res.next_indices.tolist() == onext.tolist()
        np.testing.assert_array_equal(dst.alpha.cpu().numpy(), ost.alpha)


def test_promotion_ties_and_large_budget(device):
    """Many equal deviations: the stable order (descending, lower index first)."""
    T = 5000
    rng = np.random.default_rng(12)
    levels = rng.integers(0, 6, T).astype(np.float64)  # heavy ties
    fresh = torch.from_numpy(np.sqrt(levels)[:, None, None]).float()
    cached = torch.zeros((T, 1, 1))
    reused = torch.ones(T, dtype=torch.bool)
    mandatory = torch.zeros(T, dtype=torch.bool)
    mandatory[-1] = True
    ost = orc.State(cached.double().numpy(), fresh.double().numpy(), reused.numpy(), mandatory.numpy(),
                    fraction=0.4)
    dst = WCAState.initialize(cached.to(device), fresh.to(device), reused.to(device), mandatory.to(device),
                              WCAConfig(correction_fraction=0.4))
    assert dst.budget == ost.budget
    assert dst.selected_indices.tolist() == np.flatnonzero(ost.selected).tolist()
    fresh_order = ost.promote  # the promoted order is checked through _promote below
    dst.selected_mask.zero_()
    ost.selected[:] = False
    promoted_dev = dst._promote().tolist()
    promoted_orc = fresh_order().tolist()
    assert promoted_dev == promoted_orc


def test_bf16_head_cosine_matches_oracle(device):
    """bf16 rows take the vectorised cosine kernel: same values as the fp64
    oracle up to summation order, including zero heads and the clamp."""
    a = seeded((300, 8, 128), 700, dtype=torch.bfloat16)
    b = (a.double() + seeded((300, 8, 128), 701, scale=0.5).double()).to(torch.bfloat16)
    a[3] = 0  # all-zero rows: eps scaling, cosine 0
    b[4] = a[4]  # identical rows: cosine clamps at 1
    got = mean_head_cosine(a.to(device), b.to(device)).cpu().numpy()
    want = orc.mean_head_cosine(a.double().numpy(), b.double().numpy())
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-14)
    assert got[3] == 0.0 and abs(got[4] - 1.0) < 1e-14


def test_promotion_multi_chunk_beyond_lds_rank(device):
    """40000 tokens (three selection chunks) and a budget of 10400 (ranked
    from global memory): same selection and promotion order as the oracle."""
    T = 40000
    rng = np.random.default_rng(13)
    levels = rng.integers(0, 300, T).astype(np.float64)  # ties across chunks
    fresh = torch.from_numpy(np.sqrt(levels)[:, None, None]).float()
    cached = torch.zeros((T, 1, 1))
    reused = torch.ones(T, dtype=torch.bool)
    reused[T - 5:] = False
    mandatory = ~reused
    ost = orc.State(cached.double().numpy(), fresh.double().numpy(), reused.numpy(), mandatory.numpy(),
                    fraction=0.26)
    dst = WCAState.initialize(cached.to(device), fresh.to(device), reused.to(device), mandatory.to(device),
                              WCAConfig(correction_fraction=0.26))
    assert dst.budget == ost.budget > 4096
    assert dst.selected_indices.tolist() == np.flatnonzero(ost.selected).tolist()
    assert dst.active_indices.tolist() == ost.active.tolist()
    dst.selected_mask.zero_()  # in-place change: the cached active indices must be recounted
    ost.selected[:] = False
    assert dst.active_indices.tolist() == ost.active.tolist()
    assert dst._promote().tolist() == ost.promote().tolist()
    assert dst.active_indices.tolist() == ost.active.tolist()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64])
def test_finite_check_vector_path(device, dtype):
    """Contiguous tensors are checked 16 bytes at a time: one inf or NaN anywhere
    (first, last, middle element) is found; finite extremes are not flagged."""
    x = seeded((513, 8, 128), 702, dtype=dtype).to(device)
    x[7, 3, 5] = torch.finfo(dtype).max
    x[8, 0, 0] = -torch.finfo(dtype).max
    squared_deviation(x, x.clone())  # finite extremes pass the check
    for where, bad in (((0, 0, 0), float("inf")), ((512, 7, 127), float("nan")),
                       ((300, 4, 64), float("-inf"))):
        y = x.clone()
        y[where] = bad
        with pytest.raises(WCANumericalError, match="cached_k must have finite values"):
            squared_deviation(y, x)


@pytest.mark.parametrize("weight_update, mode, dtype", [
    ("previous_layer", "paper_cosine_lt", torch.bfloat16),
    ("same_layer", "distance_lt", torch.float32),
])
def test_single_call_update_equals_checked_update(device, weight_update, mode, dtype):
    """update() makes its device work one cs_wca_update call when the host checks
    pass; it must equal the step-by-step checked path bit for bit."""
    gen = torch.Generator().manual_seed(77)
    T, H, D = 600, 2, 64
    fresh = torch.randn(T, H, D, generator=gen)
    cached = (fresh + 0.05 * torch.randn(T, H, D, generator=gen)).to(dtype).to(device)
    fresh = fresh.to(dtype).to(device)
    reused = torch.ones(T, dtype=torch.bool, device=device)
    reused[-3:] = False
    config = WCAConfig(weight_update=weight_update, convergence_mode=mode, gate_interval=2,
                       convergence_threshold=0.999 if mode == "paper_cosine_lt" else 0.001)
    fast = WCAState.initialize(cached, fresh, reused, ~reused, config)
    slow = WCAState.initialize(cached, fresh, reused, ~reused, config)
    for layer in range(2, 8):
        layer_fresh = fresh * (1 + 0.01 * layer)
        rows = fast.active_indices
        assert torch.equal(rows, slow.active_indices)
        rk, rv = layer_fresh[rows], (2 * layer_fresh)[rows]
        a = fast.update(layer, cached, cached * 0.5, rk, rv, computed_indices=rows.clone())
        b = slow._update_checked(layer, device, cached, cached * 0.5, rk, rv, rows.clone())
        for name in ("indices", "fused_k", "fused_v", "alpha", "removed_indices", "promoted_indices",
                     "next_indices"):
            x, y = getattr(a, name), getattr(b, name)
            assert x.dtype == y.dtype and torch.equal(x, y), (layer, name)
        for name in ("alpha", "selected_mask", "candidate_mask", "removed_mask"):
            assert torch.equal(getattr(fast, name), getattr(slow, name)), (layer, name)
    # a failing device check still rolls the single call back: nothing is committed
    rows = fast.active_indices
    before = (fast.alpha.clone(), fast.selected_mask.clone(), fast.last_layer)
    bad = fresh[rows].clone()
    bad[0, 0, 0] = float("nan")
    with pytest.raises(WCANumericalError, match="recomputed_k must have finite values"):
        fast.update(fast.last_layer + 1, cached, cached, bad, fresh[rows])
    assert torch.equal(fast.alpha, before[0]) and torch.equal(fast.selected_mask, before[1])
    assert fast.last_layer == before[2]


def test_single_call_update_follows_the_current_stream(device):
    """Each update launches on the caller's current stream at that call: inputs
    produced on a side stream just before the update are read complete."""
    gen = torch.Generator().manual_seed(91)
    T, H, D = 4096, 8, 128
    fresh = torch.randn(T, H, D, generator=gen).to(torch.bfloat16).to(device)
    cached = (fresh.float() + 0.05).to(torch.bfloat16)
    reused = torch.ones(T, dtype=torch.bool, device=device)
    config = WCAConfig(gate_interval=2)
    fast = WCAState.initialize(cached, fresh, reused, ~reused, config)
    slow = WCAState.initialize(cached, fresh, reused, ~reused, config)
    side = torch.cuda.Stream(device)
    for layer in range(2, 6):
        rows = fast.active_indices
        stream = side if layer % 2 else torch.cuda.current_stream(device)
        with torch.cuda.stream(stream):
            # produced on the stream the update then runs on
            big = (fresh.float() * (1 + 0.01 * layer)).to(torch.bfloat16)
            rk, rv = big[rows], (2 * big)[rows]
            a = fast.update(layer, cached, cached, rk, rv)
            b = slow._update_checked(layer, device, cached, cached, rk, rv, None)
        torch.cuda.synchronize(device)
        for name in ("fused_k", "fused_v", "alpha", "removed_indices", "promoted_indices", "next_indices"):
            assert torch.equal(getattr(a, name), getattr(b, name)), (layer, name)


def test_fused_update_checks_raise_in_reference_order(device):
    """The single-launch checks of cached K/V, the computed rows and recomputed
    K/V raise their own errors, the first in the reference's order when several
    fire, and commit nothing."""
    gen = torch.Generator().manual_seed(5)
    cached = torch.randn(300, 2, 16, generator=gen).to(torch.bfloat16).to(device)
    fresh = (cached.float() + 0.1).to(torch.bfloat16)
    reused = torch.ones(300, dtype=torch.bool, device=device)
    reused[-1] = False
    state = WCAState.initialize(cached, fresh, reused, ~reused)
    rows = state.active_indices
    rk, rv = fresh[rows], fresh[rows]
    bad_rows = rows.clone()
    bad_rows[3] += 1

    def nan(t, at):
        t = t.clone()
        t.view(-1)[at] = float("nan")
        return t

    cases = [
        (dict(cached_k=nan(cached, 7)), WCANumericalError, "cached_k must have finite values"),
        (dict(cached_v=nan(cached, 9000)), WCANumericalError, "cached_v must have finite values"),
        (dict(computed=bad_rows), ValueError, "computed_indices must equal"),
        (dict(rk=nan(rk, 1)), WCANumericalError, "recomputed_k must have finite values"),
        (dict(rv=nan(rv, rv.numel() - 1)), WCANumericalError, "recomputed_v must have finite values"),
        # several at once: the first check in the reference's order wins
        (dict(cached_v=nan(cached, 5), computed=bad_rows, rk=nan(rk, 0)), WCANumericalError,
         "cached_v must have finite values"),
        (dict(computed=bad_rows, rv=nan(rv, 2)), ValueError, "computed_indices must equal"),
    ]
    alpha, selected = state.alpha.clone(), state.selected_mask.clone()
    for overrides, exc, message in cases:
        args = dict(cached_k=cached, cached_v=cached, rk=rk, rv=rv, computed=rows.clone())
        args.update(overrides)
        assert state._inputs_pass(args["cached_k"], args["cached_v"], args["rk"], args["rv"], args["computed"])
        with pytest.raises(exc, match=message):
            state.update(2, args["cached_k"], args["cached_v"], args["rk"], args["rv"],
                         computed_indices=args["computed"])
        assert torch.equal(state.alpha, alpha) and torch.equal(state.selected_mask, selected)
        assert state.last_layer == 1
    result = state.update(2, cached, cached, rk, rv, computed_indices=rows.clone())
    assert result.fused_k.shape == rk.shape and state.last_layer == 2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,fraction", [(1, 0.15), (700, 0.15), (5000, 0.5), (16384, 0.15), (20000, 0.3)])
def test_single_call_initialize_equals_checked_initialize(device, monkeypatch, dtype, n, fraction):
    """initialize makes its device work one cs_wca_initialize call (budget on
    the device, one readback) when the host checks pass; every field of the
    state equals the step-by-step path's, bit for bit."""
    import cacheslide_amd.wca as wca_mod

    gen = torch.Generator().manual_seed(n)
    cached = torch.randn(n, 2, 16, generator=gen).to(dtype)
    fresh = (cached.float() + 0.05 * torch.randn(n, 2, 16, generator=gen)).to(dtype)
    fresh[: n // 7] = cached[: n // 7]  # zero deviations: not candidates
    cached, fresh = cached.to(device), fresh.to(device)
    reused = torch.rand(n, generator=gen).to(device) < 0.97
    config = WCAConfig(correction_fraction=fraction, clamp_alpha=n % 2 == 0)
    calls = []
    real = wca_mod.call

    def spy(name, *args):
        calls.append(name)
        return real(name, *args)

    monkeypatch.setattr(wca_mod, "call", spy)
    fast = WCAState.initialize(cached, fresh, reused, ~reused, config)
    assert calls == ["cs_wca_initialize"]
    monkeypatch.setattr(wca_mod, "_initialize_inputs_pass", lambda *a: False)
    slow = WCAState.initialize(cached, fresh, reused, ~reused, config)
    assert "cs_wca_initialize" not in calls[1:]
    assert fast.budget == slow.budget
    for name in ("initial_deviation", "alpha", "candidate_mask", "selected_mask", "removed_mask",
                 "reused_mask", "mandatory_mask"):
        a, b = getattr(fast, name), getattr(slow, name)
        assert a.dtype == b.dtype and a.shape == b.shape, name
        if a.dtype == torch.float64:
            assert torch.equal(a.view(torch.int64), b.view(torch.int64)), name
        else:
            assert torch.equal(a, b), name
    assert torch.equal(fast.active_indices, slow.active_indices)
    # and the states continue alike
    idx = fast.active_indices
    u1 = fast.update(2, cached, cached, fresh[idx], fresh[idx])
    u2 = slow.update(2, cached, cached, fresh[idx], fresh[idx])
    assert torch.equal(u1.next_indices, u2.next_indices) and torch.equal(u1.fused_k, u2.fused_k)


def test_single_call_initialize_raises_in_reference_order(device):
    """The one-call initialize raises the checked path's first error."""
    cached = torch.randn(300, 2, 16, device=device)
    fresh = cached + 0.1
    reused = torch.ones(300, dtype=torch.bool, device=device)
    reused[-1] = False
    bad = cached.clone()
    bad[5, 1, 3] = float("nan")
    with pytest.raises(WCANumericalError, match="cached_k must have finite values"):
        WCAState.initialize(bad, fresh, reused, ~reused)
    with pytest.raises(WCANumericalError, match="recomputed_k must have finite values"):
        WCAState.initialize(cached, bad, reused, ~reused)
    # NaN in cached K and a token neither reused nor mandatory: the finite check first
    none = torch.zeros(300, dtype=torch.bool, device=device)
    with pytest.raises(WCANumericalError, match="cached_k must have finite values"):
        WCAState.initialize(bad, fresh, reused, none)
    with pytest.raises(ValueError, match="mandatory"):
        WCAState.initialize(cached, fresh, reused, none)
    huge = torch.full((4, 1, 1), 1e308, dtype=torch.float64, device=device)
    with pytest.raises(WCANumericalError, match="deviation overflow"):
        WCAState.initialize(torch.zeros_like(huge), huge, reused[:4], ~reused[:4])
    state = WCAState.initialize(cached, fresh, reused, ~reused)
    # ceil(0.26 * 299) = 78 of 299 candidates, plus the mandatory token
    assert state.budget == 78 and state.active_indices.numel() == 79
