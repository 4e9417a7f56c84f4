"""Pins the CPU oracle (oracle/) against the reference's own known answers.

Every vector here is a closed form from the reference test-suite (file:line
cited), a brute-force / textbook restatement, or a library reduction, chosen
so that a dropped term, sign or index in the oracle fails at least one case.
CPU only.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ccpe, rows, slide, wca


def f32(x):
    return np.asarray(x, dtype=np.float32)


# ---------------------------------------------------------------- positions
def test_gate_masking_reverse_cumsum_and_clamp():
    # tests/test_position.py:16-23
    logits = np.zeros((1, 3, 3), np.float32)
    allowed = np.tril(np.ones((3, 3), bool))[None]
    logits[~allowed] = 1000
    p = ccpe.contextual_positions(logits, allowed, 2)
    np.testing.assert_array_equal(p, f32([[[0.5, 0, 0], [1, 0.5, 0], [1, 1, 0.5]]]))


def test_interpolation_known_answer():
    # tests/test_position.py:26-35: E = [0, 2, 6, 10], q = 2, p = [.25, 1.5, 3] -> [1, 8, 20]
    e = np.array([[0, 2, 6, 10]], np.float64)
    q = np.array([[[2.0]]])
    p = np.array([[[0.25, 1.5, 3.0]]])
    np.testing.assert_allclose(ccpe.positional_bias(q, e, p), [[[1, 8, 20]]])


def test_linear_table_bias_equals_position_including_top_knot():
    # tests/test_position.py:48-62
    e = np.arange(4, dtype=np.float64)[None]
    q = np.ones((1, 1, 1))
    p = np.array([[[0.0, 1.0, 2.0, 2.5, 3.0]]])
    np.testing.assert_allclose(ccpe.positional_bias(q, e, p), p)


def test_two_causal_sigmoid_zero_gates_give_position_one():
    # tests/test_position.py:65-77
    q = np.ones((1, 1, 1))
    k = np.zeros((3, 1, 1))
    lg = ccpe.logits(q, k)
    allowed = ccpe.allowed_mask(np.array([1]), np.arange(3), 1)
    p = ccpe.contextual_positions(lg, allowed, 4)
    assert p[0, 0, 0] == 1.0 and p[0, 0, 2] == 0.0


def test_attention_matches_textbook_loop_gqa_arbitrary_rows():
    # tests/test_position.py:99-115 (dense_reference is the reference's own oracle)
    rng = np.random.default_rng(3)
    e = rng.standard_normal((3, 7))
    q = rng.standard_normal((3, 4, 3))
    k = rng.standard_normal((6, 2, 3))
    v = rng.standard_normal((6, 2, 5))
    qpos, kpos = np.array([4, 1, 5]), np.arange(6)
    expected = ccpe.dense_reference(q, k, v, e, qpos, kpos, 7)
    out, trace = ccpe.cope_attention(q, k, v, e, qpos, query_chunk_size=1, return_positions=True)
    np.testing.assert_allclose(out, expected, rtol=1e-12, atol=1e-12)
    assert trace.shape == (4, 3, 6)
    decode = ccpe.cope_attention(q[-1:], k, v, e, np.array([5]))
    np.testing.assert_allclose(decode, expected[-1:], rtol=1e-12, atol=1e-12)


def test_future_keys_do_not_change_earlier_rows():
    # tests/test_position.py:118-128
    rng = np.random.default_rng(8)
    e = rng.standard_normal((2, 6)).astype(np.float32)
    q, k, v = (rng.standard_normal((4, 2, 2)).astype(np.float32) for _ in range(3))
    base = ccpe.cope_attention(q, k, v, e, np.arange(4))
    k2, v2 = k.copy(), v.copy()
    k2[2:] *= -100
    v2[2:] += 100
    changed = ccpe.cope_attention(q, k2, v2, e, np.arange(4))
    np.testing.assert_allclose(changed[:2], base[:2], rtol=1e-6)


def test_all_masked_rows_are_zero():
    # tests/test_position.py:131-137
    q = k = v = np.ones((2, 1, 2), np.float32)
    mask = np.array([[False, False], [True, True]])
    out = ccpe.cope_attention(q, k, v, np.zeros((2, 4), np.float32), np.arange(2), attention_mask=mask)
    assert np.abs(out[0]).sum() == 0 and np.isfinite(out).all()


def test_visibility_after_gates_known_answer():
    # tests/test_position.py:146-171: output 50.5, trace [1.5, 1, .5]; as a gate mask p[0] = 1
    q, k = np.ones((1, 1, 1), np.float32), np.zeros((3, 1, 1), np.float32)
    v = np.array([1.0, 10.0, 100.0], np.float32)[:, None, None]
    vis = np.array([[True, False, True]])
    e = np.zeros((1, 8), np.float32)
    out, trace = ccpe.cope_attention(q, k, v, e, np.array([2]), visibility_mask=vis, return_positions=True)
    assert out.item() == 50.5
    np.testing.assert_array_equal(trace, f32([[[1.5, 1.0, 0.5]]]))
    _, masked = ccpe.cope_attention(q, k, v, e, np.array([2]), attention_mask=vis, return_positions=True)
    assert masked[0, 0, 0] == 1


def test_selected_association_known_answers():
    # tests/test_attention_policies.py:131-153
    queries, keys = np.array([4, 1, 2]), np.arange(6)
    mask = ccpe.selected_visibility(queries, keys, (0, 2, 4), np.array([4, 2]))
    assert mask.tolist() == [
        [False, True, False, True, True, True],
        [True, True, True, True, True, True],
        [False, True, True, True, False, True],
    ]
    q = np.ones((3, 1, 1))
    k = np.zeros((6, 1, 1))
    v = np.arange(6, dtype=np.float64)[:, None, None]
    out = ccpe.cope_attention(
        q, k, v, np.zeros((1, 16)), queries,
        visibility_transform=lambda qq, kk: ccpe.selected_visibility(qq, kk, (0, 2, 4), np.array([4, 2])),
        query_chunk_size=1,
    )
    np.testing.assert_allclose(out[:, 0, 0], [8 / 3, 0.5, 1.5])


def test_wca_association_applied_after_gates_known_answer():
    # tests/test_attention_policies.py:156-190
    e = np.arange(16, dtype=np.float64)[None]
    q, k = np.ones((1, 1, 1)), np.zeros((5, 1, 1))
    v = np.array([1, 10, 100, 1000, 10000], np.float64)[:, None, None]
    queries, keys = np.array([4]), np.arange(5)
    assoc = lambda qq, kk: ccpe.selected_visibility(qq, kk, (0, 2, 4), np.array([4]))
    out, pos = ccpe.cope_attention(q, k, v, e, queries, visibility_transform=assoc, return_positions=True)
    np.testing.assert_allclose(pos, [[[2.5, 2, 1.5, 1, 0.5]]])
    visible = assoc(queries, keys)[0]
    p = pos[0, 0, visible]
    expected = (np.exp(p - p.max()) / np.exp(p - p.max()).sum()) @ v[visible, 0, 0]
    np.testing.assert_allclose(out[0, 0, 0], expected)
    _, wrong = ccpe.cope_attention(q, k, v, e, queries, attention_mask=assoc(queries, keys), return_positions=True)
    assert wrong[0, 0, 1] == 1.5


def test_library_reduction_zero_table_is_causal_softmax_attention():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((40, 4, 16)).astype(np.float32)
    k = rng.standard_normal((40, 2, 16)).astype(np.float32)
    v = rng.standard_normal((40, 2, 16)).astype(np.float32)
    out = ccpe.cope_attention(q, k, v, np.zeros((16, 8), np.float32), np.arange(40))
    kk = torch.from_numpy(np.repeat(k, 2, 1)).permute(1, 0, 2)
    vv = torch.from_numpy(np.repeat(v, 2, 1)).permute(1, 0, 2)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).permute(1, 0, 2), kk, vv, is_causal=True
    ).permute(1, 0, 2)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-5, atol=1e-5)


def test_saturated_cells_take_the_last_table_entry():
    # gates ~1 and P = 4: all but the last few causal keys of a row sit at p = P-1,
    # where lower = upper = P-1 and frac = 0, so the bias is exactly QE[P-1]
    rng = np.random.default_rng(6)
    d = 8
    q = np.abs(rng.standard_normal((30, 1, d))) * 4
    k = np.abs(rng.standard_normal((30, 1, d))) * 4
    e = rng.standard_normal((d, 4))
    lg = ccpe.logits(q, k)
    allowed = ccpe.allowed_mask(np.arange(30), np.arange(30), 1)
    p = ccpe.contextual_positions(lg, allowed, 4)
    sat = (p == 3) & allowed
    assert sat.sum() > 300
    bias = ccpe.positional_bias(q, e, p)
    table = ccpe.qe_table(q, e)
    np.testing.assert_array_equal(bias[sat], np.broadcast_to(table[..., 3:4], p.shape)[sat])


def test_identical_table_columns_reduce_to_plain_attention():
    # QE[p] is then the same for every p: a per-row constant that softmax cancels
    rng = np.random.default_rng(7)
    q = rng.standard_normal((25, 2, 8))
    k = rng.standard_normal((25, 1, 8))
    v = rng.standard_normal((25, 1, 8))
    column = rng.standard_normal((8, 1))
    out = ccpe.cope_attention(q, k, v, np.repeat(column, 5, axis=1), np.arange(25))
    plain = ccpe.cope_attention(q, k, v, np.zeros((8, 5)), np.arange(25))
    np.testing.assert_allclose(out, plain, rtol=1e-12, atol=1e-12)


def test_float32_cumsum_accumulates_in_float64():
    # 2^24 + 1 style: float32 sequential sums lose the small gates, fp64 keeps them
    logits = np.full((1, 1, 5), -50.0, np.float32)
    logits[..., -1] = 30.0
    p = ccpe.contextual_positions(logits, np.ones_like(logits, bool), 8)
    g = ccpe.sigmoid(logits)
    expected = np.flip(np.cumsum(np.flip(g.astype(np.float64), -1), -1), -1).astype(np.float32)
    np.testing.assert_array_equal(p, expected)


# ---------------------------------------------------------------- validation
def test_validation_accepts_genuine_and_rejects_available():
    # tests/test_position.py:174-187
    q = np.ones((3, 4, 2), np.float32)
    k = np.zeros((5, 2, 2), np.float32)
    qpos, kpos = np.array([4, 0, 2]), np.arange(5)
    allowed = ccpe.allowed_mask(qpos, kpos, 4)
    p = ccpe.contextual_positions(ccpe.logits(q, k), allowed, 3)
    ccpe.validate_contextual_path(p, qpos, kpos)
    p2 = np.where(allowed, p, np.float32(0.75))
    ccpe.validate_contextual_path(p2, qpos, kpos)
    p2[0, 1, 0] = 1.1
    with pytest.raises(ccpe.PathError) as err:
        ccpe.validate_contextual_path(p2, qpos, kpos)
    assert err.value.kind == "available"


def test_validation_rejects_hybrid_nonmonotonic():
    # tests/test_position.py:190-209
    hybrid = f32([[[1.5, 2, 1.5, 1, 0.5]]])
    with pytest.raises(ccpe.PathError) as err:
        ccpe.validate_contextual_path(hybrid, np.array([4]), np.arange(5))
    assert err.value.kind == "nonincreasing"


def test_validation_sparse_coordinates_and_masked_segments():
    # tests/test_position.py:212-226
    ccpe.validate_contextual_path(f32([[[2.25, 0.5]]]), np.array([2]), np.array([0, 2]))
    with pytest.raises(ccpe.PathError) as err:
        ccpe.validate_contextual_path(f32([[[2.75, 0.5]]]), np.array([2]), np.array([0, 2]))
    assert err.value.kind == "gap"
    ccpe.validate_contextual_path(
        f32([[[1, 99, 0.5]]]), np.array([2]), np.arange(3),
        attention_mask=np.array([[True, False, True]]),
    )


def test_validation_tolerates_binade_roundoff():
    # tests/test_position.py:229-237
    logits = f32([100.0] * 128 + [-11.5])[None, None]
    p = ccpe.contextual_positions(logits, np.ones_like(logits, bool), 256)
    assert (p[..., :-1] - p[..., 1:]).max() > 1 + 1e-6
    ccpe.validate_contextual_path(p, np.array([128]), np.arange(129))


def test_validation_negative_position():
    with pytest.raises(ccpe.PathError) as err:
        ccpe.validate_contextual_path(f32([[[0.5, -0.01]]]), np.array([1]), np.arange(2))
    assert err.value.kind == "nonnegative"


def test_canonical_policy_strict_and_mixed_known_answers():
    # tests/test_attention_policies.py:63-92: fixed (0, 4); canonical from a 3-token
    # trace projected to fixed (0, 2): [[1.5? ...]] gives hybrid [1.5, 2, 1.5, 1, .5]
    q3 = np.ones((3, 2, 1))
    k3 = np.zeros((3, 1, 1))
    allowed = ccpe.allowed_mask(np.arange(3), np.arange(3), 2)
    trace = ccpe.contextual_positions(ccpe.logits(q3, k3), allowed, 16)
    canonical = trace[:, [0, 2]][:, :, [0, 2]]  # projected fixed x fixed
    contextual = ccpe.contextual_positions(
        ccpe.logits(np.ones((1, 2, 1)), np.zeros((5, 1, 1))),
        ccpe.allowed_mask(np.array([4]), np.arange(5), 2), 16,
    )
    with pytest.raises(ccpe.PathError) as err:
        ccpe.canonical_policy(contextual, np.array([4]), np.arange(5), (0, 4), canonical, [0, 1], True)
    assert err.value.kind == "nonincreasing"
    mixed = ccpe.canonical_policy(contextual, np.array([4]), np.arange(5), (0, 4), canonical, [0, 1], False)
    np.testing.assert_array_equal(mixed, np.broadcast_to([[1.5, 2, 1.5, 1, 0.5]], (2, 1, 5)))


# ---------------------------------------------------------------- WCA
def make_state(**kw):
    # tests/test_wca.py:14-20
    cached = np.ones((6, 1, 2))
    fresh = np.broadcast_to(np.array([5, 4, 3, 2, 1, 100.0])[:, None, None], cached.shape).copy()
    reused = np.array([True] * 5 + [False])
    return wca.State(cached, fresh, reused, ~reused, **kw), cached


def test_wca_budget_selection_and_active():
    # tests/test_wca.py:23-32
    state, _ = make_state()
    assert state.budget == 2
    assert np.flatnonzero(state.selected).tolist() == [0, 1]
    assert state.active.tolist() == [0, 1, 5]
    assert state.candidate.tolist() == [True, True, True, True, False, False]


def test_wca_deviation_and_ties():
    # tests/test_wca.py:35-43
    cached = np.ones((7, 2, 3))
    mask = np.ones(7, bool)
    s = wca.State(cached, cached + 1, mask, ~mask)
    assert np.flatnonzero(s.selected).tolist() == [0, 1]
    assert wca.squared_deviation(cached, cached + 1).tolist() == [6.0] * 7
    empty = wca.State(cached, cached, mask, ~mask)
    assert empty.budget == 0 and empty.active.size == 0


def test_wca_weight_known_answers():
    # tests/test_wca.py:46-60
    cached = np.zeros((1, 1, 2))
    assert wca.adaptation_weight(cached, np.ones_like(cached), epsilon=0.5).item() == 4
    assert wca.adaptation_weight(cached, np.ones_like(cached), epsilon=0.5, clamp=True).item() == 1
    assert wca.adaptation_weight(cached, cached).item() == 0
    huge = np.full((1, 1, 2), 1e30)
    assert wca.adaptation_weight(huge, 2 * huge).item() == pytest.approx(1.0)
    with pytest.raises(wca.NumericalError, match="overflow"):
        wca.adaptation_weight(np.zeros((1, 1, 1)), np.full((1, 1, 1), 1e308))


@pytest.mark.parametrize("mode, expected", [("previous_layer", 4), ("same_layer", 1)])
def test_wca_weight_order_known_answers(mode, expected):
    # tests/test_wca.py:63-85
    cached = np.ones((2, 1, 1))
    reused = np.array([True, False])
    s = wca.State(cached, np.array([3.0, 9.0])[:, None, None], reused, ~reused,
                  fraction=1, epsilon=1e-20, weight_update=mode)
    idx, fk, fv, used, *_ = s.update(2, cached, cached * 2, np.array([2.0, 7.0])[:, None, None],
                                     np.array([4.0, 8.0])[:, None, None])
    assert used.tolist() == pytest.approx([expected, 1])
    assert fk[:, 0, 0].tolist() == pytest.approx([1 + expected, 7])
    assert fv[:, 0, 0].tolist() == pytest.approx([2 + 2 * expected, 8])
    assert s.alpha[0] == pytest.approx(1)


def test_wca_gate_promotion_known_answers():
    # tests/test_wca.py:88-101
    s, cached = make_state(gate_interval=2)
    rows = s.active
    _, _, _, _, removed, promoted, nxt = s.update(2, cached, cached, -cached[rows], cached[rows])
    assert removed.tolist() == [0, 1] and promoted.tolist() == [2, 3] and nxt.tolist() == [2, 3, 5]
    rows = s.active
    s.update(3, cached, cached, -cached[rows], cached[rows])
    _, _, _, _, removed, promoted, nxt = s.update(4, cached, cached, -cached[rows], cached[rows])
    assert removed.tolist() == [2, 3] and promoted.size == 0 and nxt.tolist() == [5]


def test_wca_cosine_zero_heads():
    # tests/test_wca.py:117-120
    a = np.array([[[1.0, 0], [0, 1]], [[0, 0], [0, 0]]])
    b = np.array([[[1.0, 0], [0, -1]], [[1, 1], [1, 1]]])
    assert wca.mean_head_cosine(a, b).tolist() == [0, 0]


def test_wca_exact_sum_differs_from_naive_float_sum():
    # the oracle's fsum is exact: a naive float64 sum of these squares is not
    vals = np.array([1e16, 1.0, -1e16, 1.0])
    cached = np.zeros((1, 1, 4))
    fresh = np.sqrt(np.abs(vals))[None, None, :] * 0 + np.array([1e8, 1.0, 1e8, 1.0])[None, None]
    err = wca.squared_deviation(cached, fresh)
    assert err[0] == math.fsum([1e16, 1.0, 1e16, 1.0])


def test_wca_blend_rounds_like_separate_operations():
    w = np.array([0.1])
    fresh = np.full((1, 1, 1), 3.3)
    old = np.full((1, 1, 1), 1.7)
    expected = 0.1 * 3.3 + (1 - 0.1) * 1.7  # python floats: each op rounded
    assert wca.blend(w, fresh, old, "float64")[0, 0, 0] == expected


# ---------------------------------------------------------------- SLIDE
def test_scatter_gather_identity_and_fixture_slots():
    # tests/test_paged.py:13-23, 245-247: table [4, 1, 6, 3], bs 2 -> canonical slots
    table, bs = [4, 1, 6, 3], 2
    slots = [table[t // bs] * bs + t % bs for t in range(5)]
    assert slots == [8, 9, 2, 3, 12]
    rng = np.random.default_rng(0)
    cache = np.zeros((8, 2, 2, 6), np.uint16)
    side_k = np.zeros((2, 2, 3), np.uint16)
    side_v = np.zeros_like(side_k)
    key = rng.integers(0, 2**16, (5, 2, 3), dtype=np.uint16)
    value = rng.integers(0, 2**16, (5, 2, 3), dtype=np.uint16)
    slots2 = slots[:3] + [16, 17]  # two sidecar rows (native total = 16)
    slide.slot_scatter(cache, side_k, side_v, slots2, key, value)
    k2, v2 = slide.slot_gather(cache, side_k, side_v, slots2)
    np.testing.assert_array_equal(k2, key)
    np.testing.assert_array_equal(v2, value)
    assert (cache[0] == 0).all()


def test_fresh_slot_order_and_free_list_agree():
    # tests/test_slide.py:18-36: unused returned slots come first, lowest first
    assert slide.fresh_slot_sequence({5, 2}, 7, 4) == [2, 5, 7, 8]
    free = np.zeros(12, bool)
    free[[2, 5]] = True
    free[7:] = True
    assert slide.acquire_lowest(free, 4).tolist() == [2, 5, 7, 8]
    assert slide.acquire_lowest(free, 10) is None


def test_page_and_slot_copy():
    rng = np.random.default_rng(1)
    cache = rng.integers(0, 2**16, (2, 6, 2, 4, 8), dtype=np.uint16)
    ref = cache.copy()
    slide.page_copy(cache, [0, 3], [5, 1])
    np.testing.assert_array_equal(cache[:, 5], ref[:, 0])
    np.testing.assert_array_equal(cache[:, 1], ref[:, 3])
    cache2 = ref.copy()
    slide.slot_copy(cache2, [0, 9], [21, 2])
    np.testing.assert_array_equal(cache2[:, 5, :, 1], ref[:, 0, :, 0])
    np.testing.assert_array_equal(cache2[:, 0, :, 2], ref[:, 2, :, 1])


# ------------------------------------------------------------ runtime rows
def _brute_next_rows(hidden, residual, previous, active, fixed, snap_h, snap_r):
    """Row by row from the definition: a continuing token keeps its previous
    row, a newly active fixed token takes its snapshot row, anything else is
    lost (runtime.py:408-432)."""
    prev, fix = list(previous), list(fixed)
    out_h, out_r, restored = [], [], 0
    for t in active:
        if t in prev:
            out_h.append(hidden[prev.index(t)])
            out_r.append(residual[prev.index(t)])
        elif t in fix:
            out_h.append(snap_h[fix.index(t)])
            out_r.append(snap_r[fix.index(t)])
            restored += 1
        else:
            raise rows.RowLost
    return np.array(out_h), np.array(out_r), restored


def test_next_layer_rows_against_the_definition():
    rng = np.random.default_rng(5)
    n, h = 40, 6
    for trial in range(20):
        fixed = np.sort(rng.choice(n, 25, replace=False))
        mandatory = np.setdiff1d(np.arange(n), fixed)[:3]
        previous = np.sort(np.concatenate([rng.choice(fixed, 8, replace=False), mandatory]))
        active = np.sort(np.concatenate([rng.choice(fixed, 6, replace=False), mandatory]))
        # every row carries its token and its source, so any mix-up shows
        hidden = previous[:, None] * 10.0 + np.arange(h) / 10
        residual = -hidden
        snap_h = fixed[:, None] * 10.0 + 1000 + np.arange(h) / 10
        snap_r = -snap_h
        got = rows.next_layer_rows(hidden, residual, previous, active, fixed, snap_h, snap_r, n)
        want = _brute_next_rows(hidden, residual, previous, active, fixed, snap_h, snap_r)
        np.testing.assert_array_equal(got[0], want[0])
        np.testing.assert_array_equal(got[1], want[1])
        assert got[2] == want[2]
    # unordered lists give the same rows (the lookup tables need no order)
    perm = rng.permutation(len(previous))
    a = rows.next_layer_rows(hidden, residual, previous, active, fixed, snap_h, snap_r, n)
    b = rows.next_layer_rows(hidden[perm], residual[perm], previous[perm], active, fixed, snap_h, snap_r, n)
    np.testing.assert_array_equal(a[0], b[0])
    # a dynamic (non-fixed) token that was dropped is lost
    keep = previous != mandatory[0]
    with pytest.raises(rows.RowLost):
        rows.next_layer_rows(hidden[keep], residual[keep], previous[keep], active, fixed, snap_h, snap_r, n)


def test_scatter_and_gather_rows():
    x = np.arange(12.0).reshape(4, 3)
    out = rows.scatter_rows(x, [1, 4, 5, 9], 10)
    assert out.shape == (10, 3)
    np.testing.assert_array_equal(out[[1, 4, 5, 9]], x)
    assert not out[[0, 2, 3, 6, 7, 8]].any()
    np.testing.assert_array_equal(rows.gather_rows(out, [9, 1]), x[[3, 0]])
