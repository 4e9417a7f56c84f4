"""Pins of the oracle's numeric conventions against torch and closed forms.

The reference computes these steps with torch on the CPU
(src/cacheslide_vllm/position.py:295-307, wca.py:55-112, and every
``.to(dtype)``); the oracle restates them in numpy.  Each test below is
chosen so that a plausible restatement mistake fails it: a sum taken for a
mean, a dropped amax scaling or clamp, a float32 cumulative sum, a single
rounding where torch rounds twice, a naive reduction where the oracle sums
exactly.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ccpe, wca


# ------------------------------------------------------------ mean_head_cosine
def test_mean_over_heads_with_different_cosines():
    # head 0 parallel (cos 1), head 1 orthogonal (cos 0): the mean is 0.5,
    # a sum over heads would give 1
    a = np.array([[[1.0, 0.0], [1.0, 0.0]]])
    b = np.array([[[2.0, 0.0], [0.0, 3.0]]])
    assert wca.mean_head_cosine(a, b).tolist() == [0.5]
    # cosines 1, -1 and 1/2 (60 degrees): mean 1/6
    a = np.array([[[1.0, 0.0], [1.0, 0.0], [1.0, 0.0]]])
    b = np.array([[[5.0, 0.0], [-2.0, 0.0], [1.0, math.sqrt(3.0)]]])
    np.testing.assert_allclose(wca.mean_head_cosine(a, b), [1 / 6], rtol=0, atol=1e-15)


def test_amax_scaling_keeps_extreme_magnitudes_exact():
    # squares of 1e-200 underflow and of 1e200 overflow in float64: without
    # the per-head amax scaling the cosine of parallel rows would be lost
    a = np.array([[[3e-200, 4e-200], [1.0, 0.0]]])
    b = np.array([[[6e200, 8e200], [0.0, 1e-300]]])
    out = wca.mean_head_cosine(a, b)
    np.testing.assert_allclose(out, [0.5], rtol=0, atol=1e-15)


def test_cosine_is_clamped_to_one():
    # rows whose unclamped dot of unit vectors rounds above 1
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4000, 1, 7))
    scaled = x / np.abs(x).max(-1, keepdims=True)
    unit = scaled / np.sqrt((scaled * scaled).sum(-1, keepdims=True))
    raw = (unit * unit).sum(-1)[:, 0]
    over = raw > 1.0
    assert over.any()
    out = wca.mean_head_cosine(x, x)
    assert (out[over] == 1.0).all() and (out <= 1.0).all()


def test_cosine_matches_torch_on_random_heads():
    # library routine: torch's cosine_similarity of float64 rows, mean over heads
    rng = np.random.default_rng(8)
    a = rng.standard_normal((300, 8, 128))
    b = a + 0.3 * rng.standard_normal((300, 8, 128))
    ref = torch.nn.functional.cosine_similarity(torch.from_numpy(a), torch.from_numpy(b), dim=-1).mean(-1)
    np.testing.assert_allclose(wca.mean_head_cosine(a, b), ref.numpy(), rtol=0, atol=1e-14)


# ------------------------------------------------------------ positions vs torch
def test_reverse_cumsum_equals_torch_cpu_bit_for_bit():
    # torch's CPU cumsum of float32 (position.py:305-307: flip, cumsum, flip);
    # long rows of small gates where a float32 running sum would drift
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((4, 16, 6000)).astype(np.float32) * 3 - 4
    allowed = rng.random((4, 16, 6000)) > 0.05
    gates = torch.where(torch.from_numpy(allowed), torch.sigmoid(torch.from_numpy(logits)), torch.tensor(0.0))
    torch_suffix = torch.flip(torch.cumsum(torch.flip(gates, [-1]), -1), [-1])
    oracle_suffix = np.flip(np.cumsum(np.flip(gates.numpy().astype(np.float64), -1), -1), -1).astype(np.float32)
    np.testing.assert_array_equal(oracle_suffix, torch_suffix.numpy())
    naive = np.flip(np.cumsum(np.flip(gates.numpy(), -1), -1, dtype=np.float32), -1)
    assert not np.array_equal(naive, torch_suffix.numpy())   # a float32 scan is not what torch does


def test_contextual_positions_match_torch_pipeline():
    # the whole CoPE.contextual_positions step in torch (sigmoid -> flipped
    # cumsum -> clamp) against the oracle: the sigmoid may differ in the last
    # ulp between libraries, so positions agree to a few ulps of P
    rng = np.random.default_rng(10)
    logits = rng.standard_normal((2, 8, 3000)).astype(np.float32) * 2 - 3
    allowed = np.tril(np.ones((8, 3000), bool), k=2992)[None].repeat(2, 0)
    lt = torch.from_numpy(logits).masked_fill(~torch.from_numpy(allowed), float("-inf"))
    ref = torch.flip(torch.cumsum(torch.flip(torch.sigmoid(lt), [-1]), -1), [-1]).clamp(0, 63)
    out = ccpe.contextual_positions(logits, allowed, 64)
    np.testing.assert_allclose(out, ref.numpy(), rtol=0, atol=64 * 4 * np.finfo(np.float32).eps)


def test_sigmoid_within_four_ulps_of_torch():
    # the oracle's float32 1 / (1 + exp(-x)) against torch.sigmoid on the CPU:
    # the two exp implementations differ by up to 4 ulps (measured maximum;
    # only for negative x), far inside the attention tolerance
    x = np.linspace(-30, 30, 200001, dtype=np.float32)
    ours = ccpe.sigmoid(x)
    ref = torch.sigmoid(torch.from_numpy(x)).numpy()
    ulp = np.spacing(np.maximum(np.abs(ref), np.float32(1e-38)))
    assert (np.abs(ours - ref) <= 4 * ulp).all()
    assert (ours[x > 10] == ref[x > 10]).all()


# ------------------------------------------------------------ roundings vs torch
def _f32(bits: list[int]) -> np.ndarray:
    return np.array(bits, dtype=np.uint32).view(np.float32)


def test_bf16_round_equals_torch_on_ties_subnormals_and_overflow():
    special = _f32([
        0x3F808000, 0x3F818000,          # exact ties: round to even (down, up)
        0x3F808001, 0x3F807FFF,          # just above / below a tie
        0x00000001, 0x00008000, 0x00018000, 0x807F8000,   # subnormals and ties among them
        0x7F7F8000, 0x7F7FFFFF, 0xFF7F8000,   # ties and values that round to infinity
        0x7F800000, 0xFF800000, 0x7FC00000,   # inf, -inf, nan
        0x80000000, 0x00000000,
    ])
    rng = np.random.default_rng(11)
    rand = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([special, rand])
    ours = ccpe.bf16_round(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy()
    nan = np.isnan(ref)
    assert (np.isnan(ours) == nan).all()
    np.testing.assert_array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype, tdtype", [("bfloat16", torch.bfloat16), ("float16", torch.float16),
                                           ("float32", torch.float32)])
def test_to_dtype_equals_torch_cpu_conversion(dtype, tdtype):
    # float64 -> 16-bit: torch rounds through float32 (two roundings).  Values
    # just above a 16-bit tie whose float32 rounding lands on the tie separate
    # the two conventions.
    rng = np.random.default_rng(12)
    base = rng.standard_normal(100000)
    f32 = base.astype(np.float32)
    if dtype == "bfloat16":
        tie = (f32.view(np.uint32) & np.uint32(0xFFFF0000)) | np.uint32(0x8000)
        half_ulp32 = np.spacing(tie.view(np.float32)).astype(np.float64) / 4
        near = tie.view(np.float32).astype(np.float64) + half_ulp32   # rounds to the tie in float32
    else:
        near = f32.astype(np.float64) * (1 + 2**-30)
    x = np.concatenate([base, near, [1e300, -1e300, 6.5e4, 65520.0, 5.9604644775390625e-08 * 0.75, 0.0, -0.0]])
    with np.errstate(over="ignore"):
        ours = wca.to_dtype(x, dtype)
    ref = torch.from_numpy(x.copy()).to(tdtype).double().numpy()
    np.testing.assert_array_equal(ours, ref)
    if dtype == "bfloat16":
        # above the bf16 midpoint, yet rounded toward zero: only a rounding
        # through float32 (onto the tie, then ties-to-even) does that
        r = ref[base.size:base.size + near.size]
        assert (np.abs(r) < np.abs(near)).any()


# ------------------------------------------------------------ WCA sums vs torch
def test_exact_deviation_sums_vs_torch_fp64_reduction():
    """The oracle's per-token sums are correctly rounded (math.fsum); the
    reference's ``(new - old).square().sum((1, 2))`` in float64 rounds along
    torch's reduction tree.  At the WCA workload shape (16384 tokens x 8 heads
    x 128, bf16 KV with N(0, 0.05) drift) the two differ by at most one ulp,
    on a few tokens, and the top-15% selection (stable descending order of the
    deviation, ties to the lower index) is identical."""
    T, H, D = 16384, 8, 128
    gen = torch.Generator().manual_seed(4000)
    fresh = torch.randn((T, H, D), generator=gen).to(torch.bfloat16)
    cached = (fresh.float() + torch.randn((T, H, D), generator=gen) * 0.05).to(torch.bfloat16)
    ref = (fresh.double() - cached.double()).square().sum((1, 2)).numpy()
    ours = wca.squared_deviation(cached.double().numpy(), fresh.double().numpy())
    ulps = np.abs(ours - ref) / np.spacing(ref)
    assert ulps.max() <= 1.0
    budget = math.ceil(0.15 * T)
    take_ref = np.argsort(-ref, kind="stable")[:budget]
    take_ours = np.argsort(-ours, kind="stable")[:budget]
    assert np.array_equal(np.sort(take_ref), np.sort(take_ours))
    norm_ref = cached.double().square().sum((1, 2)).numpy()
    alpha_ref = ref / (norm_ref + 1e-8)
    alpha = wca.adaptation_weight(cached.double().numpy(), fresh.double().numpy())
    assert (np.abs(alpha - alpha_ref) / np.spacing(alpha_ref)).max() <= 2.0
