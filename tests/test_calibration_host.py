"""The calibration decision of CCPEProfile.calibrate (position.py:676-688), on
the host: each sample's positions are quantised to the histogram bin width as
one joint pattern, and the first sample of the most frequent pattern wins,
ties going to the lexicographically smallest pattern.

The quantisation is pinned to torch (the reference's arithmetic dependency,
``(positions / width).round().long()`` on the positions tensor): the quotient
is rounded to the positions' dtype before the bin is taken, which at width
0.1 differs from a float64 division on about a third of the half-bin values.
Each decision test is chosen so that a plausible wrong rule fails it: taking
the first sample, taking per-cell modes, or dividing in float64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd.position import _modal_sample, _quantise


def torch_bins(sample: torch.Tensor, width: float) -> tuple[int, ...]:
    return tuple((sample / width).round().long().flatten().tolist())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("width", [0.1, 0.25, 0.3, 0.7])
def test_quantise_matches_torch_at_half_bins(dtype, width):
    # half-bin values, their neighbours one ulp away and random positions
    half = (torch.arange(630, dtype=torch.float64) + 0.5) * width
    gen = torch.Generator().manual_seed(11)
    values = torch.cat([half, torch.nextafter(half, half + 1), torch.nextafter(half, half - 1),
                        torch.rand(500, generator=gen, dtype=torch.float64) * 63]).to(dtype)
    assert _quantise(values, width) == torch_bins(values, width)


def test_quantise_is_not_a_float64_division():
    # the fp32 quotient and the fp64 quotient of fp32 half-bin values round
    # differently on many of them: the pattern must follow the fp32 one
    values = ((torch.arange(630, dtype=torch.float64) + 0.5) * 0.1).float()
    fp64 = tuple(int(np.rint(v / 0.1)) for v in values.double().tolist())
    mine = _quantise(values, 0.1)
    assert mine == torch_bins(values, 0.1)
    assert sum(a != b for a, b in zip(mine, fp64)) > 100


def test_quantise_keeps_shape_order():
    s = torch.tensor([[[0.0, 1.0], [2.0, 3.0]]])
    assert _quantise(s, 1.0) == (0, 1, 2, 3)


def test_first_sample_is_not_taken_when_another_pattern_is_modal():
    a = torch.tensor([[[0.5, 0.0], [1.5, 1.0]]])
    b = torch.tensor([[[1.0, 0.0], [2.0, 1.0]]])
    samples = [a, b, b.clone()]
    assert _modal_sample(samples, 0.25) is samples[1]


def test_modal_pattern_returns_its_first_real_sample():
    # two samples in one bin (not bit-identical) and one elsewhere: the first of
    # the two is returned as it is, not the later one or a mean of them
    a1 = torch.tensor([[[1.00, 0.5]]])
    other = torch.tensor([[[2.00, 0.5]]])
    a2 = torch.tensor([[[1.05, 0.5]]])
    samples = [a1, other, a2]
    out = _modal_sample(samples, 0.25)
    assert out is a1 and not torch.equal(out, a2)


def test_tie_is_order_independent_and_a_real_pattern():
    # three patterns once each; per-cell modes would give [0, 0, 0], which no
    # sample has; the lexicographically smallest pattern (0, 0, 1) wins
    samples = [torch.tensor([[[1.0, 0.0, 0.0]]]), torch.tensor([[[0.0, 1.0, 0.0]]]),
               torch.tensor([[[0.0, 0.0, 1.0]]])]
    forward = _modal_sample(samples, 0.25)
    backward = _modal_sample(samples[::-1], 0.25)
    assert torch.equal(forward, backward) and torch.equal(forward, samples[2])
    cell_modes = torch.stack(samples).mode(0).values
    assert not any(torch.equal(cell_modes, s) for s in samples)


def test_more_frequent_pattern_beats_a_smaller_one():
    small = torch.tensor([[[0.0]]])
    big = torch.tensor([[[5.0]]])
    assert torch.equal(_modal_sample([small, big, big.clone()], 1.0), big)
    assert torch.equal(_modal_sample([big, small, small.clone(), big.clone()], 1.0), small)
