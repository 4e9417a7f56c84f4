"""CCPEProfile.calibrate on the device: the reference's own known answers for
the joint-histogram decision (tests/test_position.py:360-486), carried over
through ``cacheslide_amd`` with the traces built by the device's
``CoPE.position_trace``, plus a modal pattern whose first sample is not the
first trace.
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch

from cacheslide_amd import CCPEProfile, ChunkIdentity, CoPE

pytestmark = pytest.mark.gpu


def make_trace(device, value=0.0):
    # tests/test_position.py:360-365
    cope = CoPE(1, 8, device=device)
    q = torch.ones(3, 1, 1, device=device)
    k = torch.full((3, 1, 1), float(value), device=device)
    return cope.position_trace(q, k, torch.arange(3, device=device), checkpoint_id="trained-cope-v1")


def test_profile_joint_histogram_keeps_observed_trace_and_strict_identity(device):
    # tests/test_position.py:368-408
    traces = [make_trace(device, 0), make_trace(device, 0.7), make_trace(device, 0.7)]
    chunks = [ChunkIdentity("system", "a" * 64, 1), ChunkIdentity("context", "b" * 64, 2)]
    profile = CCPEProfile.calibrate(traces, chunks, trained_profile_version="task-v1")
    torch.testing.assert_close(profile.canonical_positions, traces[1].positions)
    selected = profile.lookup(chunks, torch.tensor([2, 0]), checkpoint_id="trained-cope-v1",
                              trained_profile_version="task-v1")
    torch.testing.assert_close(selected.cpu(), traces[1].positions[:, [2, 0]])
    with pytest.raises(ValueError, match="identities"):
        profile.lookup(chunks[::-1], torch.tensor([0]), checkpoint_id="trained-cope-v1",
                       trained_profile_version="task-v1")
    assert profile.lookup(chunks, torch.tensor([3]), checkpoint_id="trained-cope-v1",
                          trained_profile_version="task-v1", strict=False) is None
    with pytest.raises(ValueError, match="version"):
        profile.lookup(chunks, torch.tensor([0]), checkpoint_id="untrained", trained_profile_version="task-v1")


def test_profile_rejects_fabricated_positions_and_oversized_trace(device):
    # tests/test_position.py:429-451
    trace = make_trace(device)
    chunks = [ChunkIdentity("fixed", "c" * 64, 3)]
    with pytest.raises(ValueError, match="CoPE gates"):
        CCPEProfile.calibrate([replace(trace, positions=trace.positions + 1)], chunks,
                              trained_profile_version="v1")
    with pytest.raises(ValueError, match="max_elements"):
        CCPEProfile.calibrate([trace], chunks, trained_profile_version="v1", max_elements=2)
    with pytest.raises(ValueError, match="genuine"):
        CCPEProfile.calibrate([torch.arange(3)], chunks, trained_profile_version="v1")
    with pytest.raises(ValueError, match="max_elements"):
        CoPE(1, 4, device=device).position_trace(torch.ones(3, 1, 1, device=device),
                                                 torch.ones(3, 1, 1, device=device),
                                                 torch.arange(3, device=device), checkpoint_id="trained",
                                                 max_elements=5)


def test_joint_histogram_tie_is_order_independent_and_uses_real_pattern(device):
    # tests/test_position.py:454-486
    cope = CoPE(1, 8, device=device)
    q = torch.ones(3, 1, 1, device=device)
    traces = [
        cope.position_trace(q, torch.tensor(values, device=device)[:, None, None],
                            torch.arange(3, device=device), checkpoint_id="trained")
        for values in ([0.0, 0.0, 3.0], [0.0, 3.0, 0.0], [3.0, 0.0, 0.0])
    ]
    chunks = [ChunkIdentity("fixed", "d" * 64, 3)]
    first = CCPEProfile.calibrate(traces, chunks, trained_profile_version="v1")
    reversed_samples = CCPEProfile.calibrate(traces[::-1], chunks, trained_profile_version="v1")
    torch.testing.assert_close(first.canonical_positions, reversed_samples.canonical_positions)
    assert any(torch.equal(first.canonical_positions, trace.positions) for trace in traces)
    independent_modes = torch.stack([trace.positions for trace in traces]).mode(0).values
    assert not any(torch.equal(independent_modes, trace.positions) for trace in traces)


def test_modal_pattern_is_not_the_first_trace(device):
    # the first trace is alone in its bin; the modal pattern's first sample is
    # traces[1] (traces[2] shares its bin at width 0.25 but not its values)
    traces = [make_trace(device, 2.0), make_trace(device, -1.0), make_trace(device, -1.01)]
    assert not torch.equal(traces[1].positions, traces[2].positions)
    chunks = [ChunkIdentity("fixed", "e" * 64, 3)]
    profile = CCPEProfile.calibrate(traces, chunks, trained_profile_version="v1")
    assert torch.equal(profile.canonical_positions, traces[1].positions)
