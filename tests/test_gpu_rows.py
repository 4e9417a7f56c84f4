"""Selective-prefill row bookkeeping on the MI355X vs the oracle (runtime.py:408-456).

Rows move bit for bit, so every comparison is on raw bits; widths and strides
cover every copy width the kernels choose (16, 8, 4, 2 and 1 bytes).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cacheslide_amd.runtime_rows import ReuseFailure, gather_rows, next_layer_rows, scatter_rows
from oracle import rows as orc

pytestmark = pytest.mark.gpu

_BITS = {torch.bfloat16: torch.int16, torch.float16: torch.int16, torch.float32: torch.int32,
         torch.float64: torch.int64, torch.uint8: torch.uint8}


def bits(x: torch.Tensor) -> np.ndarray:
    return x.detach().contiguous().view(_BITS[x.dtype]).cpu().numpy()


def random_rows(rows, width, dtype, gen):
    if dtype == torch.uint8:
        return torch.randint(0, 256, (rows, width), generator=gen, dtype=torch.uint8)
    return torch.randn(rows, width, generator=gen, dtype=torch.float64).to(dtype)


def case(seed, n=300, n_fixed=200, keep=60, add=40, mandatory=8):
    rng = np.random.default_rng(seed)
    fixed = np.sort(rng.choice(n, n_fixed, replace=False))
    dynamic = np.setdiff1d(np.arange(n), fixed)[:mandatory]
    previous = np.sort(np.concatenate([rng.choice(fixed, keep, replace=False), dynamic]))
    active = np.sort(np.concatenate([rng.choice(fixed, add, replace=False), dynamic]))
    return fixed, previous, active


@pytest.mark.parametrize("dtype, width", [
    (torch.bfloat16, 4096), (torch.bfloat16, 7), (torch.float16, 130), (torch.float32, 33),
    (torch.float64, 5), (torch.uint8, 9), (torch.bfloat16, 1),
])
def test_next_layer_rows_bit_exact(device, dtype, width):
    fixed, previous, active = case(width)
    gen = torch.Generator().manual_seed(width)
    hidden = random_rows(len(previous), width, dtype, gen)
    residual = random_rows(len(previous), width, dtype, gen)
    snap_h = random_rows(len(fixed), width, dtype, gen)
    snap_r = random_rows(len(fixed), width, dtype, gen)
    want = orc.next_layer_rows(bits(hidden), bits(residual), previous, active, fixed,
                               bits(snap_h), bits(snap_r), 300)
    got = next_layer_rows(hidden.to(device), residual.to(device), torch.from_numpy(previous),
                          torch.from_numpy(active), torch.from_numpy(fixed),
                          {"hidden": snap_h.to(device), "residual": snap_r.to(device)})
    np.testing.assert_array_equal(bits(got.hidden), want[0])
    np.testing.assert_array_equal(bits(got.residual), want[1])
    assert int(got.restored.item()) == want[2] > 0


def test_strided_rows_and_no_residual(device):
    fixed, previous, active = case(11)
    gen = torch.Generator().manual_seed(11)
    wide = random_rows(len(previous), 80, torch.bfloat16, gen)
    snap = random_rows(len(fixed), 80, torch.bfloat16, gen)
    hidden = wide.to(device)[:, 8:72]          # row stride 80, width 64, 16-byte aligned
    snap_h = snap.to(device)[:, 3:67]          # 6-byte offset: narrower copies
    want = orc.next_layer_rows(bits(hidden), None, previous, active, fixed, bits(snap_h), None, 300)
    got = next_layer_rows(hidden, None, torch.from_numpy(previous), torch.from_numpy(active),
                          torch.from_numpy(fixed), {"hidden": snap_h})
    assert got.residual is None
    np.testing.assert_array_equal(bits(got.hidden), want[0])


def test_snapshot_is_read_only_when_rows_are_restored(device):
    fixed, previous, active = case(3)
    hidden = torch.randn(len(previous), 16, device=device)
    residual = torch.randn_like(hidden)
    reads = []

    def read():
        reads.append(1)
        return {"hidden": torch.randn(len(fixed), 16, device=device),
                "residual": torch.randn(len(fixed), 16, device=device)}

    # the same tokens again: everything continues, no snapshot read
    same = next_layer_rows(hidden, residual, torch.from_numpy(previous), torch.from_numpy(previous),
                           torch.from_numpy(fixed), read_snapshot=read)
    assert reads == [] and int(same.restored.item()) == 0
    assert torch.equal(same.hidden, hidden) and torch.equal(same.residual, residual)
    got = next_layer_rows(hidden, residual, torch.from_numpy(previous), torch.from_numpy(active),
                          torch.from_numpy(fixed), read_snapshot=read)
    assert reads == [1] and int(got.restored.item()) == len(np.setdiff1d(active, previous))


def test_lost_rows_and_bad_lists(device):
    fixed, previous, active = case(5)
    hidden = torch.randn(len(previous), 8, device=device)
    snap = {"hidden": torch.randn(len(fixed), 8, device=device),
            "residual": torch.randn(len(fixed), 8, device=device)}
    dynamic = np.setdiff1d(previous, fixed)
    keep = previous != dynamic[0]
    with pytest.raises(ReuseFailure, match="a mandatory dynamic row was lost"):
        next_layer_rows(hidden[torch.from_numpy(keep).to(device)], None, torch.from_numpy(previous[keep]),
                        torch.from_numpy(active), torch.from_numpy(fixed), snap)
    deferred = next_layer_rows(hidden[torch.from_numpy(keep).to(device)], None,
                               torch.from_numpy(previous[keep]), torch.from_numpy(active),
                               torch.from_numpy(fixed), snap, check=False)
    with pytest.raises(ReuseFailure):
        deferred.check()
    with pytest.raises(ValueError, match="ascending and distinct"):
        next_layer_rows(hidden, None, torch.from_numpy(previous[::-1].copy()), torch.from_numpy(active),
                        torch.from_numpy(fixed), snap)
    with pytest.raises(ValueError, match="HIP device only"):
        next_layer_rows(hidden.cpu(), None, torch.from_numpy(previous), torch.from_numpy(active),
                        torch.from_numpy(fixed), snap)


@pytest.mark.parametrize("dtype, width", [(torch.bfloat16, 4096), (torch.float32, 3), (torch.float16, 5)])
def test_scatter_and_gather_rows(device, dtype, width):
    gen = torch.Generator().manual_seed(width)
    tokens = np.sort(np.random.default_rng(width).choice(500, 123, replace=False))
    rows = random_rows(len(tokens), width, dtype, gen)
    out = scatter_rows(rows.to(device), torch.from_numpy(tokens), 500)
    np.testing.assert_array_equal(bits(out), orc.scatter_rows(bits(rows), tokens, 500))
    idx = np.random.default_rng(1).permutation(500)[:77]
    np.testing.assert_array_equal(bits(gather_rows(out, torch.from_numpy(idx))), orc.gather_rows(bits(out), idx))
    with pytest.raises(ValueError, match="outside the source rows"):
        gather_rows(out, torch.tensor([0, 500]))
    with pytest.raises(ValueError, match="outside the source rows"):
        scatter_rows(rows.to(device), torch.from_numpy(tokens), int(tokens[-1]))
    with pytest.raises(ValueError, match="ascending and distinct"):
        scatter_rows(rows.to(device), torch.from_numpy(tokens[::-1].copy()), 500)


def test_layer_chain_at_bench_size(device):
    """Four layers of a 16384-token prompt, hidden 4096 bf16, 90% fixed tokens:
    each layer's active set is the dynamic tokens plus a fresh 15% draw of the
    fixed ones, so every layer both keeps and restores rows."""
    n, width = 16384, 4096
    rng = np.random.default_rng(16384)
    fixed = np.sort(rng.choice(n, n * 9 // 10, replace=False))
    dynamic = np.setdiff1d(np.arange(n), fixed)
    gen = torch.Generator().manual_seed(16384)
    snap_h = random_rows(len(fixed), width, torch.bfloat16, gen)
    snap_r = random_rows(len(fixed), width, torch.bfloat16, gen)
    snap = {"hidden": snap_h.to(device), "residual": snap_r.to(device)}
    previous = np.sort(np.concatenate([dynamic, rng.choice(fixed, len(fixed) * 15 // 100, replace=False)]))
    hidden_bits = bits(random_rows(len(previous), width, torch.bfloat16, gen))
    residual_bits = bits(random_rows(len(previous), width, torch.bfloat16, gen))
    hidden = torch.from_numpy(hidden_bits).view(torch.bfloat16).to(device)
    residual = torch.from_numpy(residual_bits).view(torch.bfloat16).to(device)
    for layer in range(4):
        active = np.sort(np.concatenate([dynamic, rng.choice(fixed, len(fixed) * 15 // 100, replace=False)]))
        want_h, want_r, want_n = orc.next_layer_rows(hidden_bits, residual_bits, previous, active, fixed,
                                                     bits(snap_h), bits(snap_r), n)
        got = next_layer_rows(hidden, residual, torch.from_numpy(previous), torch.from_numpy(active),
                              torch.from_numpy(fixed), snap)
        np.testing.assert_array_equal(bits(got.hidden), want_h, err_msg=f"layer {layer}")
        np.testing.assert_array_equal(bits(got.residual), want_r, err_msg=f"layer {layer}")
        assert int(got.restored.item()) == want_n > 0
        previous, hidden, residual, hidden_bits, residual_bits = active, got.hidden, got.residual, want_h, want_r
    full = scatter_rows(hidden, torch.from_numpy(previous), n)
    np.testing.assert_array_equal(bits(full), orc.scatter_rows(hidden_bits, previous, n))
    # gather(scatter(rows)) is the rows again
    np.testing.assert_array_equal(bits(gather_rows(full, torch.from_numpy(previous))), hidden_bits)


def test_empty_active_list(device):
    fixed, previous, _ = case(2)
    hidden = torch.randn(len(previous), 8, device=device)
    empty = torch.zeros(0, dtype=torch.long)
    got = next_layer_rows(hidden, hidden.clone(), torch.from_numpy(previous), empty, torch.from_numpy(fixed),
                          {"hidden": torch.randn(len(fixed), 8, device=device),
                           "residual": torch.randn(len(fixed), 8, device=device)})
    assert got.hidden.shape == (0, 8) and got.residual.shape == (0, 8) and int(got.restored.item()) == 0
    assert scatter_rows(got.hidden, empty, 300).abs().sum().item() == 0
    assert gather_rows(got.hidden, empty).shape == (0, 8)
    # every active token restored from the snapshot: no previous rows at all
    fixed_t = torch.from_numpy(fixed)
    snap = {"hidden": torch.randn(len(fixed), 8, device=device)}
    only = next_layer_rows(snap["hidden"][:3], None, fixed_t[:3], fixed_t[:5], fixed_t, snap)
    assert torch.equal(only.hidden, snap["hidden"][:5]) and int(only.restored.item()) == 2
