"""cs_ccpe_decode_bf16_noalloc: the decode step with its workspace in a static
device array instead of a caller allocation.

Called through the C ABI and compared bit for bit with cs_ccpe_decode_bf16
(the same kernels over a caller workspace) on two calls in a row, the second
smaller, so the second call runs over the first call's leftover scratch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from cacheslide_amd import CoPE, _hip
from cacheslide_amd.ccpe import _paged_source, decode_workspace, decode_workspace_bytes
from tests._helpers import seeded

pytestmark = pytest.mark.gpu


def _case(device, lens, hq, hkv, seed, bs=16):
    per = [(n + bs - 1) // bs for n in lens]
    nb = sum(per) + 3
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))
    table = torch.full((len(lens), max(per)), -1, dtype=torch.int32)
    at = 0
    for b, pb in enumerate(per):
        table[b, :pb] = perm[at:at + pb].to(torch.int32)
        at += pb
    cache = seeded((nb, hkv, bs, 256), seed + 1, dtype=torch.bfloat16).to(device)
    q = seeded((len(lens), hq, 128), seed + 2, dtype=torch.bfloat16).to(device)
    cope = CoPE(128, 64, device=device)
    with torch.no_grad():
        cope.position_embeddings.copy_(seeded((128, 64), seed + 3, scale=0.02))
    return cache, table.to(device), q, cope


def _run(lib, name, device, cache, table, q, cope, lens, split, workspace=None):
    b, hq = q.shape[0], q.shape[1]
    hkv = cache.shape[1]
    nk = torch.tensor(lens, dtype=torch.int32, device=device)
    max_nk = max(lens)
    src = _paged_source(cache, table)
    out = torch.full((b, hq, 128), float("nan"), dtype=torch.bfloat16, device=device)
    flags = _hip.new_flags(device)
    e = cope.position_embeddings.detach()
    head = [_hip.ptr(q), q.stride(0), q.stride(1), b, hq, hkv, _hip.ptr(nk), max_nk, ctypes.byref(src),
            _hip.ptr(e), cope.max_positions, split]
    if workspace is None:
        status = getattr(lib, name)(*head, _hip.ptr(out), _hip.ptr(flags), _hip.stream_of(device))
    else:
        status = getattr(lib, name)(*head, _hip.ptr(workspace), workspace.numel(), _hip.ptr(out),
                                    _hip.ptr(flags), _hip.stream_of(device))
    _hip.check(status, name)
    torch.cuda.synchronize(device)
    assert _hip.read_flags(flags)[0] == 0
    return out


def test_noalloc_decode_equals_workspace_decode_twice(device):
    lib = _hip.load()
    calls = [([3000, 1, 2049, 700], 32, 8, 256, 1200), ([700, 65], 8, 2, 128, 1300)]
    for lens, hq, hkv, split, seed in calls:
        cache, table, q, cope = _case(device, lens, hq, hkv, seed)
        ws = decode_workspace(len(lens), hq, max(lens), split, device)
        want = _run(lib, "cs_ccpe_decode_bf16", device, cache, table, q, cope, lens, split, workspace=ws)
        got = _run(lib, "cs_ccpe_decode_bf16_noalloc", device, cache, table, q, cope, lens, split)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (lens, hq, hkv)


def test_noalloc_decode_refuses_more_than_its_scratch(device):
    lib = _hip.load()
    b, hq, split = 64, 32, 64
    max_nk = 1 << 20
    assert decode_workspace_bytes(b, hq, max_nk, split) > _hip.DECODE_SCRATCH_BYTES
    cache = torch.zeros((4, 8, 16, 256), dtype=torch.bfloat16, device=device)
    table = torch.zeros((b, 4), dtype=torch.int32, device=device)
    q = torch.zeros((b, hq, 128), dtype=torch.bfloat16, device=device)
    nk = torch.ones(b, dtype=torch.int32, device=device)
    out = torch.zeros_like(q)
    flags = _hip.new_flags(device)
    e = torch.zeros((128, 64), device=device)
    src = _paged_source(cache, table)
    status = lib.cs_ccpe_decode_bf16_noalloc(
        _hip.ptr(q), q.stride(0), q.stride(1), b, hq, 8, _hip.ptr(nk), max_nk, ctypes.byref(src),
        _hip.ptr(e), 64, split, _hip.ptr(out), _hip.ptr(flags), _hip.stream_of(device))
    assert status == _hip.CS_EINVAL
    assert b"static scratch holds" in lib.cs_last_error()
