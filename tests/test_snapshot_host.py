"""Snapshot page codec on the CPU, against the safetensors library (runtime.py:192-256).

The reference writes snapshot pages with ``safetensors.torch.save`` and reads
them with ``safetensors.torch.load`` (runtime.py:17-18), pinned at
safetensors==0.8.0 (constraints/cpu-tests.txt:4).  That version is installed
here, so it is the known answer: the page header and layout built
by ``snapshot_header`` must reproduce its bytes exactly, and ``parse_snapshot``
must accept what it loads and reject what it refuses.
"""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import load as st_load
from safetensors.torch import save as st_save

from cacheslide_amd.snapshot import check_schema, parse_snapshot, snapshot_header, snapshot_shapes

DTYPES = [torch.float64, torch.float32, torch.bfloat16, torch.float16, torch.int64, torch.int32,
          torch.int16, torch.int8, torch.uint8, torch.bool, torch.float8_e4m3fn, torch.float8_e5m2]


def random_tensor(gen, dtype, shape):
    x = torch.randn(shape, generator=gen, dtype=torch.float64) * 3
    if dtype == torch.bool:
        return x > 0
    if not dtype.is_floating_point:
        return x.to(torch.int64).to(dtype)
    return x.to(dtype)


def host_encode(tensors):
    """Page bytes from the header builder plus the tensors' little-endian bytes."""
    header, layout = snapshot_header({n: (t.dtype, tuple(t.shape)) for n, t in tensors.items()})
    body = b"".join(tensors[t.name].contiguous().view(-1).view(torch.uint8).numpy().tobytes() for t in layout)
    return header + body


@pytest.mark.parametrize("seed", range(12))
def test_header_and_layout_match_safetensors(seed):
    gen = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    names = ["k", "v", "hidden", "residual", "a", "é-名", "x" * 40, "z0"]
    tensors = {}
    for name in rng.choice(names, size=rng.integers(1, 7), replace=False):
        dtype = DTYPES[rng.integers(len(DTYPES))]
        shape = tuple(int(s) for s in rng.integers(0, 5, size=rng.integers(0, 4)))
        tensors[str(name)] = random_tensor(gen, dtype, shape)
    want = st_save(tensors)
    assert host_encode(tensors) == want
    parsed, start = parse_snapshot(want)
    _, layout = snapshot_header({n: (t.dtype, tuple(t.shape)) for n, t in tensors.items()})
    assert sorted(parsed, key=lambda t: t.begin) == layout
    assert start == 8 + struct.unpack("<Q", want[:8])[0]
    loaded = st_load(want)
    for t in parsed:
        assert t.torch_dtype == loaded[t.name].dtype and t.shape == tuple(loaded[t.name].shape)


def test_runtime_pages_and_empty_page():
    gen = torch.Generator().manual_seed(0)
    kv = {"k": random_tensor(gen, torch.bfloat16, (37, 8, 128)), "v": random_tensor(gen, torch.bfloat16, (37, 8, 128))}
    state0 = {"hidden": random_tensor(gen, torch.float16, (5, 64)), "residual": torch.empty(0, dtype=torch.float16)}
    for tensors in (kv, state0, {}):
        assert host_encode(tensors) == st_save(tensors)
    # K precedes V in the data region; the residual of layer 0 is an empty range
    tensors, start = parse_snapshot(st_save(kv))
    assert [(t.name, t.begin) for t in sorted(tensors, key=lambda t: t.begin)] == [("k", 0), ("v", 37 * 8 * 128 * 2)]
    tensors, _ = parse_snapshot(st_save(state0))
    assert {t.name: t.end - t.begin for t in tensors} == {"hidden": 640, "residual": 0}


def _page(entries, body, pad=True, metadata=None):
    header = dict(entries)
    if metadata is not None:
        header = {"__metadata__": metadata, **header}
    text = json.dumps(header, separators=(",", ":")).encode()
    if pad:
        text += b" " * (-len(text) % 8)
    return struct.pack("<Q", len(text)) + text + body


def _entry(dtype, shape, begin, end):
    return {"dtype": dtype, "shape": shape, "data_offsets": [begin, end]}


GOOD = _page({"k": _entry("F32", [2], 0, 8), "v": _entry("F32", [2], 8, 16)}, bytes(16))

MALFORMED = {
    "short": b"\x00" * 7,
    "header_past_end": struct.pack("<Q", 1000) + b"{}",
    "huge_header": struct.pack("<Q", 100_000_001) + b"{}",
    "not_utf8": struct.pack("<Q", 2) + b"\xff\xfe",
    "not_object": struct.pack("<Q", 2) + b"[]",
    "bad_json": struct.pack("<Q", 3) + b"{x}",
    "unknown_dtype": _page({"k": _entry("F24", [2], 0, 6)}, bytes(6)),
    "gap": _page({"k": _entry("F32", [2], 0, 8), "v": _entry("F32", [2], 12, 20)}, bytes(20)),
    "overlap": _page({"k": _entry("F32", [2], 0, 8), "v": _entry("F32", [2], 4, 12)}, bytes(12)),
    "not_from_zero": _page({"k": _entry("F32", [2], 4, 12)}, bytes(12)),
    "size_mismatch": _page({"k": _entry("F32", [3], 0, 8)}, bytes(8)),
    "trailing_bytes": GOOD + b"\x00",
    "truncated_data": GOOD[:-1],
    "negative_shape": _page({"k": _entry("F32", [-2], 0, 8)}, bytes(8)),
    "float_shape": _page({"k": _entry("F32", [2.0], 0, 8)}, bytes(8)),
    "missing_offsets": _page({"k": {"dtype": "F32", "shape": [2]}}, bytes(8)),
    "reversed_offsets": _page({"k": _entry("F32", [0], 8, 0)}, bytes(8)),
    "entry_not_object": _page({"k": [1, 2]}, b""),
    "metadata_not_strings": _page({"k": _entry("F32", [2], 0, 8)}, bytes(8), metadata={"a": 1}),
}


@pytest.mark.parametrize("case", sorted(MALFORMED))
def test_malformed_pages_rejected_like_safetensors(case):
    data = MALFORMED[case]
    with pytest.raises(Exception):
        st_load(data)
    with pytest.raises(ValueError):
        parse_snapshot(data)


@pytest.mark.parametrize("page", [
    GOOD,
    _page({"k": _entry("F32", [2], 0, 8)}, bytes(8), pad=False),                      # unpadded header
    _page({"k": _entry("F32", [2], 0, 8)}, bytes(8), metadata={"format": "pt"}),      # metadata
    _page({"v": _entry("F32", [2], 8, 16), "k": _entry("F32", [2], 0, 8)}, bytes(16)),  # entries out of order
    _page({"k": _entry("BF16", [0, 3], 0, 0), "v": _entry("U8", [3], 0, 3)}, bytes(3)),  # empty tensor
])
def test_unusual_but_valid_pages_accepted_like_safetensors(page):
    loaded = st_load(page)
    tensors, start = parse_snapshot(page)
    assert {t.name for t in tensors} == set(loaded)
    for t in tensors:
        assert t.torch_dtype == loaded[t.name].dtype and t.shape == tuple(loaded[t.name].shape)
        raw = page[start + t.begin:start + t.end]
        assert raw == loaded[t.name].contiguous().view(-1).view(torch.uint8).numpy().tobytes()


def test_runtime_schema():
    # runtime.py:207-226
    assert snapshot_shapes("kv", 3, 10, kv_heads=8, head_dim=128, hidden_size=4096) == {
        "k": (10, 8, 128), "v": (10, 8, 128)}
    assert snapshot_shapes("state", 0, 10, kv_heads=8, head_dim=128, hidden_size=64) == {
        "hidden": (10, 64), "residual": (0,)}
    assert snapshot_shapes("state", 1, 10, kv_heads=8, head_dim=128, hidden_size=64)["residual"] == (10, 64)
    with pytest.raises(ValueError):
        snapshot_shapes("other", 0, 1, kv_heads=1, head_dim=1, hidden_size=1)
    shapes = {"k": (2, 1, 4), "v": (2, 1, 4)}

    def page(**tensors):
        return parse_snapshot(st_save(tensors))[0]

    ok = torch.zeros(2, 1, 4, dtype=torch.bfloat16)
    check_schema(page(k=ok, v=ok.float()), shapes)
    with pytest.raises(ValueError, match="fields differ"):
        check_schema(page(k=ok), shapes)
    with pytest.raises(ValueError, match="fields differ"):
        check_schema(page(k=ok, v=ok.clone(), w=ok.clone()), shapes)
    with pytest.raises(ValueError, match="geometry"):
        check_schema(page(k=ok, v=torch.zeros(3, 1, 4)), shapes)
    with pytest.raises(ValueError, match="geometry"):
        check_schema(page(k=ok, v=torch.zeros(2, 1, 4, dtype=torch.int32)), shapes)
    # float8 pages are floating point for the reference but have no device check here
    with pytest.raises(ValueError, match="not supported"):
        check_schema(page(k=ok, v=torch.zeros(2, 1, 4, dtype=torch.float8_e4m3fn)), shapes)


from hypothesis import HealthCheck, given, settings  # noqa: E402
from hypothesis import strategies as hst  # noqa: E402

_FUZZ_DTYPES = [torch.float32, torch.bfloat16, torch.float16, torch.float64, torch.int32, torch.uint8]


@hst.composite
def mutated_pages(draw):
    names = draw(hst.lists(hst.sampled_from(["k", "v", "hidden", "residual", "x"]), min_size=1, max_size=3,
                           unique=True))
    tensors = {}
    for name in names:
        dtype = draw(hst.sampled_from(_FUZZ_DTYPES))
        shape = tuple(draw(hst.lists(hst.integers(0, 3), min_size=0, max_size=3)))
        tensors[name] = torch.arange(math_prod(shape), dtype=torch.float64).reshape(shape).to(dtype)
    page = bytearray(st_save(tensors))
    kind = draw(hst.sampled_from(["flip", "truncate", "append", "digit", "none"]))
    if kind == "flip":
        at = draw(hst.integers(0, len(page) - 1))
        page[at] ^= draw(hst.integers(1, 255))
    elif kind == "truncate":
        page = page[:draw(hst.integers(0, len(page) - 1))]
    elif kind == "append":
        page += bytes(draw(hst.integers(1, 9)))
    elif kind == "digit":
        header_end = 8 + int.from_bytes(page[:8], "little")
        digits = [i for i in range(8, min(header_end, len(page))) if chr(page[i]).isdigit()]
        if digits:
            at = draw(hst.sampled_from(digits))
            page[at] = ord(str((int(chr(page[at])) + draw(hst.integers(1, 9))) % 10))
    return bytes(page)


def math_prod(shape):
    out = 1
    for s in shape:
        out *= s
    return out


@settings(max_examples=300, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(mutated_pages())
def test_parse_accepts_exactly_what_safetensors_loads(page):
    try:
        loaded = st_load(page)
    except Exception:
        loaded = None
    try:
        tensors, start = parse_snapshot(page)
    except ValueError:
        tensors = None
    assert (loaded is None) == (tensors is None)
    if loaded is not None:
        assert {t.name for t in tensors} == set(loaded)
        for t in tensors:
            assert t.torch_dtype == loaded[t.name].dtype and t.shape == tuple(loaded[t.name].shape)
            assert page[start + t.begin:start + t.end] == loaded[t.name].contiguous().view(-1).view(
                torch.uint8).numpy().tobytes()
