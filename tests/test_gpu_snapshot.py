"""Layer snapshots through the page store and HBM on the MI355X (runtime.py:192-272).

Known answers: the safetensors library (the reference's codec) for page
bytes and decoded values, and torch's CPU ``.to`` for dtype conversions, all
compared bit for bit.
"""

from __future__ import annotations

import pytest
import torch
from safetensors.torch import load as st_load
from safetensors.torch import save as st_save

from cacheslide_amd import RequestPlan
from cacheslide_amd.runtime_rows import ReuseFailure
from cacheslide_amd.snapshot import LayerSnapshots, SnapshotUploader, encode_snapshot, parse_snapshot
from cacheslide_amd.pagestore import PageStore

pytestmark = pytest.mark.gpu

HKV, D, HID = 2, 16, 32


def plan(n_fixed=24, n=30):
    doc = {"version": 1, "operation": "populate", "namespace": "ns", "task_id": "t",
           "chunks": [{"id": "doc", "role": "reuse", "start": 0, "end": n_fixed},
                      {"id": "q", "role": "recompute", "start": n_fixed, "end": n}]}
    return RequestPlan.parse(doc, list(range(100, 100 + n)))


def bits(x: torch.Tensor) -> torch.Tensor:
    x = x.detach().cpu().contiguous()
    return x.view({2: torch.int16, 4: torch.int32, 8: torch.int64}[x.element_size()])


def snapshots(tmp_path, device, cpu=1 << 24, write_cache=True, **kwargs):
    store = PageStore(tmp_path / "pages", cpu_budget_bytes=cpu, disk_budget_bytes=1 << 26)
    snaps = LayerSnapshots(store, plan(), "model", device, layers=4, kv_heads=HKV, head_dim=D,
                           hidden_size=HID, write_cache=write_cache, **kwargs)
    return store, snaps


def layer_tensors(layer, device, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(layer)
    kv = {"k": torch.randn(24, HKV, D, generator=g), "v": torch.randn(24, HKV, D, generator=g)}
    state = {"hidden": torch.randn(24, HID, generator=g),
             "residual": torch.randn(24, HID, generator=g) if layer else torch.empty(0)}
    return ({n: t.to(device=device, dtype=dtype) for n, t in kv.items()},
            {n: t.to(device=device, dtype=dtype) for n, t in state.items()})


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64])
def test_encode_matches_safetensors(device, dtype):
    kv, state = layer_tensors(1, device, dtype)
    mixed = {"a": kv["k"], "b": kv["v"].float(), "c": state["hidden"][:, ::2]}   # strided source
    for tensors in (kv, state, layer_tensors(0, device, dtype)[1], mixed):
        assert encode_snapshot(tensors) == st_save({n: t.cpu().contiguous() for n, t in tensors.items()})


def test_put_read_round_trip_and_keys(device, tmp_path):
    store, snaps = snapshots(tmp_path, device)
    for layer in range(3):
        kv, state = layer_tensors(layer, device)
        snaps.put(layer, "state", state)
        snaps.put(layer, "kv", kv)
    assert len(snaps.created_keys) == 6
    assert snaps.key(1, "kv") == plan().cache_key("model", 1) + "/kv"
    assert store.keys() == tuple(sorted(snaps.created_keys))
    assert all(store.metadata(k)["backed"] for k in snaps.created_keys)   # spilled on put
    written = sum(store.metadata(k)["size"] for k in snaps.created_keys)
    assert snaps.metrics["snapshot_bytes_written"] == written
    for layer in range(3):
        kv, state = layer_tensors(layer, device)
        for kind, want in (("kv", kv), ("state", state)):
            got = snaps.read(layer, kind, torch.bfloat16)
            assert set(got) == set(want)
            for name in want:
                assert got[name].device == device and got[name].dtype == torch.bfloat16
                assert torch.equal(bits(got[name]), bits(want[name]))
        # the stored page is what safetensors decodes to the same values
        page = st_load(store.read(snaps.key(layer, "kv")))
        assert torch.equal(bits(page["k"]), bits(kv["k"]))
    with pytest.raises(ReuseFailure, match="cannot persist kv snapshot at layer 1"):
        snaps.put(1, "kv", layer_tensors(1, device)[0])   # immutable pages collide
    store.close()


@pytest.mark.parametrize("src, dst", [(torch.float32, torch.bfloat16), (torch.float32, torch.float16),
                                      (torch.float64, torch.bfloat16), (torch.float64, torch.float16),
                                      (torch.float64, torch.float32), (torch.bfloat16, torch.float32),
                                      (torch.float16, torch.bfloat16), (torch.bfloat16, torch.float64)])
def test_read_converts_like_torch(device, tmp_path, src, dst):
    store, snaps = snapshots(tmp_path, device)
    g = torch.Generator().manual_seed(7)
    k = torch.randn(24, HKV, D, generator=g, dtype=torch.float64) * 4
    # rounding edge cases: ties, values just under/over the 16-bit maxima, subnormals
    edge = torch.tensor([1 + 2**-8, 1 + 3 * 2**-8, 65504.0, 65519.99, 65520.0, 3.3895e38, 3.39e38,
                         2**-24, 2**-25, 1e-39, -2**-14 * 1.5, 1 + 2**-24 + 2**-53], dtype=torch.float64)
    k.view(-1)[:edge.numel()] = edge
    kv = {"k": k.to(src), "v": (-k).to(src)}
    if not all(torch.isfinite(t).all() for t in kv.values()):
        kv = {n: torch.nan_to_num(t, posinf=1.0, neginf=-1.0) for n, t in kv.items()}
    snaps.put(2, "kv", {n: t.to(device) for n, t in kv.items()})
    got = snaps.read(2, "kv", dst)
    for name in kv:
        assert torch.equal(bits(got[name]), bits(kv[name].to(dst))), name
    store.close()


def test_invalid_pages_raise_reuse_failure(device, tmp_path):
    store, snaps = snapshots(tmp_path, device)
    kv, state = layer_tensors(1, device)
    bad = dict(kv)
    bad["v"] = kv["v"].clone()
    bad["v"][3, 1, 5] = float("inf")
    snaps.put(1, "kv", bad)
    with pytest.raises(ReuseFailure, match="invalid kv snapshot at layer 1") as info:
        snaps.read(1, "kv", torch.bfloat16)
    assert "nonfinite" in str(info.value.__cause__)
    snaps.put(2, "kv", {"k": kv["k"], "v": kv["v"][:5]})            # wrong geometry
    with pytest.raises(ReuseFailure, match="invalid kv snapshot at layer 2"):
        snaps.read(2, "kv", torch.bfloat16)
    snaps.put(2, "state", {"hidden": state["hidden"]})                # missing field
    with pytest.raises(ReuseFailure, match="invalid state snapshot at layer 2"):
        snaps.read(2, "state", torch.bfloat16)
    with pytest.raises(ReuseFailure, match="invalid kv snapshot at layer 3"):
        snaps.read(3, "kv", torch.bfloat16)                           # no such page
    key = snaps.key(3, "kv")
    store.put(key, st_save({"k": torch.zeros(24, HKV, D, dtype=torch.int16),
                            "v": torch.zeros(24, HKV, D, dtype=torch.int16)}))
    with pytest.raises(ReuseFailure, match="invalid kv snapshot at layer 3"):
        snaps.read(3, "kv", torch.bfloat16)                           # not floating point
    store.close()


def test_prefetch_from_disk_overlaps_and_matches(device, tmp_path):
    # a RAM budget of one page: every other page is read back from its file
    page = len(encode_snapshot(layer_tensors(0, device)[0]))
    store, snaps = snapshots(tmp_path, device, cpu=page)
    for layer in range(4):
        snaps.put(layer, "kv", layer_tensors(layer, device)[0])
    reader = LayerSnapshots(store, plan(), "model", device, layers=4, kv_heads=HKV, head_dim=D,
                            hidden_size=HID, uploader=snaps.uploader)
    busy = torch.randn(2048, 2048, device=device)
    reader.prefetch(0, torch.bfloat16)
    for layer in range(4):
        for _ in range(3):
            busy = torch.tanh(busy @ busy.T * 1e-3)                       # compute while the page moves
        got = reader.read(layer, "kv", torch.bfloat16)
        reader.prefetch(layer + 1, torch.bfloat16)                        # layer 4 does not exist: no-op
        want = layer_tensors(layer, device)[0]
        for name in want:
            assert torch.equal(bits(got[name]), bits(want[name]))
    assert reader.kv_future is None
    reader.prefetch(1, torch.bfloat16)
    with pytest.raises(RuntimeError, match="more than one outstanding KV prefetch"):
        reader.prefetch(2, torch.bfloat16)
    got = reader.read(1, "kv", torch.float32)                             # prefetched for bf16
    assert torch.equal(bits(got["k"]), bits(layer_tensors(1, device)[0]["k"].float()))
    reader.prefetch(2, torch.bfloat16)
    reader.release()
    assert reader.kv_future is None
    assert store.stats()["inflight_loads"] == 0
    reader.uploader.close()
    store.close()


def test_uploader_streams_pages_in_order(device):
    uploader = SnapshotUploader(device, slots=2)
    pages = []
    for i in range(6):
        g = torch.Generator().manual_seed(i)
        t = {"k": torch.randn(64, 4, 8, generator=g).bfloat16(), "v": torch.randn(64, 4, 8, generator=g).bfloat16()}
        pages.append((t, st_save(t)))
    futures = [uploader.submit(lambda d=d: d, {"k": (64, 4, 8), "v": (64, 4, 8)}, torch.bfloat16)
               for _, d in pages]
    for (want, data), future in zip(pages, futures):
        got = SnapshotUploader.take(future)
        assert torch.equal(bits(got["k"]), bits(want["k"])) and torch.equal(bits(got["v"]), bits(want["v"]))
        assert parse_snapshot(data)[1] > 8
    assert uploader.uploaded_bytes == sum(len(d) - parse_snapshot(d)[1] for _, d in pages)
    with pytest.raises(ValueError):
        uploader.submit(lambda: pages[0][1], {"k": (64, 4, 8), "v": (64, 4, 8)}, torch.int32)
    uploader.close()


def test_prefetch_depth_keeps_layers_in_flight(device, tmp_path):
    store, snaps = snapshots(tmp_path, device)
    for layer in range(4):
        snaps.put(layer, "kv", layer_tensors(layer, device)[0])
    reader = LayerSnapshots(store, plan(), "model", device, layers=4, kv_heads=HKV, head_dim=D,
                            hidden_size=HID, prefetch_depth=3)
    reader.prefetch(0, torch.bfloat16)
    assert sorted(reader._pending) == [0, 1, 2] and reader.kv_future_layer == 0
    for layer in range(4):
        got = reader.read(layer, "kv", torch.bfloat16)
        reader.prefetch(layer + 1, torch.bfloat16)
        assert len(reader._pending) <= 3
        want = layer_tensors(layer, device)[0]
        assert all(torch.equal(bits(got[n]), bits(want[n])) for n in want)
    assert reader.kv_future is None
    with pytest.raises(ValueError):
        LayerSnapshots(store, plan(), "model", device, layers=4, kv_heads=HKV, head_dim=D,
                       hidden_size=HID, prefetch_depth=0)
    reader.uploader.close()
    snaps.uploader.close()
    store.close()


def _hand_page(entries, body, pad=True, metadata=None):
    import json
    import struct
    header = dict(entries)
    if metadata is not None:
        header = {"__metadata__": metadata, **header}
    text = json.dumps(header, separators=(",", ":")).encode()
    if pad:
        text += b" " * (-len(text) % 8)
    return struct.pack("<Q", len(text)) + text + body


@pytest.mark.parametrize("layout", ["reversed_entries", "unpadded_metadata", "odd_offsets"])
def test_unusual_valid_pages_decode_like_safetensors(device, layout):
    g = torch.Generator().manual_seed(3)
    k = torch.randn(5, 2, 3, generator=g).to(torch.bfloat16)
    v = torch.randn(5, 2, 3, generator=g).to(torch.float32)
    kb, vb = k.view(torch.uint8).numpy().tobytes(), v.view(torch.uint8).numpy().tobytes()
    ek = {"dtype": "BF16", "shape": [5, 2, 3]}
    ev = {"dtype": "F32", "shape": [5, 2, 3]}
    if layout == "reversed_entries":    # v first in the data region, entries listed k first
        page = _hand_page({"k": {**ek, "data_offsets": [len(vb), len(vb) + len(kb)]},
                           "v": {**ev, "data_offsets": [0, len(vb)]}}, vb + kb)
    elif layout == "unpadded_metadata":
        page = _hand_page({"k": {**ek, "data_offsets": [0, len(kb)]},
                           "v": {**ev, "data_offsets": [len(kb), len(kb) + len(vb)]}}, kb + vb,
                          pad=False, metadata={"format": "pt"})
    else:                               # k (60 bytes) first: v starts 4-byte aligned only
        page = _hand_page({"k": {**ek, "data_offsets": [0, 60]},
                           "v": {**ev, "data_offsets": [60, 60 + len(vb)]}}, kb + vb)
    want = st_load(page)
    uploader = SnapshotUploader(device)
    for dtype in (torch.bfloat16, torch.float32):
        got = SnapshotUploader.take(uploader.submit(lambda: page, {"k": (5, 2, 3), "v": (5, 2, 3)}, dtype))
        for name in ("k", "v"):
            assert torch.equal(bits(got[name]), bits(want[name].to(dtype))), (layout, dtype, name)
    uploader.close()
