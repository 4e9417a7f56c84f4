"""LayerSnapshots' host logic on the CPU (runtime.py:192-272).

Keys, the write_cache switch, immutable-page collisions, the error mapping to
ReuseFailure with the reference's messages, and the prefetch bookkeeping
(one outstanding K/V prefetch at depth 1, a window at larger depths) do not
need the device: a stand-in uploader decodes pages with the safetensors
library after the same header and schema checks, and pages are encoded by
safetensors as the reference's _put does.
"""

from __future__ import annotations

from concurrent.futures import Future

import pytest
import torch
from safetensors.torch import load as st_load
from safetensors.torch import save as st_save

from cacheslide_amd import RequestPlan
from cacheslide_amd import snapshot as snap
from cacheslide_amd.runtime_rows import ReuseFailure
from cacheslide_amd.pagestore import PageStore

HKV, D, HID = 2, 4, 8


class HostUploader:
    """Decodes on the CPU what SnapshotUploader uploads: same checks, same errors."""

    def __init__(self):
        self.submitted = 0
        self.drained = 0

    def submit(self, fetch, shapes, dtype):
        self.submitted += 1
        future = Future()
        try:
            data = fetch()
            tensors, _ = snap.parse_snapshot(data)
            snap.check_schema(tensors, shapes)
            out = {n: t.to(dtype) for n, t in st_load(data).items()}
            if not all(torch.isfinite(t).all() for t in out.values()):
                raise ValueError("snapshot tensor is nonfinite")
            future.set_result(out)
        except Exception as exc:  # the device uploader fails the future the same way
            future.set_exception(exc)
        return future

    @staticmethod
    def take(future):
        return future.result()

    def drain(self, future):
        self.drained += 1


def plan():
    doc = {"version": 1, "operation": "populate", "namespace": "ns", "task_id": "t",
           "chunks": [{"id": "doc", "role": "reuse", "start": 0, "end": 6},
                      {"id": "q", "role": "recompute", "start": 6, "end": 8}]}
    return RequestPlan.parse(doc, list(range(10, 18)))


@pytest.fixture
def env(tmp_path, monkeypatch):
    # pages encoded from CPU tensors as the reference's _put does
    monkeypatch.setattr(snap, "encode_snapshot", lambda tensors: st_save(
        {n: t.detach().contiguous().cpu() for n, t in tensors.items()}))
    store = PageStore(tmp_path / "pages", cpu_budget_bytes=1 << 20, disk_budget_bytes=1 << 22)
    yield store
    store.close()


def snapshots(store, **kwargs):
    kwargs.setdefault("uploader", HostUploader())
    return snap.LayerSnapshots(store, plan(), "model", "cpu", layers=4, kv_heads=HKV, head_dim=D,
                               hidden_size=HID, **kwargs)


def kv(layer):
    g = torch.Generator().manual_seed(layer)
    return {"k": torch.randn(6, HKV, D, generator=g), "v": torch.randn(6, HKV, D, generator=g)}


def test_keys_and_write_switch(env):
    s = snapshots(env)
    assert s.key(2, "kv") == plan().cache_key("model", 2) + "/kv"
    assert s.key(2, "state") == plan().cache_key("model", 2) + "/state"
    s.put(1, "kv", kv(1))                       # write_cache False: nothing persisted
    assert env.keys() == () and s.created_keys == []
    w = snapshots(env, write_cache=True)
    w.put(1, "kv", kv(1))
    assert env.keys() == (w.key(1, "kv"),) and w.created_keys == [w.key(1, "kv")]
    assert env.metadata(w.key(1, "kv"))["backed"]
    assert w.metrics["snapshot_bytes_written"] == env.metadata(w.key(1, "kv"))["size"]
    with pytest.raises(ReuseFailure, match="cannot persist kv snapshot at layer 1"):
        w.put(1, "kv", kv(1))
    got = w.read(1, "kv", torch.float32)
    assert all(torch.equal(got[n], kv(1)[n]) for n in ("k", "v"))


def test_read_errors_map_to_reuse_failure(env):
    s = snapshots(env, write_cache=True)
    with pytest.raises(ReuseFailure, match="invalid kv snapshot at layer 0"):
        s.read(0, "kv", torch.float32)          # no page
    s.put(0, "kv", {"k": kv(0)["k"]})           # a field missing
    with pytest.raises(ReuseFailure, match="invalid kv snapshot at layer 0"):
        s.read(0, "kv", torch.float32)
    s.put(0, "state", {"hidden": torch.zeros(6, HID), "residual": torch.zeros(6, HID)})
    with pytest.raises(ReuseFailure, match="invalid state snapshot at layer 0") as info:
        s.read(0, "state", torch.float32)       # layer 0 stores an empty residual
    assert "geometry" in str(info.value.__cause__)
    s.put(1, "state", {"hidden": torch.zeros(6, HID), "residual": torch.full((6, HID), float("inf"))})
    with pytest.raises(ReuseFailure, match="invalid state snapshot at layer 1") as info:
        s.read(1, "state", torch.float32)
    assert "nonfinite" in str(info.value.__cause__)
    s.put(2, "state", {"hidden": torch.zeros(6, HID), "residual": torch.empty(0)})
    with pytest.raises(ReuseFailure, match="invalid state snapshot at layer 2"):
        s.read(2, "state", torch.float32)       # only layer 0 may have an empty residual


def test_prefetch_depth_one_is_the_reference_policy(env):
    w = snapshots(env, write_cache=True)
    for layer in range(4):
        w.put(layer, "kv", kv(layer))
    up = HostUploader()
    s = snapshots(env, uploader=up)
    assert s.kv_future is None and s.kv_future_layer == -1
    s.prefetch(0, torch.float32)
    assert s.kv_future_layer == 0 and up.submitted == 1
    with pytest.raises(RuntimeError, match="more than one outstanding KV prefetch"):
        s.prefetch(1, torch.float32)
    got = s.read(0, "kv", torch.float32)        # consumes the prefetch
    assert torch.equal(got["k"], kv(0)["k"]) and s.kv_future is None
    s.prefetch(4, torch.float32)                # past the last layer: nothing
    s.prefetch(3, torch.float32)
    assert s.kv_future_layer == 3
    s.release()
    assert s.kv_future is None and up.drained == 1
    off = snapshots(env, uploader=HostUploader(), reuse=False)
    off.prefetch(0, torch.float32)
    assert off.kv_future is None


def test_prefetch_window(env):
    w = snapshots(env, write_cache=True)
    for layer in range(4):
        w.put(layer, "kv", kv(layer))
    s = snapshots(env, prefetch_depth=3)
    s.prefetch(0, torch.float32)
    assert sorted(s._pending) == [0, 1, 2]
    s.read(0, "kv", torch.float32)
    s.prefetch(1, torch.float32)                # tops the window up to layers 1..3
    assert sorted(s._pending) == [1, 2, 3]
    for layer in (1, 2, 3):
        assert torch.equal(s.read(layer, "kv", torch.float32)["v"], kv(layer)["v"])
    assert s._pending == {}
    with pytest.raises(ValueError):
        snapshots(env, prefetch_depth=0)


def test_close_drains_and_closes_only_an_owned_uploader(env):
    w = snapshots(env, write_cache=True)
    w.put(0, "kv", kv(0))

    class Owned(HostUploader):
        closed = False

        def close(self):
            self.closed = True

    shared = Owned()
    with snapshots(env, uploader=shared) as s:
        s.prefetch(0, torch.float32)
    assert s.kv_future is None and shared.drained == 1 and not shared.closed
    owned = snapshots(env)
    owned._owns_uploader, owned.uploader = True, Owned()
    owned.close()
    assert owned.uploader.closed
