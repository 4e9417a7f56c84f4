"""The RAM/SSD page store of layer snapshots, on the CPU (tests/test_storage.py).

Each test restates one of the reference's storage tests (cited by line); the
format tests pin the ``cacheslide-pages-v1`` page file against values fixed by
the format itself: sha256 of known payloads and a page file assembled by hand
the way storage.py:176-190 and 326-368 lay it out.
"""

from __future__ import annotations

import hashlib
import json
import os
import threading
from concurrent.futures import ThreadPoolExecutor

import pytest

from cacheslide_amd.storage import (
    CacheCapacityError,
    CacheIntegrityError,
    StaleCompletionError,
    TieredPageStore,
    encode_page_header,
    page_filename,
)

SHA_DATA = "3a6eb0790f39ac87c94f3856b2dd2c5d110e6811602261a9a923d3bb23adc8b7"  # sha256(b"data")


def store_at(tmp_path, cpu=16, disk=100_000, **kwargs):
    return TieredPageStore(tmp_path / "pages", cpu_budget_bytes=cpu, disk_budget_bytes=disk, **kwargs)


def page_files(tmp_path):
    return sorted((tmp_path / "pages").glob("*.page"))


# ----------------------------------------------------------------- format
def test_page_file_layout_is_the_reference_format(tmp_path):
    key = "model/adapter:../../request?layer=2"
    with store_at(tmp_path) as store:
        store.put(key, b"data", selected_count=2)
        store.submit_spill(key).result(timeout=5)
        generation = store.metadata(key)["generation"]
    (path,) = page_files(tmp_path)
    assert path.name == hashlib.sha256(key.encode()).hexdigest() + "." + generation + ".page"
    assert ".." not in path.name and "/" not in path.name
    header = ('{"checksum":"' + SHA_DATA + '","format":"cacheslide-pages-v1","generation":"'
              + generation + '","key":"' + key + '","selected_count":2,"size":4}\n').encode()
    assert path.read_bytes() == header + b"data"
    marker = json.loads((tmp_path / "pages" / ".cacheslide-store.json").read_text())
    assert marker == {"format": "cacheslide-pages-v1"}
    assert not (tmp_path / "pages" / ".writer.lock").exists()


def test_hand_written_page_directory_is_adopted(tmp_path):
    root = tmp_path / "pages"
    root.mkdir()
    (root / ".cacheslide-store.json").write_text('{"format": "cacheslide-pages-v1"}')
    generation = "0123456789abcdef0123456789abcdef"
    header = encode_page_header("layer:7/kv", generation, SHA_DATA, 4, 0)
    assert header == ('{"checksum":"' + SHA_DATA + '","format":"cacheslide-pages-v1","generation":"'
                      + generation + '","key":"layer:7/kv","selected_count":0,"size":4}\n').encode()
    name = "b04265acb3b6302c3ea0a60b16931b832b1b72179893f7e10df4d2267c1308f9." + generation + ".page"
    assert page_filename("layer:7/kv", generation) == name
    (root / name).write_bytes(header + b"data")
    with store_at(tmp_path) as store:
        assert store.keys() == ("layer:7/kv",)
        meta = store.metadata("layer:7/kv")
        assert meta["backed"] and not meta["resident"] and meta["generation"] == generation
        assert store.read("layer:7/kv") == b"data"
        assert store.stats()["live_disk_bytes"] == len(header) + 4


@pytest.mark.parametrize("damage", ["rename", "size", "format", "selected", "header", "checksum"])
def test_damaged_page_directories_are_refused(tmp_path, damage):
    root = tmp_path / "pages"
    root.mkdir()
    (root / ".cacheslide-store.json").write_text('{"format": "cacheslide-pages-v1"}')
    generation = "g"
    fields = {"checksum": SHA_DATA, "format": "cacheslide-pages-v1", "generation": generation,
              "key": "k", "selected_count": 0, "size": 4}
    payload, name = b"data", page_filename("k", generation)
    if damage == "rename":
        name = page_filename("other", generation)
    elif damage == "size":
        fields["size"] = 5
    elif damage == "format":
        fields["format"] = "cacheslide-pages-v0"
    elif damage == "selected":
        fields["selected_count"] = -1
    elif damage == "checksum":
        payload = b"dat!"
    line = json.dumps(fields, sort_keys=True, separators=(",", ":")).encode()
    if damage == "header":
        line = line[:-1]
    (root / name).write_bytes(line + b"\n" + payload)
    with pytest.raises(CacheIntegrityError):
        store_at(tmp_path)
    assert not (root / ".writer.lock").exists()


def test_pending_write_and_symlink_pages_require_recovery(tmp_path):
    with store_at(tmp_path):
        pass
    pending = tmp_path / "pages" / ".pending-abc"
    pending.write_bytes(b"x")
    with pytest.raises(CacheIntegrityError, match="unfinished"):
        store_at(tmp_path)
    pending.unlink()
    (tmp_path / "pages" / "x.page").symlink_to(tmp_path / "elsewhere")
    with pytest.raises(CacheIntegrityError):
        store_at(tmp_path)


def test_budget_arguments_and_long_keys(tmp_path):
    with pytest.raises(ValueError):
        TieredPageStore(tmp_path / "a", cpu_budget_bytes=-1, disk_budget_bytes=1)
    with pytest.raises(ValueError):
        TieredPageStore(tmp_path / "b", cpu_budget_bytes=1, disk_budget_bytes=1, max_workers=0)
    with store_at(tmp_path) as store:
        with pytest.raises(ValueError, match="too long"):
            store.put("k" * 70_000, b"")
        assert store.stats()["pages"] == 0
        for bad in ((1, b""), ("", b""), ("k", "text"), ("k", b"", -1), ("k", b"", True)):
            with pytest.raises(ValueError):
                store.put(*bad)
        with pytest.raises(CacheCapacityError, match="exceeds the CPU budget"):
            store.put("big", b"x" * 17)


# ----------------------------------------------- the reference's storage tests
def test_immutable_pages_survive_restart(tmp_path):
    # tests/test_storage.py:21-39
    key = "model/adapter:../../request?layer=2"
    with store_at(tmp_path) as store:
        store.put(key, b"data", selected_count=2)
        store.put(key, b"data", selected_count=2)
        with pytest.raises(ValueError):
            store.put(key, b"changed", selected_count=2)
        with pytest.raises(ValueError):
            store.put(key, b"data", selected_count=3)
        store.submit_spill(key).result(timeout=5)
        assert store.read(key) == b"data"
        stats = store.stats()
        assert stats["payload_write_bytes"] == 4
        assert stats["physical_host_write_bytes"] > 4
        assert len(page_files(tmp_path)) == 1
    with store_at(tmp_path) as reopened:
        assert reopened.stats()["live_cpu_bytes"] == 0
        assert reopened.read(key) == b"data"
        assert reopened.stats()["inflight_cpu_reserved_bytes"] == 0
        # re-put of a disk-only page is checked against its published copy
        reopened.put(key, b"data", selected_count=2)


def test_eviction_order(tmp_path):
    # tests/test_storage.py:42-53: clean first, then descending selected count, LRU ties
    with store_at(tmp_path, cpu=4) as store:
        store.put("dirty-two-old", b"a", selected_count=2)
        store.put("clean", b"b")
        store.put("dirty-five", b"c", selected_count=5)
        store.put("dirty-two-new", b"d", selected_count=2)
        assert [store.evict()[0] for _ in range(4)] == ["clean", "dirty-five", "dirty-two-old",
                                                         "dirty-two-new"]
        assert store.stats()["live_cpu_bytes"] == 0
        with pytest.raises(CacheCapacityError):
            store.evict()


def test_required_bytes_eviction_and_lru_refresh(tmp_path):
    with store_at(tmp_path, cpu=6) as store:
        store.put("a", b"aa")
        store.put("b", b"bb")
        store.put("c", b"cc")
        store.read("a")                       # a becomes the most recent
        assert store.evict(3) == ["b", "c"]
        assert store.evict(2) == []
        with pytest.raises(ValueError):
            store.evict(-1)
        with pytest.raises(CacheCapacityError):
            store.evict(7)


def test_pinned_capacity_raises_without_discarding(tmp_path):
    # tests/test_storage.py:56-68
    with store_at(tmp_path, cpu=4) as store:
        store.put("a", b"aaaa")
        with store.pin("a") as data:
            assert data == b"aaaa"
            assert store.stats()["pinned_pages"] == 1
            with pytest.raises(CacheCapacityError):
                store.put("b", b"bbbb")
            with pytest.raises(CacheCapacityError):
                store.evict()
            with pytest.raises(CacheCapacityError):
                store.delete("a")
        assert store.read("a") == b"aaaa"
        assert store.stats()["pinned_pages"] == 0


def test_unbacked_page_kept_when_disk_is_full(tmp_path):
    # tests/test_storage.py:71-80
    with store_at(tmp_path, cpu=4, disk=1) as store:
        store.put("a", b"aaaa")
        with pytest.raises(CacheCapacityError):
            store.put("b", b"bbbb")
        assert store.read("a") == b"aaaa"
        assert store.stats()["live_cpu_bytes"] == 4
        assert store.stats()["live_disk_bytes"] == 0
        assert not page_files(tmp_path)


def test_corrupt_backing_blocks_eviction_and_reopen(tmp_path):
    # tests/test_storage.py:83-97
    with store_at(tmp_path) as store:
        store.put("a", b"original")
        store.submit_spill("a").result(timeout=5)
        (path,) = page_files(tmp_path)
        with path.open("r+b") as stream:
            stream.seek(-1, 2)
            stream.write(b"!")
        with pytest.raises(CacheIntegrityError):
            store.evict()
        assert store.read("a") == b"original"
    with pytest.raises(CacheIntegrityError):
        store_at(tmp_path)


def test_resident_payload_is_verified_on_read(tmp_path):
    with store_at(tmp_path) as store:
        store.put("a", b"data")
        store._pages["a"].payload = b"dat!"   # memory corruption of the resident copy
        with pytest.raises(CacheIntegrityError):
            store.read("a")
        with pytest.raises(CacheIntegrityError):
            store.submit_spill("a").result(timeout=5)
        assert not page_files(tmp_path)


def test_async_loads_reserve_capacity(tmp_path, monkeypatch):
    # tests/test_storage.py:100-130
    with store_at(tmp_path, cpu=8, max_workers=2) as store:
        store.put("a", b"aaaa")
        store.put("b", b"bbbb")
        store.evict()
        store.evict()
        entered, release = threading.Event(), threading.Event()
        read = store._read_disk

        def held(entry):
            entered.set()
            assert release.wait(5)
            return read(entry)

        monkeypatch.setattr(store, "_read_disk", held)
        first = store.submit_load("a")
        assert entered.wait(5)
        second = store.submit_load("b")
        try:
            assert store.submit_load("a") is first
            assert store.stats()["inflight_cpu_reserved_bytes"] == 8
            assert store.stats()["inflight_pages"] == 2
            with pytest.raises(CacheCapacityError):
                store.put("c", b"cccc")
            with pytest.raises(CacheCapacityError):
                store.delete("a")
        finally:
            release.set()
        assert first.result(timeout=5) == b"aaaa"
        assert second.result(timeout=5) == b"bbbb"
        stats = store.stats()
        assert stats["live_cpu_bytes"] == 8 and stats["inflight_cpu_reserved_bytes"] == 0


def test_failed_load_releases_reservation(tmp_path, monkeypatch):
    # tests/test_storage.py:133-147
    with store_at(tmp_path, cpu=4) as store:
        store.put("a", b"aaaa")
        store.evict()
        read = store._read_disk

        def fail(_):
            raise OSError("injected")

        monkeypatch.setattr(store, "_read_disk", fail)
        with pytest.raises(OSError):
            store.submit_load("a").result(timeout=5)
        assert store.stats()["inflight_cpu_reserved_bytes"] == 0
        assert store.stats()["live_disk_bytes"] > 0
        monkeypatch.setattr(store, "_read_disk", read)
        assert store.read("a") == b"aaaa"


def test_failed_write_keeps_payload(tmp_path, monkeypatch):
    # tests/test_storage.py:150-163
    with store_at(tmp_path, cpu=4) as store:
        store.put("a", b"aaaa")

        def fail(*_):
            raise OSError("injected")

        monkeypatch.setattr(store, "_write_page", fail)
        with pytest.raises(OSError):
            store.submit_spill("a").result(timeout=5)
        stats = store.stats()
        assert stats["inflight_disk_reserved_bytes"] == 0 and stats["inflight_pages"] == 0
        assert store.read("a") == b"aaaa"


def test_refuses_foreign_root_and_second_writer(tmp_path):
    # tests/test_storage.py:166-175
    foreign = tmp_path / "foreign"
    foreign.mkdir()
    (foreign / "user.txt").write_text("keep")
    with pytest.raises(ValueError):
        TieredPageStore(foreign, cpu_budget_bytes=8, disk_budget_bytes=1000)
    assert (foreign / "user.txt").read_text() == "keep"
    other = tmp_path / "other"
    other.mkdir()
    (other / ".cacheslide-store.json").write_text('{"format": "something-else"}')
    with pytest.raises(ValueError, match="unrecognized"):
        TieredPageStore(other, cpu_budget_bytes=8, disk_budget_bytes=1000)
    link = tmp_path / "link"
    link.symlink_to(foreign)
    with pytest.raises(ValueError, match="symbolic link"):
        TieredPageStore(link, cpu_budget_bytes=8, disk_budget_bytes=1000)
    with store_at(tmp_path):
        with pytest.raises(RuntimeError, match="already has a writer"):
            store_at(tmp_path)


def test_concurrent_put_read(tmp_path):
    # tests/test_storage.py:178-190
    with store_at(tmp_path, cpu=64) as store:

        def use(i):
            key, payload = f"model:layer:{i % 4}", bytes([i % 4]) * 4
            store.put(key, payload)
            return store.read(key)

        with ThreadPoolExecutor(max_workers=4) as pool:
            results = list(pool.map(use, range(40)))
        assert all(r == bytes([i % 4]) * 4 for i, r in enumerate(results))
        assert store.stats()["pages"] == 4


def test_partial_write_never_publishes(tmp_path, monkeypatch):
    # tests/test_storage.py:193-219: the second write call (the payload) fails
    with store_at(tmp_path, cpu=4) as store:
        store.put("a", b"aaaa")
        real_write, calls = os.write, []

        def flaky(fd, data):
            calls.append(len(data))
            if len(calls) == 2:
                raise OSError("injected interrupted payload write")
            return real_write(fd, data)

        with monkeypatch.context() as patch:
            patch.setattr(os, "write", flaky)
            with pytest.raises(OSError):
                store.submit_spill("a").result(timeout=5)
        assert store.read("a") == b"aaaa"
        stats = store.stats()
        assert stats["physical_host_write_bytes"] > 0 and stats["payload_write_bytes"] == 0
        assert stats["live_disk_bytes"] == 0 and stats["inflight_disk_reserved_bytes"] == 0
        assert not page_files(tmp_path)
        assert not list(store.root.glob(".pending-*"))


def test_retired_load_cannot_publish(tmp_path, monkeypatch):
    # tests/test_storage.py:222-256
    with store_at(tmp_path, cpu=4) as store:
        store.put("a", b"aaaa")
        store.evict()
        entered, release, closing = threading.Event(), threading.Event(), threading.Event()
        read, shutdown = store._read_disk, store._executor.shutdown

        def held(entry):
            entered.set()
            assert release.wait(5)
            return read(entry)

        def observed(*args, **kwargs):
            closing.set()
            return shutdown(*args, **kwargs)

        monkeypatch.setattr(store, "_read_disk", held)
        monkeypatch.setattr(store._executor, "shutdown", observed)
        loading = store.submit_load("a")
        assert entered.wait(5)
        with ThreadPoolExecutor(max_workers=1) as pool:
            closed = pool.submit(store.close, cancel_pending=True)
            try:
                assert closing.wait(5)
            finally:
                release.set()
            closed.result(timeout=5)
        with pytest.raises(StaleCompletionError):
            loading.result(timeout=5)
        assert store.stats()["live_cpu_bytes"] == 0
        assert store.stats()["inflight_cpu_reserved_bytes"] == 0
        with pytest.raises(RuntimeError, match="closed"):
            store.put("b", b"b")


def test_callbacks_see_settled_bookkeeping(tmp_path):
    # tests/test_storage.py:259-277
    with store_at(tmp_path, cpu=4) as store:
        store.put("a", b"aaaa")
        store.evict()
        seen, done = [], threading.Event()

        def observe(_):
            seen.append(store.stats())
            done.set()

        loading = store.submit_load("a")
        loading.add_done_callback(observe)
        loading.result(timeout=5)
        assert done.wait(5)
        assert seen[0]["live_cpu_bytes"] == 4
        assert seen[0]["inflight_cpu_reserved_bytes"] == 0 and seen[0]["inflight_pages"] == 0


def test_catalog_lookups_load_nothing(tmp_path, monkeypatch):
    # tests/test_storage.py:280-300
    with store_at(tmp_path) as store:
        store.put("model:layer:1", b"data", selected_count=2)
        store.evict()

        def forbidden(_):
            raise AssertionError("catalog lookup must not load a payload")

        monkeypatch.setattr(store, "_read_disk", forbidden)
        before = store.stats()
        assert store.contains("model:layer:1") and not store.contains("model:layer:2")
        assert store.keys("model:") == ("model:layer:1",) and store.keys("other:") == ()
        meta = store.metadata("model:layer:1")
        assert (meta["size"], meta["selected_count"], meta["pins"]) == (4, 2, 0)
        assert meta["resident"] is False and meta["backed"] is True
        assert isinstance(meta["generation"], str)
        assert store.stats() == before
        with pytest.raises(KeyError):
            store.metadata("missing")
        with pytest.raises(ValueError):
            store.keys(3)


def test_catalog_snapshots_are_copies_and_closed_store_refuses(tmp_path):
    # tests/test_storage.py:303-314
    with store_at(tmp_path) as store:
        store.put("layer:1", b"data")
        keys = store.keys()
        meta = store.metadata("layer:1")
        meta["size"] = meta["pins"] = 999
        assert store.metadata("layer:1")["size"] == 4
        with store.pin("layer:1"):
            assert store.metadata("layer:1")["pins"] == 1
        assert store.metadata("layer:1")["pins"] == 0
        store.put("layer:2", b"more")
        assert keys == ("layer:1",) and store.keys() == ("layer:1", "layer:2")
    for lookup in (lambda: store.contains("layer:1"), store.keys, lambda: store.metadata("layer:1")):
        with pytest.raises(RuntimeError, match="closed"):
            lookup()


def test_delete_removes_file_and_accounting(tmp_path):
    with store_at(tmp_path) as store:
        store.put("a", b"aaaa")
        store.submit_spill("a").result(timeout=5)
        store.put("b", b"bb")
        store.delete("a")
        store.delete("b")
        assert not page_files(tmp_path)
        stats = store.stats()
        assert stats["pages"] == 0 and stats["live_cpu_bytes"] == 0 and stats["live_disk_bytes"] == 0
        with pytest.raises(KeyError):
            store.delete("a")
