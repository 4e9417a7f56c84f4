"""The layer-snapshot page store: page file format, write-through publication,
RAM cache bounds, integrity checks and the single-writer rule (CPU only).

The page file is the reference's ``cacheslide-pages-v1`` format
(src/cacheslide_vllm/storage.py:158-236); a page written here by hand from
that format is adopted, and the store's own files are checked byte for byte
against it.
"""

from __future__ import annotations

import hashlib
import json

import pytest

from cacheslide_amd.errors import CacheCapacityError, CacheIntegrityError
from cacheslide_amd.pagestore import MARKER, PAGE_FORMAT, PageStore, page_filename

SHA_DATA = "3a6eb0790f39ac87c94f3856b2dd2c5d110e6811602261a9a923d3bb23adc8b7"   # sha256(b"data")


def store_at(path, cpu=1 << 20, disk=1 << 22):
    return PageStore(path, cpu_budget_bytes=cpu, disk_budget_bytes=disk)


def test_page_file_format_known_answer(tmp_path):
    assert hashlib.sha256(b"data").hexdigest() == SHA_DATA
    with store_at(tmp_path / "s") as store:
        store.put("layer/0/kv", b"data", selected_count=3)
        meta = store.metadata("layer/0/kv")
        name = page_filename("layer/0/kv", meta["generation"])
        assert name.startswith(hashlib.sha256(b"layer/0/kv").hexdigest() + ".")
        blob = (tmp_path / "s" / name).read_bytes()
    header = (
        '{"checksum":"' + SHA_DATA + '","format":"cacheslide-pages-v1","generation":"'
        + meta["generation"] + '","key":"layer/0/kv","selected_count":3,"size":4}\n'
    ).encode()
    assert blob == header + b"data"
    assert json.loads((tmp_path / "s" / MARKER).read_text()) == {"format": PAGE_FORMAT}


def test_hand_written_page_is_adopted(tmp_path):
    root = tmp_path / "s"
    root.mkdir()
    (root / MARKER).write_text(json.dumps({"format": PAGE_FORMAT}))
    head = {"checksum": SHA_DATA, "format": PAGE_FORMAT, "generation": "g1", "key": "k", "selected_count": 0,
            "size": 4}
    line = json.dumps(head, sort_keys=True, separators=(",", ":")).encode() + b"\n"
    (root / page_filename("k", "g1")).write_bytes(line + b"data")
    with store_at(root) as store:
        assert store.keys() == ("k",)
        assert store.read("k") == b"data"
        assert store.metadata("k")["resident"]


def test_round_trip_reopen_and_delete(tmp_path):
    root = tmp_path / "s"
    with store_at(root) as store:
        for i in range(5):
            store.put(f"p/{i}", bytes([i]) * (100 + i))
        assert store.keys("p/") == tuple(f"p/{i}" for i in range(5))
        assert store.submit_spill("p/3").result() is None
        futures = [store.submit_load(f"p/{i}") for i in range(5)]
        assert [f.result() for f in futures] == [bytes([i]) * (100 + i) for i in range(5)]
        store.delete("p/1")
        assert not store.contains("p/1")
        with pytest.raises(KeyError):
            store.read("p/1")
        assert store.stats()["inflight_loads"] == 0
    with store_at(root) as store:                    # the pages outlive the process's store
        assert store.keys() == ("p/0", "p/2", "p/3", "p/4")
        assert store.read("p/4") == bytes([4]) * 104
        assert not store.metadata("p/0")["resident"] or store.stats()["resident_pages"] >= 1
    assert len(list(root.glob("*.page"))) == 4


def test_pages_are_immutable(tmp_path):
    with store_at(tmp_path / "s") as store:
        store.put("k", b"abc")
        store.put("k", b"abc")                       # the same bytes again: no-op
        with pytest.raises(ValueError, match="immutable"):
            store.put("k", b"abd")
        assert store.read("k") == b"abc"
        assert len(list((tmp_path / "s").glob("*.page"))) == 1


def test_corrupt_payload_is_detected_on_read(tmp_path):
    root = tmp_path / "s"
    with store_at(root) as store:
        store.put("k", b"payload-bytes")
    path = next(root.glob("*.page"))
    blob = bytearray(path.read_bytes())
    blob[-1] ^= 1
    path.write_bytes(bytes(blob))
    with store_at(root) as store:
        with pytest.raises(CacheIntegrityError, match="checksum"):
            store.read("k")
        with pytest.raises(CacheIntegrityError):
            store.submit_load("k").result()


def test_truncated_page_is_refused_at_open(tmp_path):
    root = tmp_path / "s"
    with store_at(root) as store:
        store.put("k", b"payload-bytes")
    path = next(root.glob("*.page"))
    path.write_bytes(path.read_bytes()[:-3])
    with pytest.raises(CacheIntegrityError):
        store_at(root)


def test_budgets(tmp_path):
    with store_at(tmp_path / "s", cpu=250, disk=1100) as store:
        store.put("a", b"a" * 100)
        store.put("b", b"b" * 100)
        store.put("c", b"c" * 100)                   # RAM holds two of three
        stats = store.stats()
        assert stats["resident_bytes"] <= 250 and stats["resident_pages"] == 2
        assert not store.metadata("a")["resident"]   # least recently used left first
        assert store.read("a") == b"a" * 100         # from its file
        with pytest.raises(CacheCapacityError):
            store.put("d", b"d" * 400)               # headers count against the disk budget
        assert not store.contains("d")
        assert len(list((tmp_path / "s").glob("*"))) == 3 + 2   # pages + marker + lock


def test_single_writer_and_foreign_directories(tmp_path):
    root = tmp_path / "s"
    first = store_at(root)
    with pytest.raises(RuntimeError, match="another writer"):
        store_at(root)
    first.close()
    store_at(root).close()                           # the lock is released on close
    foreign = tmp_path / "f"
    foreign.mkdir()
    (foreign / "notes.txt").write_text("x")
    with pytest.raises(ValueError, match="not empty"):
        store_at(foreign)
    closed = store_at(tmp_path / "c")
    closed.close()
    with pytest.raises(RuntimeError, match="closed"):
        closed.put("k", b"x")


def test_resident_page_is_verified_on_read(tmp_path):
    """A RAM-resident payload is checked against the page's sha256 on every
    read, as storage.py:453-460 re-verifies resident pages on load."""
    with store_at(tmp_path / "s") as store:
        store.put("k", b"data")
        assert store.metadata("k")["resident"]
        assert store.read("k") == b"data"
        store._ram["k"] = b"dat4"          # the resident copy goes bad in memory
        with pytest.raises(CacheIntegrityError, match="resident page checksum"):
            store.read("k")


def test_concurrent_puts_of_one_key_publish_one_generation(tmp_path, monkeypatch):
    """A second put of the same key that publishes while the first is still
    writing its file wins; the first withdraws its file and, holding
    different bytes, is refused.  The directory then reopens with one page."""
    import os

    from cacheslide_amd import pagestore

    real_fsync = os.fsync
    nested = {"done": False}
    store = store_at(tmp_path / "s")

    def racing_fsync(fd):
        real_fsync(fd)
        if not nested["done"]:
            nested["done"] = True
            store.put("k", b"second")       # publishes while the first put is mid-write

    monkeypatch.setattr(pagestore.os, "fsync", racing_fsync)
    with pytest.raises(ValueError, match="immutable"):
        store.put("k", b"first!")
    monkeypatch.setattr(pagestore.os, "fsync", real_fsync)
    assert store.read("k") == b"second"
    disk = store.stats()["disk_bytes"]
    files = [p for p in (tmp_path / "s").iterdir() if p.name.endswith(".page")]
    assert len(files) == 1 and disk == files[0].stat().st_size
    # same bytes racing: the loser returns quietly
    nested["done"] = False

    def same_fsync(fd):
        real_fsync(fd)
        if not nested["done"]:
            nested["done"] = True
            store.put("j", b"same")

    monkeypatch.setattr(pagestore.os, "fsync", same_fsync)
    store.put("j", b"same")
    monkeypatch.setattr(pagestore.os, "fsync", real_fsync)
    store.close()
    with store_at(tmp_path / "s") as again:
        assert again.read("k") == b"second" and again.read("j") == b"same"
        assert again.stats()["pages"] == 2
