"""Random operation sequences against TieredPageStore on the CPU (storage.py:47-611).

A model keeps what the store must hold: every page put is readable with its
bytes; resident bytes never exceed the RAM budget and equal the sum of the
resident pages; disk bytes equal the sum of the published page files; no
temporary file survives an operation; a reopened store sees exactly the
published pages.  Capacity errors are allowed (the caller falls back): a put
that fails leaves the catalog as it was, and an eviction that cannot free
enough still publishes what it dropped, as storage.py:311-324 does.
"""

from __future__ import annotations

import shutil
import tempfile
from pathlib import Path

import hypothesis.strategies as st
from hypothesis import HealthCheck, settings
from hypothesis.stateful import RuleBasedStateMachine, invariant, rule

from cacheslide_amd.storage import CacheCapacityError, TieredPageStore

KEYS = st.sampled_from([f"model:layer:{i}" for i in range(6)])
PAYLOADS = st.binary(min_size=0, max_size=24)


class StoreMachine(RuleBasedStateMachine):
    def __init__(self):
        super().__init__()
        self.tmp = Path(tempfile.mkdtemp(prefix="store-"))
        self.cpu, self.disk = 48, 400
        self.store = self.open()
        self.pages: dict[str, tuple[bytes, int]] = {}   # key -> (payload, selected_count)

    def open(self):
        return TieredPageStore(self.tmp / "pages", cpu_budget_bytes=self.cpu, disk_budget_bytes=self.disk)

    def teardown(self):
        self.store.close()
        shutil.rmtree(self.tmp, ignore_errors=True)

    def snapshot(self):
        return self.store.stats()

    @rule(key=KEYS, payload=PAYLOADS, count=st.integers(0, 3))
    def put(self, key, payload, count):
        before = self.snapshot()
        if key in self.pages:
            same = self.pages[key] == (payload, count)
            try:
                self.store.put(key, payload, count)
                assert same
            except ValueError:
                assert not same
            except CacheCapacityError:
                pass
            return
        try:
            self.store.put(key, payload, count)
        except CacheCapacityError:
            after = self.snapshot()
            assert after["pages"] == before["pages"]
            assert not self.store.contains(key)
            return
        self.pages[key] = (payload, count)

    @rule(key=KEYS)
    def read(self, key):
        if key not in self.pages:
            return
        try:
            assert self.store.read(key) == self.pages[key][0]
        except CacheCapacityError:
            pass

    @rule()
    def evict_one(self):
        try:
            (key,) = self.store.evict()
        except CacheCapacityError:
            return
        meta = self.store.metadata(key)
        assert key in self.pages and not meta["resident"] and meta["backed"]

    @rule(need=st.integers(1, 60))
    def evict_bytes(self, need):
        # an impossible request still publishes and drops what it could (storage.py:311-324)
        try:
            for key in self.store.evict(need):
                assert self.store.metadata(key)["backed"]
        except CacheCapacityError:
            pass

    @rule(key=KEYS)
    def spill(self, key):
        if key not in self.pages:
            return
        try:
            self.store.submit_spill(key).result(timeout=5)
            assert self.store.metadata(key)["backed"]
        except CacheCapacityError:
            pass

    @rule(key=KEYS)
    def delete(self, key):
        if key not in self.pages:
            return
        self.store.delete(key)
        del self.pages[key]

    @rule()
    def reopen(self):
        """Close and reopen: only published pages survive, unpublished RAM pages go."""
        published = {k for k in self.pages if self.store.metadata(k)["backed"]}
        self.store.close()
        self.store = self.open()
        self.pages = {k: v for k, v in self.pages.items() if k in published}
        assert set(self.store.keys()) == set(self.pages)
        for key in self.pages:
            assert not self.store.metadata(key)["resident"]

    @invariant()
    def consistent(self):
        stats = self.store.stats()
        assert stats["pages"] == len(self.pages)
        assert set(self.store.keys()) == set(self.pages)
        resident = 0
        disk = 0
        for key, (payload, count) in self.pages.items():
            meta = self.store.metadata(key)
            assert meta["size"] == len(payload) and meta["selected_count"] == count
            if meta["resident"]:
                resident += len(payload)
            assert meta["resident"] or meta["backed"]        # never lost
        for path in (self.tmp / "pages").glob("*.page"):
            disk += path.stat().st_size
        assert stats["live_cpu_bytes"] == resident <= self.cpu
        assert stats["live_disk_bytes"] == disk <= self.disk
        assert stats["inflight_cpu_reserved_bytes"] == 0 and stats["inflight_disk_reserved_bytes"] == 0
        assert not list((self.tmp / "pages").glob(".pending-*"))


TestStoreMachine = StoreMachine.TestCase
TestStoreMachine.settings = settings(max_examples=60, stateful_step_count=30, deadline=None,
                                     suppress_health_check=[HealthCheck.too_slow])
