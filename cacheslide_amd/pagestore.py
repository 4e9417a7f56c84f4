"""A small page store for layer snapshots: one file per page, written through
to disk at ``put``, with a bounded RAM cache of recently used pages.

The layer-snapshot path (``cacheslide_amd.snapshot``) needs a store that
keeps immutable byte pages by key, reads them back (optionally on a worker
thread) and guarantees that a page is on disk once it has been published.
This store does exactly that and no more; it is not the reference's tiered
RAM/SSD engine (src/cacheslide_vllm/storage.py), whose dirty-page eviction,
spill scheduling and budget accounting are outside the reuse-attention path.

What is shared with the reference is the page file, so cache directories move
both ways (storage.py:158-236):

    <sha256(key) hex>.<generation>.page =
        compact key-sorted JSON header {"checksum", "format":
        "cacheslide-pages-v1", "generation", "key", "selected_count", "size"}
        + b"\\n" + payload            (checksum = sha256(payload) hex)

A store directory carries the marker file ``.cacheslide-store.json`` and is
opened by one writer at a time (an exclusive lock on ``.writer.lock``).
Pages are published by an atomic rename of a fully written, fsynced file.
"""

from __future__ import annotations

import fcntl
import hashlib
import json
import os
import threading
import uuid
from collections import OrderedDict
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path

from .errors import CacheCapacityError, CacheIntegrityError

PAGE_FORMAT = "cacheslide-pages-v1"
MARKER = ".cacheslide-store.json"
LOCK = ".writer.lock"
HEADER_LIMIT = 65536


def page_filename(key: str, generation: str) -> str:
    """A page file is named by the hash of its key, never by the key's text."""
    return hashlib.sha256(key.encode("utf-8")).hexdigest() + "." + generation + ".page"


def page_header(key: str, generation: str, payload: bytes, selected_count: int) -> bytes:
    fields = {"checksum": hashlib.sha256(payload).hexdigest(), "format": PAGE_FORMAT,
              "generation": generation, "key": key, "selected_count": selected_count,
              "size": len(payload)}
    line = json.dumps(fields, sort_keys=True, separators=(",", ":")).encode()
    if len(line) > HEADER_LIMIT:
        raise ValueError("page key is too long")
    return line + b"\n"


def parse_page(blob: bytes, *, expect_key: str | None = None) -> tuple[dict, bytes]:
    """Header fields and payload of a page file's bytes, checked against the
    header's size and checksum (and the expected key)."""
    end = blob.find(b"\n", 0, HEADER_LIMIT + 1)
    if end < 0:
        raise CacheIntegrityError("page header is missing or too long")
    try:
        head = json.loads(blob[:end])
    except ValueError as exc:
        raise CacheIntegrityError("page header is not JSON") from exc
    size, count = head.get("size") if isinstance(head, dict) else None, None
    if isinstance(head, dict):
        count = head.get("selected_count")
    if (not isinstance(head, dict) or head.get("format") != PAGE_FORMAT
            or type(size) is not int or size < 0 or type(count) is not int or count < 0
            or not isinstance(head.get("key"), str) or not isinstance(head.get("generation"), str)
            or not isinstance(head.get("checksum"), str)):
        raise CacheIntegrityError("invalid page metadata")
    payload = blob[end + 1:]
    if len(payload) != size:
        raise CacheIntegrityError("page size does not match metadata")
    if hashlib.sha256(payload).hexdigest() != head["checksum"]:
        raise CacheIntegrityError("page payload checksum mismatch")
    if expect_key is not None and head["key"] != expect_key:
        raise CacheIntegrityError("page key does not match its file")
    return head, payload


@dataclass
class _Page:
    generation: str
    checksum: str
    size: int
    selected_count: int
    path: Path
    file_bytes: int


class PageStore:
    """Immutable pages by key: on disk from ``put`` on, cached in RAM up to
    ``cpu_budget_bytes``; the directory holds at most ``disk_budget_bytes``."""

    def __init__(self, root: str | os.PathLike, *, cpu_budget_bytes: int, disk_budget_bytes: int,
                 workers: int = 4):
        for name, value in (("cpu_budget_bytes", cpu_budget_bytes), ("disk_budget_bytes", disk_budget_bytes)):
            if type(value) is not int or value < 0:
                raise ValueError(f"{name} must be a nonnegative integer")
        if type(workers) is not int or workers < 1:
            raise ValueError("workers must be a positive integer")
        self.root = Path(root)
        self.cpu_budget_bytes, self.disk_budget_bytes = cpu_budget_bytes, disk_budget_bytes
        self._lock = threading.Lock()
        self._pages: dict[str, _Page] = {}
        self._ram: OrderedDict[str, bytes] = OrderedDict()
        self._ram_bytes = 0
        self._disk_bytes = 0
        self._loads = 0
        self._closed = False
        self._open_directory()
        self._pool = ThreadPoolExecutor(max_workers=workers, thread_name_prefix="cacheslide-pages")

    # -- directory ---------------------------------------------------------------
    def _open_directory(self) -> None:
        self.root.mkdir(parents=True, exist_ok=True)
        if self.root.is_symlink() or not self.root.is_dir():
            raise ValueError("page store root must be a real directory")
        marker = self.root / MARKER
        entries = [p for p in self.root.iterdir() if p.name not in (MARKER, LOCK)]
        if marker.exists():
            try:
                ok = json.loads(marker.read_text()).get("format") == PAGE_FORMAT
            except (OSError, ValueError, AttributeError):
                ok = False
            if not ok:
                raise ValueError("page store marker names another format")
        elif entries:
            raise ValueError("page store root is not empty and was not created by a page store")
        else:
            marker.write_text(json.dumps({"format": PAGE_FORMAT}))
        self._lock_fd = os.open(self.root / LOCK, os.O_RDWR | os.O_CREAT, 0o600)
        try:
            fcntl.flock(self._lock_fd, fcntl.LOCK_EX | fcntl.LOCK_NB)
        except OSError as exc:
            os.close(self._lock_fd)
            raise RuntimeError("another writer holds this page store") from exc
        for path in sorted(self.root.glob("*.page")):
            self._adopt(path)

    def _adopt(self, path: Path) -> None:
        """Index a page file left by an earlier writer; the payload is checked when read."""
        with open(path, "rb") as stream:
            line = stream.readline(HEADER_LIMIT + 2)
        try:
            head = json.loads(line)
            key, generation = head["key"], head["generation"]
            size, count, checksum = head["size"], head["selected_count"], head["checksum"]
        except (ValueError, KeyError, TypeError) as exc:
            raise CacheIntegrityError(f"cannot read cache page: {path.name}") from exc
        if (head.get("format") != PAGE_FORMAT or path.name != page_filename(key, generation)
                or type(size) is not int or path.stat().st_size != len(line) + size):
            raise CacheIntegrityError(f"cannot read cache page: {path.name}")
        if key in self._pages:
            raise CacheIntegrityError(f"two generations of one page: {path.name}")
        self._pages[key] = _Page(generation, checksum, size, count, path, len(line) + size)
        self._disk_bytes += len(line) + size

    def _check_open(self) -> None:
        if self._closed:
            raise RuntimeError("page store is closed")

    # -- RAM cache -------------------------------------------------------------------
    def _cache(self, key: str, payload: bytes) -> None:
        """Keep a verified payload resident, least recently used first out."""
        if len(payload) > self.cpu_budget_bytes:
            return
        if key in self._ram:
            self._ram.move_to_end(key)
            return
        self._ram[key] = payload
        self._ram_bytes += len(payload)
        while self._ram_bytes > self.cpu_budget_bytes:
            _, old = self._ram.popitem(last=False)
            self._ram_bytes -= len(old)

    # -- pages -------------------------------------------------------------------------
    def put(self, key: str, payload: bytes, selected_count: int = 0) -> None:
        """Publish an immutable page (on disk when this returns).  Putting the
        same bytes again is a no-op; different bytes under a key are refused."""
        if not isinstance(key, str) or not key:
            raise ValueError("page key must be a non-empty string")
        if type(selected_count) is not int or selected_count < 0:
            raise ValueError("selected_count must be a nonnegative integer")
        payload = bytes(payload)
        checksum = hashlib.sha256(payload).hexdigest()
        with self._lock:
            self._check_open()
            page = self._pages.get(key)
            if page is not None:
                if page.checksum != checksum or page.size != len(payload):
                    raise ValueError("pages are immutable: the key holds different bytes")
                if key in self._ram:
                    self._ram.move_to_end(key)
                return
        generation = uuid.uuid4().hex
        header = page_header(key, generation, payload, selected_count)
        file_bytes = len(header) + len(payload)
        with self._lock:
            if self._disk_bytes + file_bytes > self.disk_budget_bytes:
                raise CacheCapacityError("page store disk budget exhausted")
            self._disk_bytes += file_bytes      # reserved while the file is written
        path = self.root / page_filename(key, generation)
        pending = self.root / f".pending-{generation}"
        try:
            fd = os.open(pending, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o600)
            with os.fdopen(fd, "wb") as stream:
                stream.write(header)
                stream.write(payload)
                stream.flush()
                os.fsync(stream.fileno())
            os.replace(pending, path)
        except BaseException:
            with self._lock:
                self._disk_bytes -= file_bytes
            pending.unlink(missing_ok=True)
            raise
        with self._lock:
            winner = self._pages.get(key)
            if winner is None and not self._closed:
                self._pages[key] = _Page(generation, checksum, len(payload), selected_count, path, file_bytes)
                self._cache(key, payload)
                return
            # a concurrent put of the same key published first (or the store
            # closed meanwhile): this generation is withdrawn
            self._disk_bytes -= file_bytes
        path.unlink(missing_ok=True)
        if winner is None:
            raise RuntimeError("page store is closed")
        if winner.checksum != checksum or winner.size != len(payload):
            raise ValueError("pages are immutable: the key holds different bytes")

    def read(self, key: str) -> bytes:
        """The page's bytes, from RAM or from its file; either way the payload's
        sha256 is checked against the page record first (a resident payload
        too, as storage.py:453-460 re-verifies it on every load)."""
        with self._lock:
            self._check_open()
            page = self._pages.get(key)
            if page is None:
                raise KeyError(key)
            hit = self._ram.get(key)
            if hit is not None:
                self._ram.move_to_end(key)
        if hit is not None:
            if len(hit) != page.size or hashlib.sha256(hit).hexdigest() != page.checksum:
                raise CacheIntegrityError("resident page checksum mismatch")
            return hit
        with open(page.path, "rb") as stream:
            blob = stream.read()
        head, payload = parse_page(blob, expect_key=key)
        if head["generation"] != page.generation:
            raise CacheIntegrityError("page generation changed under the store")
        with self._lock:
            if self._pages.get(key) is page:
                self._cache(key, payload)
        return payload

    def submit_load(self, key: str) -> Future:
        """``read`` on a worker thread."""
        with self._lock:
            self._check_open()
            if key not in self._pages:
                raise KeyError(key)
            self._loads += 1
        future = self._pool.submit(self.read, key)
        future.add_done_callback(self._load_done)
        return future

    def _load_done(self, _future: Future) -> None:
        with self._lock:
            self._loads -= 1

    def submit_spill(self, key: str) -> Future:
        """Pages are written through at ``put``: the spill has already happened."""
        with self._lock:
            self._check_open()
            if key not in self._pages:
                raise KeyError(key)
        done: Future = Future()
        done.set_result(None)
        return done

    def contains(self, key: str) -> bool:
        with self._lock:
            return key in self._pages

    def keys(self, prefix: str = "") -> tuple[str, ...]:
        with self._lock:
            return tuple(sorted(k for k in self._pages if k.startswith(prefix)))

    def metadata(self, key: str) -> dict[str, int | str | bool]:
        with self._lock:
            page = self._pages.get(key)
            if page is None:
                raise KeyError(key)
            return {"size": page.size, "selected_count": page.selected_count,
                    "generation": page.generation, "backed": True, "resident": key in self._ram}

    def delete(self, key: str) -> None:
        with self._lock:
            self._check_open()
            page = self._pages.pop(key, None)
            if page is None:
                raise KeyError(key)
            payload = self._ram.pop(key, None)
            if payload is not None:
                self._ram_bytes -= len(payload)
            self._disk_bytes -= page.file_bytes
        page.path.unlink(missing_ok=True)

    def stats(self) -> dict[str, int]:
        with self._lock:
            return {"pages": len(self._pages), "resident_pages": len(self._ram),
                    "resident_bytes": self._ram_bytes, "disk_bytes": self._disk_bytes,
                    "cpu_budget_bytes": self.cpu_budget_bytes,
                    "disk_budget_bytes": self.disk_budget_bytes, "inflight_loads": self._loads}

    def close(self) -> None:
        with self._lock:
            if self._closed:
                return
            self._closed = True
        self._pool.shutdown(wait=True)
        with self._lock:
            self._ram.clear()
            self._ram_bytes = 0
        fcntl.flock(self._lock_fd, fcntl.LOCK_UN)
        os.close(self._lock_fd)

    def __enter__(self) -> PageStore:
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()
