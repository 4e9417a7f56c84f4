"""Exception types and the RAM/SSD page store of layer snapshots.

Mirrors src/cacheslide_vllm/storage.py.  ``TieredPageStore`` keeps immutable
byte pages under a RAM budget, spills them to checksummed page files under a
disk budget and loads them back asynchronously.  The on-disk format is the
reference's ``cacheslide-pages-v1`` (storage.py:176-190), so directories are
interchangeable between the two implementations:

    <sha256(key) hex>.<generation>.page =
        json.dumps({"checksum", "format", "generation", "key",
                    "selected_count", "size"}, sort_keys, compact) + b"\\n"
        + payload                      (checksum = sha256(payload) hex)

plus ``.cacheslide-store.json`` ({"format": "cacheslide-pages-v1"}) and the
single-writer lock ``.writer.lock``.

The store moves bytes only; snapshot pages reach HBM through
``cacheslide_amd.snapshot`` (pinned staging, asynchronous DMA on an upload
stream, device-side checks).
"""

from __future__ import annotations

import hashlib
import json
import os
import threading
import uuid
from collections.abc import Iterator
from concurrent.futures import Future, ThreadPoolExecutor
from contextlib import contextmanager
from dataclasses import dataclass
from pathlib import Path

PAGE_FORMAT = "cacheslide-pages-v1"
_MARKER = ".cacheslide-store.json"
_LOCK = ".writer.lock"
_PENDING = ".pending-"
_MAX_HEADER = 65536


class CacheCapacityError(RuntimeError):
    """Not enough slots or capacity to perform an operation safely (storage.py:21-22)."""


class CacheIntegrityError(RuntimeError):
    """A persisted page failed its identity or checksum check (storage.py:25-26)."""


class StaleCompletionError(RuntimeError):
    """An asynchronous completion belongs to a retired map or generation (storage.py:29-30)."""


def _sha256(data) -> str:
    return hashlib.sha256(data).hexdigest()


def page_filename(key: str, generation: str) -> str:
    """File name of a page: the key's hash, never its text (storage.py:158-162)."""
    return _sha256(key.encode("utf-8")) + "." + generation + ".page"


def encode_page_header(key: str, generation: str, checksum: str, size: int,
                       selected_count: int) -> bytes:
    """The header line of a page file (storage.py:176-190)."""
    line = json.dumps(
        {"format": PAGE_FORMAT, "key": key, "generation": generation, "checksum": checksum,
         "size": size, "selected_count": selected_count},
        sort_keys=True, separators=(",", ":"),
    ).encode()
    if len(line) > _MAX_HEADER:
        raise ValueError("page key is too long")
    return line + b"\n"


@dataclass
class _Entry:
    """Catalog entry of one immutable page (storage.py:33-44)."""

    key: str
    generation: str
    checksum: str
    size: int
    selected_count: int
    last_access: int
    payload: bytes | None = None  # resident copy
    path: Path | None = None      # published page file
    disk_size: int = 0
    pins: int = 0
    inflight: int = 0

    def eviction_rank(self) -> tuple:
        # clean pages first, then dirty pages by descending selected count,
        # then least recently used (storage.py:293-309)
        dirty = self.selected_count > 0
        return (dirty, -self.selected_count, self.last_access, self.key)


class TieredPageStore:
    """Immutable pages with bounded resident bytes and atomic SSD publication.

    Same contract as storage.py:47-611: ``root`` is an empty directory or one
    this class created, owned by the current user, with a single writer.
    Capacity exhaustion raises ``CacheCapacityError`` so callers can fall back
    to recomputation; disk-only pages are never deleted automatically.
    """

    _FORMAT = PAGE_FORMAT
    _MAX_HEADER = _MAX_HEADER

    def __init__(self, root: str | Path, *, cpu_budget_bytes: int, disk_budget_bytes: int,
                 max_workers: int = 2):
        if cpu_budget_bytes < 0 or disk_budget_bytes < 0 or max_workers < 1:
            raise ValueError("budgets must be nonnegative and max_workers positive")
        self.root = Path(root).absolute()
        self._claim_directory()
        self._lock_path = self.root / _LOCK
        try:
            self._lock_fd = os.open(self._lock_path, os.O_CREAT | os.O_EXCL | os.O_WRONLY, 0o600)
        except FileExistsError as exc:
            raise RuntimeError(
                "cache directory already has a writer; stale locks require explicit cleanup"
            ) from exc
        self.cpu_budget_bytes = cpu_budget_bytes
        self.disk_budget_bytes = disk_budget_bytes
        self._mutex = threading.RLock()
        self._pages: dict[str, _Entry] = {}
        self._cpu_bytes = self._disk_bytes = 0
        self._cpu_reserved = self._disk_reserved = 0
        self._payload_write_bytes = self._physical_host_write_bytes = 0
        self._tick = 0
        self._epoch = 0
        self._closed = self._closing = False
        self._loads: dict[str, Future] = {}
        self._spills: dict[str, Future] = {}
        self._executor = ThreadPoolExecutor(max_workers=max_workers, thread_name_prefix="cacheslide-io")
        try:
            self._scan_pages()
        except BaseException:
            self._executor.shutdown(wait=True)
            os.close(self._lock_fd)
            self._lock_path.unlink()
            raise

    # ------------------------------------------------------------ directory
    def _claim_directory(self) -> None:
        """storage.py:68-88: refuse links, foreign owners and unrelated content."""
        if self.root.is_symlink():
            raise ValueError("cache root must not be a symbolic link")
        self.root.mkdir(parents=True, exist_ok=True)
        if not self.root.is_dir():
            raise ValueError("cache root must be a directory")
        if hasattr(os, "getuid") and self.root.stat().st_uid != os.getuid():
            raise ValueError("cache root must be owned by the current user")
        marker = self.root / _MARKER
        if marker.exists():
            if marker.is_symlink() or json.loads(marker.read_text()).get("format") != PAGE_FORMAT:
                raise ValueError("unrecognized cache directory")
            return
        if any(self.root.iterdir()):
            raise ValueError("refusing to claim a nonempty cache directory")
        with marker.open("x", encoding="utf-8") as stream:
            json.dump({"format": PAGE_FORMAT}, stream)

    def _scan_pages(self) -> None:
        """Rebuild the catalog from published page files (storage.py:123-156)."""
        if any(self.root.glob(_PENDING + "*")):
            raise CacheIntegrityError("unfinished cache writes require explicit recovery")
        for path in sorted(self.root.glob("*.page")):
            if path.is_symlink():
                raise CacheIntegrityError("symbolic links are not cache pages")
            header, _ = self._decode_file(path, materialize=False)
            key = header["key"]
            if path.name != page_filename(key, header["generation"]):
                raise CacheIntegrityError("page filename does not match its identity")
            if key in self._pages:
                raise CacheIntegrityError("duplicate immutable page identity")
            entry = _Entry(key, header["generation"], header["checksum"], header["size"],
                           header["selected_count"], self._next_tick(), path=path,
                           disk_size=path.stat().st_size)
            self._pages[key] = entry
            self._disk_bytes += entry.disk_size
        if self._disk_bytes > self.disk_budget_bytes:
            raise CacheCapacityError("existing disk pages exceed the disk budget")

    # --------------------------------------------------------------- helpers
    @staticmethod
    def _filename(key: str, generation: str) -> str:
        return page_filename(key, generation)

    def _next_tick(self) -> int:
        self._tick += 1
        return self._tick

    def _check_open(self) -> None:
        if self._closed or self._closing:
            raise RuntimeError("page store is closed")

    @staticmethod
    def _verify(entry: _Entry, payload) -> None:
        if len(payload) != entry.size or _sha256(payload) != entry.checksum:
            raise CacheIntegrityError("page payload checksum mismatch")

    def _encode_header(self, entry: _Entry) -> bytes:
        return encode_page_header(entry.key, entry.generation, entry.checksum, entry.size,
                                  entry.selected_count)

    def _decode_file(self, path: Path, *, materialize: bool = True) -> tuple[dict, bytes | None]:
        """Read and check one page file (storage.py:192-235).

        The header is bounded, its fields typed, the size bounded by the disk
        budget and equal to the file's payload length, and the checksum is
        recomputed (streamed when the payload is not wanted).
        """
        flags = os.O_RDONLY | getattr(os, "O_NOFOLLOW", 0)
        try:
            with os.fdopen(os.open(path, flags), "rb") as stream:
                line = stream.readline(_MAX_HEADER + 2)
                if len(line) > _MAX_HEADER + 1 or not line.endswith(b"\n"):
                    raise CacheIntegrityError("invalid page header")
                header = json.loads(line)
                size = header.get("size")
                count = header.get("selected_count")
                if (header.get("format") != PAGE_FORMAT or type(size) is not int or size < 0
                        or type(count) is not int or count < 0
                        or not isinstance(header.get("key"), str)
                        or not isinstance(header.get("generation"), str)):
                    raise CacheIntegrityError("invalid page metadata")
                # a corrupted size cannot cause an unbounded allocation
                if size > self.disk_budget_bytes or stream.seek(0, os.SEEK_END) != len(line) + size:
                    raise CacheIntegrityError("page size does not match metadata")
                stream.seek(len(line))
                payload = None
                if materialize:
                    payload = stream.read(size)
                    checksum = _sha256(payload)
                else:
                    digest = hashlib.sha256()
                    chunk = min(65536, max(1, self.cpu_budget_bytes))
                    while block := stream.read(chunk):
                        digest.update(block)
                    checksum = digest.hexdigest()
                if checksum != header.get("checksum"):
                    raise CacheIntegrityError("persisted page checksum mismatch")
                return header, payload
        except (OSError, ValueError, TypeError, KeyError) as exc:
            raise CacheIntegrityError(f"cannot read cache page: {path.name}") from exc

    def _read_disk(self, entry: _Entry) -> bytes:
        if entry.path is None:
            raise CacheIntegrityError("page has no backing copy")
        header, payload = self._decode_file(entry.path)
        if header["key"] != entry.key or header["generation"] != entry.generation:
            raise CacheIntegrityError("persisted page identity mismatch")
        self._verify(entry, payload)
        return payload

    # ------------------------------------------------------------------ put
    def put(self, key: str, payload: bytes, selected_count: int = 0) -> None:
        """Add an immutable page; an identical re-put only refreshes its age (storage.py:247-290)."""
        if not isinstance(key, str) or not key:
            raise ValueError("key must be a nonempty namespaced string")
        if not isinstance(payload, bytes) or type(selected_count) is not int or selected_count < 0:
            raise ValueError("payload must be bytes and selected_count nonnegative")
        with self._mutex:
            self._check_open()
            existing = self._pages.get(key)
            if existing is not None:
                self._confirm_same(existing, payload, selected_count)
                existing.last_access = self._next_tick()
                return
            if len(payload) > self.cpu_budget_bytes:
                raise CacheCapacityError("page exceeds the CPU budget")
            self._make_cpu_space(len(payload))
            entry = _Entry(key, uuid.uuid4().hex, _sha256(payload), len(payload), selected_count,
                           self._next_tick(), payload=payload)
            self._encode_header(entry)  # the header must fit before the page is committed
            self._pages[key] = entry
            self._cpu_bytes += len(payload)

    def _confirm_same(self, entry: _Entry, payload: bytes, selected_count: int) -> None:
        if (len(payload) != entry.size or _sha256(payload) != entry.checksum
                or entry.selected_count != selected_count):
            raise ValueError("immutable page key already exists with different data")
        if entry.payload is not None:
            self._verify(entry, entry.payload)
            if entry.payload != payload:
                raise ValueError("immutable page key collision")
        else:
            # the published copy is checked by streaming, without a second resident payload
            self._spill_sync(entry)

    # ------------------------------------------------------------- eviction
    def _candidates(self, exclude: str | None = None) -> list[_Entry]:
        eligible = [e for e in self._pages.values()
                    if e.payload is not None and not e.pins and not e.inflight and e.key != exclude]
        return sorted(eligible, key=_Entry.eviction_rank)

    def _fits(self, needed: int) -> bool:
        return self._cpu_bytes + self._cpu_reserved + needed <= self.cpu_budget_bytes

    def _make_cpu_space(self, needed: int, exclude: str | None = None) -> list[str]:
        """Spill-then-drop resident pages in eviction order until ``needed`` fits (storage.py:311-324)."""
        evicted = []
        for entry in self._candidates(exclude):
            if self._fits(needed):
                break
            self._drop_resident(entry)
            evicted.append(entry.key)
        if not self._fits(needed):
            raise CacheCapacityError("CPU capacity unavailable: pages are pinned or in flight")
        return evicted

    def _drop_resident(self, entry: _Entry) -> None:
        # publication precedes removal of the resident copy, clean pages included
        self._spill_sync(entry)
        self._cpu_bytes -= entry.size
        entry.payload = None

    def evict(self, required_bytes: int = 0) -> list[str]:
        """Ensure ``required_bytes`` free RAM; zero evicts exactly one page (storage.py:400-415)."""
        if required_bytes < 0:
            raise ValueError("required_bytes must be nonnegative")
        with self._mutex:
            self._check_open()
            if required_bytes:
                return self._make_cpu_space(required_bytes)
            candidates = self._candidates()
            if not candidates:
                raise CacheCapacityError("no unpinned resident page can be evicted")
            self._drop_resident(candidates[0])
            return [candidates[0].key]

    # ---------------------------------------------------------- publication
    def _write_page(self, entry: _Entry, header: bytes, payload: bytes) -> Path:
        """Write, fsync, re-check and atomically rename one page file (storage.py:326-368).

        Header and payload go out in separate writes, so a failure between them
        leaves only the temporary file, which is removed.
        """
        destination = self.root / page_filename(entry.key, entry.generation)
        temporary = self.root / (_PENDING + uuid.uuid4().hex)
        fd = os.open(temporary, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o600)
        published = False
        try:
            for part in (header, payload):
                remaining = memoryview(part)
                while remaining:
                    written = os.write(fd, remaining)
                    if written <= 0:
                        raise OSError("short cache page write")
                    with self._mutex:
                        self._physical_host_write_bytes += written
                    remaining = remaining[written:]
            os.fsync(fd)
            os.close(fd)
            fd = -1
            check, _ = self._decode_file(temporary, materialize=False)
            if check["generation"] != entry.generation or check["checksum"] != entry.checksum:
                raise CacheIntegrityError("temporary page generation mismatch")
            os.replace(temporary, destination)
            published = True
            directory = os.open(self.root, os.O_RDONLY)
            try:
                os.fsync(directory)
            finally:
                os.close(directory)
            return destination
        except BaseException:
            if published:
                destination.unlink(missing_ok=True)
            raise
        finally:
            if fd >= 0:
                os.close(fd)
            if temporary.exists():
                temporary.unlink()

    def _spill_sync(self, entry: _Entry) -> None:
        """Publish a resident page, or confirm its published copy (storage.py:370-398)."""
        if entry.path is not None:
            # never drop the only valid copy when the backing file went bad
            check, _ = self._decode_file(entry.path, materialize=False)
            if (check["key"] != entry.key or check["generation"] != entry.generation
                    or check["checksum"] != entry.checksum):
                raise CacheIntegrityError("persisted page identity mismatch")
            return
        if entry.payload is None:
            raise CacheIntegrityError("cannot spill a page without resident data")
        self._verify(entry, entry.payload)
        header = self._encode_header(entry)
        encoded = len(header) + entry.size
        if self._disk_bytes + self._disk_reserved + encoded > self.disk_budget_bytes:
            raise CacheCapacityError("disk capacity unavailable; resident page preserved")
        self._disk_reserved += encoded
        try:
            entry.path = self._write_page(entry, header, entry.payload)
            entry.disk_size = encoded
            self._disk_bytes += encoded
            self._payload_write_bytes += entry.size
        finally:
            self._disk_reserved -= encoded

    # -------------------------------------------------------------- lookups
    def read(self, key: str) -> bytes:
        return self.submit_load(key).result()

    def contains(self, key: str) -> bool:
        """Catalog lookup; no payload is loaded or touched."""
        with self._mutex:
            self._check_open()
            return key in self._pages

    def keys(self, prefix: str = "") -> tuple[str, ...]:
        """A sorted snapshot of the catalog's keys."""
        if not isinstance(prefix, str):
            raise ValueError("key prefix must be a string")
        with self._mutex:
            self._check_open()
            return tuple(sorted(k for k in self._pages if k.startswith(prefix)))

    def metadata(self, key: str) -> dict[str, int | str | bool]:
        """Scalar page metadata (a copy), without loading the payload."""
        with self._mutex:
            self._check_open()
            e = self._pages[key]
            return {"size": e.size, "selected_count": e.selected_count, "generation": e.generation,
                    "resident": e.payload is not None, "backed": e.path is not None, "pins": e.pins}

    # ---------------------------------------------------------------- async
    def _retired(self, entry: _Entry, epoch: int) -> bool:
        return self._closed or epoch != self._epoch or self._pages.get(entry.key) is not entry

    def submit_load(self, key: str) -> Future:
        """Future of the page's bytes (storage.py:439-494).

        A resident page is verified and returned at once; a disk page is read on
        the I/O pool against a RAM reservation, and concurrent loads of one key
        share a future.  A load that finishes after ``close(cancel_pending=True)``
        or a delete fails with ``StaleCompletionError``.  Bookkeeping is settled
        before the future completes, so callbacks see it finished.

        The checksum of a resident page is computed after the lock is released
        (the payload is an immutable ``bytes`` held by this call), so threads
        loading different pages hash them in parallel.
        """
        with self._mutex:
            self._check_open()
            entry = self._pages[key]
            entry.last_access = self._next_tick()
            resident = entry.payload
            if resident is None:
                return self._schedule_load(key, entry)
        self._verify(entry, resident)
        ready: Future = Future()
        ready.set_result(resident)
        return ready

    def _schedule_load(self, key: str, entry: _Entry) -> Future:
        """Start a disk read of ``entry``; the caller holds the lock."""
        if key in self._loads:
            return self._loads[key]
        if entry.size > self.cpu_budget_bytes:
            raise CacheCapacityError("page exceeds the CPU budget")
        self._make_cpu_space(entry.size, exclude=key)
        self._cpu_reserved += entry.size
        entry.inflight += 1
        epoch = self._epoch
        result: Future = Future()
        result.set_running_or_notify_cancel()  # public cancel cannot stop the I/O
        self._loads[key] = result
        # scheduled under the lock, so close() cannot shut the pool down in between
        self._executor.submit(self._load_job, entry, epoch, result)
        return result

    def _load_job(self, entry: _Entry, epoch: int, result: Future) -> None:
        failure: BaseException | None = None
        payload = None
        try:
            payload = self._read_disk(entry)
        except BaseException as exc:
            failure = exc
        with self._mutex:
            if failure is None:
                if self._retired(entry, epoch):
                    failure = StaleCompletionError("page load completed for a retired generation")
                else:
                    entry.payload = payload
                    self._cpu_bytes += entry.size
            self._cpu_reserved -= entry.size
            entry.inflight -= 1
            self._loads.pop(entry.key, None)
        if failure is not None:
            result.set_exception(failure)
        else:
            result.set_result(payload)

    def submit_spill(self, key: str) -> Future:
        """Future of the page's publication on the I/O pool (storage.py:496-530)."""
        with self._mutex:
            self._check_open()
            entry = self._pages[key]
            if key in self._spills:
                return self._spills[key]
            result: Future = Future()
            result.set_running_or_notify_cancel()
            entry.inflight += 1
            epoch = self._epoch
            self._spills[key] = result
            self._executor.submit(self._spill_job, entry, epoch, result)
            return result

    def _spill_job(self, entry: _Entry, epoch: int, result: Future) -> None:
        failure: BaseException | None = None
        try:
            with self._mutex:
                if self._retired(entry, epoch):
                    raise StaleCompletionError("page spill belongs to a retired generation")
                self._spill_sync(entry)
        except BaseException as exc:
            failure = exc
        finally:
            with self._mutex:
                entry.inflight -= 1
                self._spills.pop(entry.key, None)
        if failure is not None:
            result.set_exception(failure)
        else:
            result.set_result(None)

    @contextmanager
    def pin(self, key: str) -> Iterator[bytes]:
        """Hold a page resident while its bytes are in use (storage.py:532-542)."""
        with self._mutex:
            self._check_open()
            entry = self._pages[key]
            entry.pins += 1
        try:
            yield self.read(key)
        finally:
            with self._mutex:
                entry.pins -= 1

    def delete(self, key: str) -> None:
        """Remove one page owned by this store (storage.py:544-556)."""
        with self._mutex:
            self._check_open()
            entry = self._pages[key]
            if entry.pins or entry.inflight:
                raise CacheCapacityError("cannot delete a pinned or in-flight page")
            if entry.path is not None:
                entry.path.unlink()
                self._disk_bytes -= entry.disk_size
            if entry.payload is not None:
                self._cpu_bytes -= entry.size
            del self._pages[key]

    def stats(self) -> dict[str, int]:
        with self._mutex:
            pages = self._pages.values()
            return {
                "pages": len(self._pages),
                "live_cpu_bytes": self._cpu_bytes,
                "live_disk_bytes": self._disk_bytes,
                "inflight_cpu_reserved_bytes": self._cpu_reserved,
                "inflight_disk_reserved_bytes": self._disk_reserved,
                "payload_write_bytes": self._payload_write_bytes,
                "physical_host_write_bytes": self._physical_host_write_bytes,
                "pinned_pages": sum(e.pins > 0 for e in pages),
                "inflight_pages": sum(e.inflight > 0 for e in pages),
            }

    def close(self, *, cancel_pending: bool = False) -> None:
        """Drain I/O and release the directory (storage.py:572-590).

        ``cancel_pending`` retires outstanding completions before draining.
        Resident pages that were never spilled are not persisted.
        """
        with self._mutex:
            self._closing = True
            if cancel_pending:
                self._closed = True
                self._epoch += 1
        self._executor.shutdown(wait=True)
        with self._mutex:
            if self._lock_fd >= 0:
                self._closed = True
                self._epoch += 1
                os.close(self._lock_fd)
                self._lock_fd = -1
                self._lock_path.unlink()

    def __enter__(self) -> TieredPageStore:
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()
