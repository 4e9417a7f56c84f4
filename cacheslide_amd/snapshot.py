"""Layer snapshots between the page store and HBM (src/cacheslide_vllm/runtime.py:192-272).

The reference runtime persists, per layer, the fixed tokens' K/V rows
(``"kv"``: ``k``, ``v`` of ``[fixed, kv_heads, head_dim]``) and layer inputs
(``"state"``: ``hidden``, ``residual`` of ``[fixed, hidden_size]``) as
safetensors pages in its page store, and reads them back on reuse,
prefetching the next layer's K/V while the current layer computes.  Any store
with ``put`` / ``read`` / ``contains`` / ``submit_load`` / ``submit_spill``
works here; ``cacheslide_amd.pagestore.PageStore`` is the one this package
ships.

Its read path decodes the page into CPU tensors, checks them for non-finite
values on the CPU and copies them with ``.to(device, dtype)``, all on the
compute thread after the prefetched bytes arrive.  Here:

* the page's data region is copied into pinned staging and moved to HBM in
  one DMA (``cs_copy_async``) on an upload stream of its own;
* the finite check and any dtype conversion run on that stream on the device
  (``cs_snapshot_convert``) and one 4-byte flag word comes back;
* a prefetch does the store lookup (and its checksum), the staging and the
  DMA on a worker thread, so the compute thread only waits for the flag word
  and orders its stream after the upload's event.

Pages are byte-for-byte the reference's: ``encode_snapshot`` writes what
``safetensors.torch.save`` writes for the same tensors (tensors ordered by
descending dtype rank, then name; compact JSON header padded with spaces to 8
bytes), and ``parse_snapshot`` accepts and rejects what the safetensors loader
accepts and rejects for the dtypes a snapshot can hold.
"""

from __future__ import annotations

import ctypes
import json
import math
import threading
from collections.abc import Callable, Mapping
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from . import _hip
from ._hip import call, require_device, vref
from .runtime_rows import ReuseFailure

SNAPSHOT_FIELDS = {"kv": ("k", "v"), "state": ("hidden", "residual")}

# safetensors dtype names: torch dtype (None: no snapshot may hold it), bytes per
# element.  Listed from the highest sort rank to the lowest: a page stores its
# tensors in this order, ties by name.
_ST_DTYPES: list[tuple[str, torch.dtype | None, int]] = [
    ("U64", getattr(torch, "uint64", None), 8),
    ("I64", torch.int64, 8),
    ("F64", torch.float64, 8),
    ("F32", torch.float32, 4),
    ("U32", getattr(torch, "uint32", None), 4),
    ("I32", torch.int32, 4),
    ("BF16", torch.bfloat16, 2),
    ("F16", torch.float16, 2),
    ("U16", getattr(torch, "uint16", None), 2),
    ("I16", torch.int16, 2),
    ("F8_E4M3", torch.float8_e4m3fn, 1),
    ("F8_E5M2", torch.float8_e5m2, 1),
    ("I8", torch.int8, 1),
    ("U8", torch.uint8, 1),
    ("BOOL", torch.bool, 1),
]
_RANK = {name: len(_ST_DTYPES) - i for i, (name, _, _) in enumerate(_ST_DTYPES)}
_SIZE = {name: size for name, _, size in _ST_DTYPES}
_TORCH = {name: dtype for name, dtype, _ in _ST_DTYPES}
_NAME = {dtype: name for name, dtype, _ in _ST_DTYPES if dtype is not None}
# the floating dtypes the device check and conversion handle
_DEVICE_FLOATS = {torch.float64, torch.float32, torch.bfloat16, torch.float16}
_MAX_HEADER = 100_000_000
_NONFINITE = 1


@dataclass(frozen=True)
class SnapshotTensor:
    """One tensor of a page: name, safetensors dtype, shape, byte range in the data region."""

    name: str
    dtype: str
    shape: tuple[int, ...]
    begin: int
    end: int

    @property
    def torch_dtype(self) -> torch.dtype | None:
        return _TORCH[self.dtype]


def snapshot_shapes(kind: str, layer: int, count: int, *, kv_heads: int, head_dim: int,
                    hidden_size: int) -> dict[str, tuple[int, ...]]:
    """The geometry a page must have (runtime.py:209-222); layer 0 has no residual."""
    if kind == "kv":
        return {"k": (count, kv_heads, head_dim), "v": (count, kv_heads, head_dim)}
    if kind == "state":
        return {"hidden": (count, hidden_size), "residual": (0,) if layer == 0 else (count, hidden_size)}
    raise ValueError(f"unknown snapshot kind {kind!r}")


# ------------------------------------------------------------------- format
def snapshot_header(specs: Mapping[str, tuple[torch.dtype, tuple[int, ...]]]) -> tuple[bytes, list[SnapshotTensor]]:
    """The 8-byte length, the padded JSON header and the tensor layout of a page.

    ``specs`` maps name -> (dtype, shape).  Tensors are laid out by descending
    dtype rank, then name, back to back from offset 0 of the data region.
    """
    order = []
    for name, (dtype, shape) in specs.items():
        if not isinstance(name, str):
            raise ValueError("snapshot tensor names must be strings")
        if dtype not in _NAME:
            raise ValueError(f"dtype {dtype} cannot be stored in a snapshot")
        order.append((name, _NAME[dtype], tuple(int(s) for s in shape)))
    order.sort(key=lambda item: (-_RANK[item[1]], item[0]))
    layout, pos = [], 0
    for name, st, shape in order:
        size = math.prod(shape) * _SIZE[st]
        layout.append(SnapshotTensor(name, st, shape, pos, pos + size))
        pos += size
    text = json.dumps(
        {t.name: {"dtype": t.dtype, "shape": list(t.shape), "data_offsets": [t.begin, t.end]} for t in layout},
        separators=(",", ":"), ensure_ascii=False,
    ).encode("utf-8")
    text += b" " * (-len(text) % 8)
    return len(text).to_bytes(8, "little") + text, layout


def parse_snapshot(data) -> tuple[list[SnapshotTensor], int]:
    """Tensors of a page and the offset of its data region; ValueError on any malformation.

    The checks are the safetensors loader's: header length bounded and inside
    the buffer, a UTF-8 JSON object, every entry a known dtype with a
    non-negative integer shape and offsets, offsets tiling the data region
    from 0 without gaps or overlaps, each range the size its shape and dtype
    give, and the data region ending at the end of the buffer.
    """
    buf = memoryview(data).cast("B")
    if len(buf) < 8:
        raise ValueError("snapshot is shorter than its header length")
    n = int.from_bytes(buf[:8], "little")
    if n > _MAX_HEADER:
        raise ValueError("snapshot header is too large")
    if 8 + n > len(buf):
        raise ValueError("snapshot header length exceeds the page")
    try:
        text = bytes(buf[8:8 + n]).decode("utf-8")
    except UnicodeDecodeError as exc:
        raise ValueError("snapshot header is not UTF-8") from exc
    if not text.startswith("{"):
        raise ValueError("snapshot header is not a JSON object")
    try:
        header = json.loads(text)
    except json.JSONDecodeError as exc:
        raise ValueError("snapshot header is not valid JSON") from exc
    if not isinstance(header, dict):
        raise ValueError("snapshot header is not a JSON object")
    meta = header.pop("__metadata__", None)
    if meta is not None and (not isinstance(meta, dict)
                             or not all(isinstance(v, str) for v in meta.values())):
        raise ValueError("snapshot metadata must map strings to strings")

    def count(value) -> bool:
        return type(value) is int and value >= 0

    tensors = []
    for name, info in header.items():
        if not isinstance(info, dict):
            raise ValueError(f"snapshot entry {name!r} is not an object")
        dtype, shape, offsets = info.get("dtype"), info.get("shape"), info.get("data_offsets")
        if dtype not in _SIZE:
            raise ValueError(f"snapshot entry {name!r} has an unknown dtype")
        if not isinstance(shape, list) or not all(count(s) for s in shape):
            raise ValueError(f"snapshot entry {name!r} has an invalid shape")
        if not isinstance(offsets, list) or len(offsets) != 2 or not all(count(o) for o in offsets):
            raise ValueError(f"snapshot entry {name!r} has invalid data offsets")
        tensors.append(SnapshotTensor(name, dtype, tuple(shape), offsets[0], offsets[1]))
    pos = 0
    for t in sorted(tensors, key=lambda t: (t.begin, t.end)):
        if t.begin != pos or t.end < t.begin:
            raise ValueError("snapshot data offsets do not tile the data region")
        if t.end - t.begin != math.prod(t.shape) * _SIZE[t.dtype]:
            raise ValueError(f"snapshot entry {t.name!r} size disagrees with its shape")
        pos = t.end
    if 8 + n + pos != len(buf):
        raise ValueError("snapshot data region does not end with the page")
    return tensors, 8 + n


def check_schema(tensors: list[SnapshotTensor], shapes: Mapping[str, tuple[int, ...]]) -> None:
    """runtime.py:207-226: the field set, the geometry and a floating dtype."""
    if {t.name for t in tensors} != set(shapes):
        raise ValueError("snapshot fields differ from the runtime schema")
    for t in tensors:
        dtype = t.torch_dtype
        if t.shape != tuple(shapes[t.name]) or dtype is None or not dtype.is_floating_point:
            raise ValueError("snapshot tensor geometry is incompatible")
        if dtype not in _DEVICE_FLOATS:
            raise ValueError(f"snapshot dtype {t.dtype} is not supported on the device")


# ------------------------------------------------------------------- device
class _Pinned:
    """A growable pinned host buffer whose last DMA is tracked by an event."""

    def __init__(self):
        self.buffer: Tensor | None = None
        self.event: torch.cuda.Event | None = None

    def reserve(self, nbytes: int) -> Tensor:
        if self.event is not None:
            self.event.synchronize()  # the previous DMA from this buffer has finished
        if self.buffer is None or self.buffer.numel() < nbytes:
            self.buffer = torch.empty(max(nbytes, 1), dtype=torch.uint8, pin_memory=True)
        return self.buffer


@dataclass
class _Upload:
    tensors: dict[str, Tensor]
    done: torch.cuda.Event
    flag: Tensor  # pinned int32 [1]
    nbytes: int


class SnapshotUploader:
    """Pinned staging, an upload stream and worker threads for one device.

    ``submit(fetch, shapes, dtype)`` runs ``fetch()`` (the page's bytes, with
    the store's checksum) on one of ``fetchers`` threads, then, on the single
    staging thread and in submission order, checks the header and schema,
    copies the data region into pinned memory (``copy_threads`` threads) and
    enqueues its DMA plus the device check/conversion on the upload stream.
    ``SnapshotUploader.take(future)`` waits for the flag word, raises for a
    non-finite page, and orders the caller's current stream after the upload.
    """

    _CHUNK = 8 << 20   # a DMA is issued per staged chunk of a tensor
    _PIECE = 1 << 20   # the least a staging thread copies

    def __init__(self, device, *, slots: int = 2, fetchers: int = 1, copy_threads: int = 4):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("snapshots are uploaded to a HIP device")
        _hip.load()
        with torch.cuda.device(self.device):
            self.stream = torch.cuda.Stream(self.device)  # default priority
        self._slots = [_Pinned() for _ in range(max(1, slots))]
        self._next = 0
        self._fetch = ThreadPoolExecutor(max_workers=max(1, fetchers), thread_name_prefix="cacheslide-fetch")
        self._pool = ThreadPoolExecutor(max_workers=1, thread_name_prefix="cacheslide-upload")
        self._copy = ThreadPoolExecutor(max_workers=max(1, copy_threads), thread_name_prefix="cacheslide-stage")
        self._copy_threads = max(1, copy_threads)
        self._lock = threading.Lock()
        self.uploaded_bytes = 0

    def submit(self, fetch: Callable[[], bytes], shapes: Mapping[str, tuple[int, ...]],
               dtype: torch.dtype) -> Future:
        if dtype not in _DEVICE_FLOATS:
            raise ValueError(f"snapshot target dtype {dtype} is not supported")
        fetched = self._fetch.submit(fetch)
        return self._pool.submit(self._upload, fetched, dict(shapes), dtype)

    def _stage(self, dst: np.ndarray, src: np.ndarray) -> None:
        """Copy into pinned memory in parallel pieces (numpy releases the GIL for the copies)."""
        n = len(src)
        pieces = min(self._copy_threads, max(1, n // self._PIECE))
        if pieces == 1:
            np.copyto(dst, src)
            return
        step = -(-n // pieces)
        jobs = [self._copy.submit(np.copyto, dst[a:a + step], src[a:a + step]) for a in range(0, n, step)]
        for job in jobs:
            job.result()

    def _upload(self, fetched: Future, shapes, dtype) -> _Upload:
        data = fetched.result()
        tensors, start = parse_snapshot(data)
        check_schema(tensors, shapes)
        nbytes = len(data) - start
        slot = self._slots[self._next]
        self._next = (self._next + 1) % len(self._slots)
        staging = slot.reserve(nbytes)
        stream = ctypes.c_void_p(self.stream.cuda_stream)
        host = staging.data_ptr()
        with torch.cuda.device(self.device), torch.cuda.stream(self.stream):
            # each tensor into its own allocation (aligned whatever the page's
            # offsets); its bytes are staged chunk by chunk, and each chunk's DMA
            # runs while the next chunk is copied into pinned memory
            raw = {t.name: torch.empty(t.shape, dtype=t.torch_dtype, device=self.device) for t in tensors}
            if nbytes:
                src = np.frombuffer(data, dtype=np.uint8, count=nbytes, offset=start)
                dst = staging.numpy()
                for t in tensors:
                    base = raw[t.name].data_ptr()
                    for lo in range(t.begin, t.end, self._CHUNK):
                        hi = min(lo + self._CHUNK, t.end)
                        self._stage(dst[lo:hi], src[lo:hi])
                        call("cs_copy_async", ctypes.c_void_p(base + lo - t.begin), ctypes.c_void_p(host + lo),
                             hi - lo, _hip.COPY_H2D, stream)
            slot.event = torch.cuda.Event()
            slot.event.record(self.stream)
            flags = _hip.new_flags(self.device)
            out = {}
            for t in tensors:
                src = raw[t.name]
                if src.dtype == dtype:
                    call("cs_snapshot_convert", vref(src), vref(None), _NONFINITE, _hip.ptr(flags), stream)
                    out[t.name] = src
                else:
                    dst = torch.empty(t.shape, dtype=dtype, device=self.device)
                    call("cs_snapshot_convert", vref(src), vref(dst), _NONFINITE, _hip.ptr(flags), stream)
                    out[t.name] = dst
            flag = torch.zeros(1, dtype=torch.int32, pin_memory=True)
            call("cs_copy_async", ctypes.c_void_p(flag.data_ptr()), _hip.ptr(flags), 4, _hip.COPY_D2H, stream)
            done = torch.cuda.Event()
            done.record(self.stream)
        with self._lock:
            self.uploaded_bytes += nbytes
        return _Upload(out, done, flag, nbytes)

    @staticmethod
    def take(future: Future) -> dict[str, Tensor]:
        """The uploaded tensors, usable on the caller's current stream."""
        upload: _Upload = future.result()
        upload.done.synchronize()
        if int(upload.flag[0]) & _NONFINITE:
            raise ValueError("snapshot tensor is nonfinite")
        if not upload.tensors:
            return {}
        device = next(iter(upload.tensors.values())).device
        current = torch.cuda.current_stream(device)
        current.wait_event(upload.done)
        for tensor in upload.tensors.values():
            tensor.record_stream(current)
        return upload.tensors

    @staticmethod
    def drain(future: Future) -> None:
        """Wait for an upload without taking its tensors (a dropped prefetch)."""
        future.result().done.synchronize()

    def close(self) -> None:
        self._fetch.shutdown(wait=True)
        self._pool.shutdown(wait=True)
        self._copy.shutdown(wait=True)
        self.stream.synchronize()


def encode_snapshot(tensors: Mapping[str, Tensor]) -> bytes:
    """Page bytes of device tensors, equal to ``safetensors.torch.save`` of their CPU copies.

    runtime.py:238-243 copies each tensor to pageable host memory and then
    serializes it; here every tensor is copied once, on the current stream,
    into its place in a pinned image of the page.
    """
    items = {name: t for name, t in tensors.items()}
    device = require_device(*items.values()) if items else None
    header, layout = snapshot_header({name: (t.dtype, tuple(t.shape)) for name, t in items.items()})
    total = len(header) + (layout[-1].end if layout else 0)
    image = torch.empty(total, dtype=torch.uint8, pin_memory=True)
    host = image.numpy()
    host[:len(header)] = np.frombuffer(header, dtype=np.uint8)
    if device is not None:
        stream = torch.cuda.current_stream(device)
        keep = []
        for t in layout:
            src = items[t.name].detach().contiguous()
            keep.append(src)
            call("cs_copy_async", ctypes.c_void_p(image.data_ptr() + len(header) + t.begin), _hip.ptr(src),
                 t.end - t.begin, _hip.COPY_D2H, ctypes.c_void_p(stream.cuda_stream))
        stream.synchronize()
    return host.tobytes()


def _convert(tensors: dict[str, Tensor], dtype: torch.dtype) -> dict[str, Tensor]:
    """Checked tensors converted to ``dtype`` on the current stream (a prefetch made for another dtype)."""
    out = {}
    for name, t in tensors.items():
        if t.dtype == dtype:
            out[name] = t
            continue
        dst = torch.empty(t.shape, dtype=dtype, device=t.device)
        flags = _hip.new_flags(t.device)
        call("cs_snapshot_convert", vref(t), vref(dst), _NONFINITE, _hip.ptr(flags),
             _hip.stream_of(t.device))
        out[name] = dst
    return out


# -------------------------------------------------------------------- runtime
class LayerSnapshots:
    """The runtime's snapshot reads, writes and K/V prefetch for one request.

    Mirrors ``CacheSlideRuntime._read`` / ``_put`` / ``_prefetch``
    (runtime.py:192-272) with the request's store, plan and model geometry
    bound: keys are ``plan.cache_key(identity, layer) + "/" + kind`` and
    errors are ``ReuseFailure`` with the reference's messages.  ``read``
    returns device tensors in ``dtype``.

    ``prefetch_depth`` 1 is the reference's policy: one K/V prefetch may be
    outstanding.  A larger depth keeps the next ``prefetch_depth`` layers in
    flight, so their checksums (sequential within a page) run on that many
    threads at once.
    """

    def __init__(self, store, plan, identity: str, device, *, layers: int, kv_heads: int,
                 head_dim: int, hidden_size: int, reuse: bool = True, write_cache: bool = False,
                 prefetch_depth: int = 1, uploader: SnapshotUploader | None = None):
        if prefetch_depth < 1:
            raise ValueError("prefetch_depth must be positive")
        self.store, self.plan, self.identity = store, plan, identity
        self.layers, self.reuse, self.write_cache = layers, reuse, write_cache
        self.depth = prefetch_depth
        self.geometry = {"kv_heads": kv_heads, "head_dim": head_dim, "hidden_size": hidden_size}
        self._owns_uploader = uploader is None
        self.uploader = uploader if uploader is not None else SnapshotUploader(device, fetchers=prefetch_depth)
        self._pending: dict[int, tuple[Future, torch.dtype]] = {}
        self.created_keys: list[str] = []
        self.metrics = {"snapshot_bytes_written": 0}

    @property
    def kv_future(self) -> Future | None:
        """The oldest outstanding K/V prefetch (runtime.py ``state.kv_future``)."""
        return self._pending[min(self._pending)][0] if self._pending else None

    @property
    def kv_future_layer(self) -> int:
        return min(self._pending) if self._pending else -1

    def key(self, layer: int, kind: str) -> str:
        return self.plan.cache_key(self.identity, layer) + "/" + kind

    def _shapes(self, layer: int, kind: str) -> dict[str, tuple[int, ...]]:
        return snapshot_shapes(kind, layer, len(self.plan.fixed_indices), **self.geometry)

    def read(self, layer: int, kind: str, dtype: torch.dtype) -> dict[str, Tensor]:
        """runtime.py:192-229."""
        key = self.key(layer, kind)
        try:
            if kind == "kv" and layer in self._pending:
                future, made_for = self._pending.pop(layer)
                tensors = self.uploader.take(future)
                return tensors if made_for == dtype else _convert(tensors, dtype)
            future = self.uploader.submit(lambda: self.store.read(key), self._shapes(layer, kind), dtype)
            return self.uploader.take(future)
        except (ValueError, KeyError, OSError, RuntimeError) as exc:
            raise ReuseFailure(f"invalid {kind} snapshot at layer {layer}") from exc

    def put(self, layer: int, kind: str, tensors: Mapping[str, Tensor]) -> None:
        """runtime.py:231-256: persist one layer's snapshot and publish it to disk."""
        if not self.write_cache:
            return
        key = self.key(layer, kind)
        try:
            if self.store.contains(key):
                raise ReuseFailure("population collides with immutable pages")
            data = encode_snapshot(tensors)
            self.store.put(key, data, selected_count=0)
            self.created_keys.append(key)
            # each layer is persisted rather than accumulating the model in host RAM
            self.store.submit_spill(key).result()
        except (ValueError, OSError, RuntimeError) as exc:
            raise ReuseFailure(f"cannot persist {kind} snapshot at layer {layer}") from exc
        self.metrics["snapshot_bytes_written"] += len(data)

    def prefetch(self, layer: int, dtype: torch.dtype) -> None:
        """runtime.py:267-272; the lookup, checksum, staging and DMA run on the uploader's threads."""
        if not self.reuse or layer >= self.layers:
            return
        if self.depth == 1 and self._pending:
            raise RuntimeError("more than one outstanding KV prefetch")
        for target in range(layer, min(layer + self.depth, self.layers)):
            if target in self._pending:
                continue
            if len(self._pending) >= self.depth:
                raise RuntimeError("more KV prefetches outstanding than prefetch_depth")
            key = self.key(target, "kv")
            future = self.uploader.submit(lambda key=key: self.store.submit_load(key).result(),
                                          self._shapes(target, "kv"), dtype)
            self._pending[target] = (future, dtype)

    def close(self) -> None:
        """release(), then shut down the uploader when this object created it."""
        self.release()
        if self._owns_uploader:
            self.uploader.close()

    def __enter__(self) -> LayerSnapshots:
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()

    def release(self) -> None:
        """Drain pending prefetches before the request's pages may change (runtime.py:162-171)."""
        pending, self._pending = self._pending, {}
        for future, _ in pending.values():
            try:
                self.uploader.drain(future)
            except Exception:
                pass
