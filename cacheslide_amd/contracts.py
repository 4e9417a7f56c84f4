"""Request token layouts (src/cacheslide_vllm/contracts.py:26-181), stdlib only.

What the attention policies and WCA take from a request: the ordered
reuse/recompute partition of the prompt, the fixed (reused) and mandatory
token indices, and the identity of the fixed chunks (id, content digest,
length) that keys calibrated profiles.  The request schema (version 1), the
digest (SHA-256 of canonical JSON) and the ValueError messages are the
reference's, so metadata accepted or keyed there is accepted and keyed alike.
"""

from __future__ import annotations

import hashlib
import json
from collections.abc import Mapping, Sequence
from dataclasses import dataclass

_OPERATIONS = ("recompute", "populate", "reuse", "calibrate")
_ROLES = ("reuse", "recompute")
_TOP_KEYS = frozenset(("version", "operation", "namespace", "task_id", "chunks"))
_CHUNK_KEYS = frozenset(("id", "role", "start", "end"))
_MAX_METADATA_BYTES = 1 << 20
_MAX_CHUNKS = 1024


def digest(value: object) -> str:
    """SHA-256 hex digest of ``value`` as canonical JSON (sorted keys, no spaces, ASCII)."""
    text = json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=True,
                      allow_nan=False)
    return hashlib.sha256(text.encode()).hexdigest()


def _identifier(value: object, name: str) -> str:
    if not (isinstance(value, str) and 0 < len(value) <= 256):
        raise ValueError(f"{name} must be a nonempty string of at most 256 characters")
    if min(map(ord, value)) < 32:
        raise ValueError(f"{name} must not contain control characters")
    return value


@dataclass(frozen=True)
class Chunk:
    chunk_id: str
    role: str
    start: int
    end: int

    @property
    def length(self) -> int:
        return self.end - self.start


def _document(value: str | Mapping) -> Mapping:
    if isinstance(value, str):
        if len(value.encode()) > _MAX_METADATA_BYTES:
            raise ValueError("CacheSlide request metadata exceeds 1 MiB")
        value = json.loads(value)
    if not isinstance(value, Mapping):
        raise ValueError("cacheslide must be a JSON object or encoded JSON string")
    version = value.get("version")
    if not set(value) <= _TOP_KEYS or type(version) is not int or version != 1:
        raise ValueError("unknown CacheSlide request field or schema version")
    return value


def _partition(entries: object, n_tokens: int) -> tuple[Chunk, ...]:
    """Chunks that tile [0, n_tokens) in order, each reused or recomputed, ids distinct."""
    if not isinstance(entries, (list, tuple)) or not entries:
        raise ValueError("chunks must be a nonempty list")
    if len(entries) > _MAX_CHUNKS:
        raise ValueError("at most 1024 chunks are supported")
    out: list[Chunk] = []
    ids: set[str] = set()
    for entry in entries:
        if not isinstance(entry, Mapping) or set(entry) != _CHUNK_KEYS:
            raise ValueError("each chunk needs exactly id, role, start, end")
        chunk_id = _identifier(entry["id"], "chunk id")
        start, end, role = entry["start"], entry["end"], entry["role"]
        if type(start) is not int or type(end) is not int:
            raise ValueError("chunk boundaries must be integer token offsets")
        expected_start = out[-1].end if out else 0
        if start != expected_start or not start < end <= n_tokens:
            raise ValueError("chunks must partition the prompt without gaps/overlaps")
        if not isinstance(role, str) or role not in _ROLES or chunk_id in ids:
            raise ValueError("invalid role or duplicate chunk id")
        ids.add(chunk_id)
        out.append(Chunk(chunk_id, role, start, end))
    if out[-1].end != n_tokens:
        raise ValueError("chunks must include every prompt token")
    return tuple(out)


@dataclass(frozen=True)
class RequestPlan:
    """An exact token partition of one prompt into reused and recomputed chunks."""

    operation: str
    namespace: str
    task_id: str
    chunks: tuple[Chunk, ...]
    token_ids: tuple[int, ...]

    @classmethod
    def parse(cls, value: str | Mapping, token_ids: Sequence[int]) -> "RequestPlan":
        doc = _document(value)
        operation = doc.get("operation")
        if not isinstance(operation, str) or operation not in _OPERATIONS:
            raise ValueError("operation must be recompute, populate, reuse, or calibrate")
        tokens = tuple(token_ids)
        if not tokens or not all(type(t) is int and t >= 0 for t in tokens):
            raise ValueError("prompt token ids must be nonnegative integers")
        chunks = _partition(doc.get("chunks"), len(tokens))
        return cls(operation, _identifier(doc.get("namespace"), "namespace"),
                   _identifier(doc.get("task_id"), "task_id"), chunks, tokens)

    def _tokens_of(self, role: str) -> list[int]:
        return [t for chunk in self.chunks if chunk.role == role for t in range(chunk.start, chunk.end)]

    def _memo(self, name: str, compute):
        """Derived values of this immutable plan, computed once: the runtime
        asks for them on every layer, and the attention policies key their
        device caches on the returned objects."""
        memo = self.__dict__.get("_derived")
        if memo is None:
            memo = {}
            object.__setattr__(self, "_derived", memo)
        if name not in memo:
            memo[name] = compute()
        return memo[name]

    @property
    def fixed_indices(self) -> tuple[int, ...]:
        """Token indices of the reused chunks, ascending."""
        return self._memo("fixed_indices", lambda: tuple(self._tokens_of("reuse")))

    @property
    def mandatory_indices(self) -> tuple[int, ...]:
        """Recomputed tokens plus the last prompt token, ascending."""
        return self._memo("mandatory_indices", lambda: tuple(
            sorted(set(self._tokens_of("recompute")) | {len(self.token_ids) - 1})))

    @property
    def fixed_layout(self) -> tuple[tuple[str, str, int], ...]:
        """(chunk id, digest of its token ids, length) of each reused chunk, in order."""
        return self._memo("fixed_layout", lambda: tuple(
            (c.chunk_id, digest(self.token_ids[c.start:c.end]), c.length)
            for c in self.chunks if c.role == "reuse"))

    def cache_key(self, model_identity: str, layer: int) -> str:
        """KV identity: model, namespace, task, the whole ordered fixed layout
        and the chunk roles, per layer."""
        roles = [(c.chunk_id, c.role) for c in self.chunks]
        return digest(["CacheSlide-KV-v2", model_identity, self.namespace, self.task_id,
                       self.fixed_layout, roles, layer])

    def profile_key(self, model_identity: str, layer: int) -> str:
        return digest(["CacheSlide-CCPE-v2", self.cache_key(model_identity, layer)])

    def to_json(self) -> str:
        """The version-1 request metadata this plan parses from."""
        return json.dumps({
            "version": 1,
            "operation": self.operation,
            "namespace": self.namespace,
            "task_id": self.task_id,
            "chunks": [{"id": c.chunk_id, "role": c.role, "start": c.start, "end": c.end}
                       for c in self.chunks],
        }, separators=(",", ":"))
