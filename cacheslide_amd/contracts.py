"""Request token layouts (src/cacheslide_vllm/contracts.py:26-181), stdlib only.

Only what the attention policies and WCA need from a request: the ordered
reuse/recompute chunk partition, the fixed (reused) and mandatory token
indices, and the fixed-chunk layout identity.
"""

from __future__ import annotations

import hashlib
import json
from collections.abc import Mapping, Sequence
from dataclasses import dataclass

_OPERATIONS = ("recompute", "populate", "reuse", "calibrate")
_ROLES = ("reuse", "recompute")


def digest(value: object) -> str:
    """SHA-256 of canonical JSON (sorted keys, compact separators, ASCII)."""
    text = json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=True,
                      allow_nan=False)
    return hashlib.sha256(text.encode()).hexdigest()


def _identifier(value: object, name: str) -> str:
    if not isinstance(value, str) or not value or len(value) > 256:
        raise ValueError(f"{name} must be a nonempty string of at most 256 characters")
    if any(ord(ch) < 32 for ch in value):
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


@dataclass(frozen=True)
class RequestPlan:
    operation: str
    namespace: str
    task_id: str
    chunks: tuple[Chunk, ...]
    token_ids: tuple[int, ...]

    @classmethod
    def parse(cls, value: str | Mapping, token_ids: Sequence[int]) -> "RequestPlan":
        if isinstance(value, str):
            if len(value.encode()) > 1_048_576:
                raise ValueError("CacheSlide request metadata exceeds 1 MiB")
            value = json.loads(value)
        if not isinstance(value, Mapping):
            raise ValueError("cacheslide must be a JSON object or encoded JSON string")
        if (
            set(value) - {"version", "operation", "namespace", "task_id", "chunks"}
            or type(value.get("version")) is not int
            or value["version"] != 1
        ):
            raise ValueError("unknown CacheSlide request field or schema version")
        operation = value.get("operation")
        if not isinstance(operation, str) or operation not in _OPERATIONS:
            raise ValueError("operation must be recompute, populate, reuse, or calibrate")
        tokens = tuple(token_ids)
        if not tokens or any(type(t) is not int or t < 0 for t in tokens):
            raise ValueError("prompt token ids must be nonnegative integers")
        entries = value.get("chunks")
        if not isinstance(entries, (list, tuple)) or not entries:
            raise ValueError("chunks must be a nonempty list")
        if len(entries) > 1024:
            raise ValueError("at most 1024 chunks are supported")
        chunks: list[Chunk] = []
        cursor = 0
        seen: set[str] = set()
        for entry in entries:
            if not isinstance(entry, Mapping) or set(entry) != {"id", "role", "start", "end"}:
                raise ValueError("each chunk needs exactly id, role, start, end")
            chunk_id = _identifier(entry["id"], "chunk id")
            start, end = entry["start"], entry["end"]
            if type(start) is not int or type(end) is not int:
                raise ValueError("chunk boundaries must be integer token offsets")
            if start != cursor or not start < end <= len(tokens):
                raise ValueError("chunks must partition the prompt without gaps/overlaps")
            role = entry["role"]
            if not isinstance(role, str) or role not in _ROLES or chunk_id in seen:
                raise ValueError("invalid role or duplicate chunk id")
            chunks.append(Chunk(chunk_id, role, start, end))
            seen.add(chunk_id)
            cursor = end
        if cursor != len(tokens):
            raise ValueError("chunks must include every prompt token")
        return cls(
            operation,
            _identifier(value.get("namespace"), "namespace"),
            _identifier(value.get("task_id"), "task_id"),
            tuple(chunks),
            tokens,
        )

    @property
    def fixed_indices(self) -> tuple[int, ...]:
        """Token indices of reused chunks, ascending."""
        out: list[int] = []
        for chunk in self.chunks:
            if chunk.role == "reuse":
                out.extend(range(chunk.start, chunk.end))
        return tuple(out)

    @property
    def mandatory_indices(self) -> tuple[int, ...]:
        """Recomputed tokens plus the last prompt token, ascending."""
        mandatory = {len(self.token_ids) - 1}
        for chunk in self.chunks:
            if chunk.role == "recompute":
                mandatory.update(range(chunk.start, chunk.end))
        return tuple(sorted(mandatory))

    @property
    def fixed_layout(self) -> tuple[tuple[str, str, int], ...]:
        return tuple(
            (chunk.chunk_id, digest(self.token_ids[chunk.start : chunk.end]), chunk.length)
            for chunk in self.chunks
            if chunk.role == "reuse"
        )

    def cache_key(self, model_identity: str, layer: int) -> str:
        return digest(
            [
                "CacheSlide-KV-v2",
                model_identity,
                self.namespace,
                self.task_id,
                self.fixed_layout,
                [(chunk.chunk_id, chunk.role) for chunk in self.chunks],
                layer,
            ]
        )

    def profile_key(self, model_identity: str, layer: int) -> str:
        return digest(["CacheSlide-CCPE-v2", self.cache_key(model_identity, layer)])
