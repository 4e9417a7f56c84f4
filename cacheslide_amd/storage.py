"""Exception types shared by the slot map and the paged arena.

Mirrors the exception classes of src/cacheslide_vllm/storage.py:21-30; the
host/SSD page store itself is outside this package.
"""

from __future__ import annotations


class CacheCapacityError(RuntimeError):
    """Not enough slots or capacity to perform an operation safely."""


class CacheIntegrityError(RuntimeError):
    """A persisted page failed its identity or checksum check."""


class StaleCompletionError(RuntimeError):
    """An asynchronous completion belongs to a retired map or generation."""
