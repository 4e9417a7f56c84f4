"""Exception types shared by the slot map, the relocation helpers and the page
store; the names and bases are those of src/cacheslide_vllm/storage.py:21-30
so callers catch the same types."""


class CacheCapacityError(RuntimeError):
    """Not enough slots or capacity to perform an operation safely."""


class CacheIntegrityError(RuntimeError):
    """A persisted page failed its identity or checksum check."""


class StaleCompletionError(RuntimeError):
    """An asynchronous completion belongs to a retired map or generation."""
