"""Exception types of the paged-KV path.

Same names and meaning as light-vllm's: ``KVCacheError`` for shape, dtype,
device or metadata violations (src/light_vllm/runtime/kv_cache.py:21-26),
``ExecutionError`` / ``ExecutionNotReadyError`` for execution failures and a
missing runtime dependency (src/light_vllm/runtime/execution/interfaces.py:16-21).
"""

from __future__ import annotations


class KVCacheError(RuntimeError):
    """A KV cache state or metadata contract was violated."""


class KVCacheCapacityError(KVCacheError):
    """Not enough KV slots to complete a reservation."""


class ExecutionError(RuntimeError):
    """A model computation failed."""


class ExecutionNotReadyError(ExecutionError):
    """The backend's runtime dependency (the HIP library or a GPU) is missing."""
