"""Exception classes of the paged-KV path, bound to the host's own classes.

light-vllm acts on its own exception types, not on look-alikes:

* ``PagedStepHandler.compact`` turns a ``KVCacheError`` into an
  ``ExecutionError`` (src/light_vllm/runtime/execution/worker.py:316-323);
* the engine maps ``ExecutionNotReadyError`` to "load a model" and any other
  ``ExecutionError`` to a generation error carrying its message
  (src/light_vllm/runtime/engine/core.py:89-94).

So every raise site in this package looks its class up here at raise time
(``errors.KVCacheError(...)``), and the classes here are whatever the host
bound.  On import, light-vllm's classes are bound when its modules import
(src/light_vllm/runtime/kv_cache.py:21-26,
src/light_vllm/runtime/execution/interfaces.py:16-21); otherwise the local
stand-ins below are used.  ``bind()`` re-points them explicitly, for a host
that embeds light-vllm under another name or for a test; ``bind()`` with no
arguments returns to the import-time choice.
"""

from __future__ import annotations

import importlib

# Names a host may bind, with the keyword ``bind`` takes for each.
_KEYWORDS = {
    "kv_cache_error": "KVCacheError",
    "kv_cache_capacity_error": "KVCacheCapacityError",
    "execution_error": "ExecutionError",
    "not_ready_error": "ExecutionNotReadyError",
}


def _stand_ins() -> dict[str, type]:
    """Local classes with light-vllm's names and hierarchy."""

    kv = type("KVCacheError", (RuntimeError,), {"__doc__": "A KV cache state or metadata contract was violated."})
    capacity = type("KVCacheCapacityError", (kv,), {"__doc__": "Not enough KV slots to complete a reservation."})
    execution = type("ExecutionError", (RuntimeError,), {"__doc__": "A model computation failed."})
    not_ready = type(
        "ExecutionNotReadyError", (execution,),
        {"__doc__": "The backend's runtime dependency (the HIP library or a GPU) is missing."},
    )
    found = {"KVCacheError": kv, "KVCacheCapacityError": capacity, "ExecutionError": execution,
             "ExecutionNotReadyError": not_ready}
    for cls in found.values():
        cls.__module__ = __name__
    return found


def _host_classes() -> dict[str, type] | None:
    """light-vllm's classes when its modules import, else None."""

    try:
        kv_cache = importlib.import_module("light_vllm.runtime.kv_cache")
        execution = importlib.import_module("light_vllm.runtime.execution.interfaces")
    except ImportError:
        return None
    return {
        "KVCacheError": kv_cache.KVCacheError,
        "KVCacheCapacityError": kv_cache.KVCacheCapacityError,
        "ExecutionError": execution.ExecutionError,
        "ExecutionNotReadyError": execution.ExecutionNotReadyError,
    }


_LOCAL = _stand_ins()
_DEFAULT = _host_classes() or dict(_LOCAL)
_bound: dict[str, type] = dict(_DEFAULT)


def bind(
    *,
    kv_cache_error: type | None = None,
    kv_cache_capacity_error: type | None = None,
    execution_error: type | None = None,
    not_ready_error: type | None = None,
) -> None:
    """Raise the host's classes from now on.

    Unnamed classes return to their import-time choice.  The hierarchy the
    host's handlers rely on is checked: the capacity error must derive from
    the KV cache error and the not-ready error from the execution error.
    """

    given = {"kv_cache_error": kv_cache_error, "kv_cache_capacity_error": kv_cache_capacity_error,
             "execution_error": execution_error, "not_ready_error": not_ready_error}
    chosen = dict(_DEFAULT)
    for keyword, cls in given.items():
        if cls is None:
            continue
        if not (isinstance(cls, type) and issubclass(cls, Exception)):
            raise TypeError(f"{keyword} must be an exception class")
        chosen[_KEYWORDS[keyword]] = cls
    if kv_cache_error is not None and kv_cache_capacity_error is None:
        # Keep "capacity is a KV cache error" true for the bound class.
        chosen["KVCacheCapacityError"] = type("KVCacheCapacityError", (kv_cache_error,), {"__module__": __name__})
    if execution_error is not None and not_ready_error is None:
        chosen["ExecutionNotReadyError"] = type("ExecutionNotReadyError", (execution_error,), {"__module__": __name__})
    if not issubclass(chosen["KVCacheCapacityError"], chosen["KVCacheError"]):
        raise TypeError("kv_cache_capacity_error must derive from kv_cache_error")
    if not issubclass(chosen["ExecutionNotReadyError"], chosen["ExecutionError"]):
        raise TypeError("not_ready_error must derive from execution_error")
    _bound.update(chosen)


def bound() -> dict[str, type]:
    """The classes raise sites use now, by name."""

    return dict(_bound)


def __getattr__(name: str) -> type:
    try:
        return _bound[name]
    except KeyError:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}") from None
