"""MI355X-native (gfx950) paged-KV attention backend for light-vllm.

The directory name is not a Python identifier, so the package registers itself
as ``light_vllm_amd`` on import and all of its modules use that name.  Import
it with ``importlib.import_module("light-vllm_amd")`` (the repository root on
``sys.path``), then use ``light_vllm_amd``.
"""

import sys as _sys

_sys.modules.setdefault("light_vllm_amd", _sys.modules[__name__])

from light_vllm_amd.backend import HipPagedAttention, HipPagedAttentionBackend  # noqa: E402
from light_vllm_amd import errors  # noqa: E402
from light_vllm_amd.interfaces import (  # noqa: E402
    AttentionLayerSpec,
    DraftTree,
    ModelKVCacheSpec,
    QueryLayout,
)
from light_vllm_amd.layout import (  # noqa: E402
    append_draft_layout,
    linear_query_layout,
    query_visibility,
    semantic_positions,
)
from light_vllm_amd.metadata import PagedAttentionMetadata  # noqa: E402
from light_vllm_amd.prefix_cow import SharedPrefix, copy_commands, share_prefix  # noqa: E402
from light_vllm_amd.paged_cache import (  # noqa: E402
    PagedKVCache,
    PagedKVCacheConfig,
    PagedKVWriteMapping,
    PagedLayerCache,
    hip_block_copy,
    hip_compact,
    kv_cache_bytes_per_block,
)

# ``from light_vllm_amd import errors`` registers the submodule under the
# directory's name and ``import light_vllm_amd.errors`` under the alias; a
# module found under only one of them would be loaded a second time under
# the other, with its own state (the bound exception classes, the loaded
# library).  Every submodule is imported by now: register each under both.
for _name, _module in list(_sys.modules.items()):
    for _have, _add in (("light-vllm_amd.", "light_vllm_amd."), ("light_vllm_amd.", "light-vllm_amd.")):
        if _name.startswith(_have):
            _sys.modules.setdefault(_add + _name[len(_have):], _module)
del _name, _module, _have, _add

__all__ = [
    "AttentionLayerSpec",
    "DraftTree",
    "ExecutionError",
    "ExecutionNotReadyError",
    "HipPagedAttention",
    "HipPagedAttentionBackend",
    "KVCacheCapacityError",
    "KVCacheError",
    "ModelKVCacheSpec",
    "PagedAttentionMetadata",
    "PagedKVCache",
    "PagedKVCacheConfig",
    "PagedKVWriteMapping",
    "PagedLayerCache",
    "QueryLayout",
    "SharedPrefix",
    "append_draft_layout",
    "copy_commands",
    "hip_block_copy",
    "hip_compact",
    "kv_cache_bytes_per_block",
    "linear_query_layout",
    "query_visibility",
    "semantic_positions",
    "share_prefix",
]


# The exception classes are the ones bound in ``errors`` at lookup time (the
# host's own classes when light-vllm is importable or ``errors.bind`` named
# them), so ``light_vllm_amd.KVCacheError`` is always what raise sites raise.
_ERROR_NAMES = ("ExecutionError", "ExecutionNotReadyError", "KVCacheCapacityError", "KVCacheError")


def __getattr__(name: str):
    if name in _ERROR_NAMES:
        return getattr(errors, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
