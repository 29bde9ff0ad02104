"""ctypes binding of the gfx950 HIP library (``liblvamd_hip.so``), and the
loader of the native host planner (``_lvamd_host``).

The library is the product: there is no CPU or PyTorch fallback.  ``load()``
and ``host()`` raise ``ExecutionNotReadyError`` when their module has not been
built, and every call that returns a non-zero status raises ``ExecutionError``
(the host's classes when bound, see ``errors``).
"""

from __future__ import annotations

import ctypes
import functools
import importlib.util
import re
import sysconfig
from pathlib import Path

from light_vllm_amd import errors

LIB_NAME = "liblvamd_hip.so"
ABI_VERSION = 20
PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
HEADER = REPO_ROOT / "include" / "lvamd_paged_kv.h"

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
REQ_FIELDS = 8
PIECE_FIELDS = 16
MERGE_FIELDS = 8
PREFILL_FIELDS = 16

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

# name -> (restype, argtypes); must match include/lvamd_paged_kv.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "lvamd_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "lvamd_abi_version": (ctypes.c_int, []),
    "lvamd_xcd_count": (ctypes.c_int, []),
    "lvamd_kv_append": (
        ctypes.c_int,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _i32, _i32, _i32, _p],
    ),
    "lvamd_kv_append_rotary": (
        ctypes.c_int,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _p, _i64,
         _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _p],
    ),
    "lvamd_paged_decode": (
        ctypes.c_int,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _i64,
         _p, _p, _i32, _p, _p, _p, _p, _i64,
         _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _p],
    ),
    "lvamd_paged_decode_split_groups": (ctypes.c_int, [_i32, _i32]),
    "lvamd_paged_decode_split_waves": (ctypes.c_int, [_i32, _i32]),
    "lvamd_paged_attention": (
        ctypes.c_int,
        [_p, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _f32, _p],
    ),
    "lvamd_paged_decode_resident_waves": (ctypes.c_int, [_i32, _i32, _i32]),
    "lvamd_paged_decode_tile_tokens": (ctypes.c_int, [_i32, _i32, _i32]),
    "lvamd_paged_attention_merge": (
        ctypes.c_int,
        [_p, _p, _p, _i64, _i64, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p],
    ),
    "lvamd_paged_prefill": (
        ctypes.c_int,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _i64, _p, _p, _p, _i32, _p, _p, _i64,
         _i32, _i32, _i32, _i32, _i32, _f32, _i32, _p],
    ),
    "lvamd_paged_prefill_unit_columns": (ctypes.c_int, [_i32, _i32]),
    "lvamd_paged_prefill_key_tokens": (ctypes.c_int, [_i32, _i32]),
    "lvamd_paged_prefill_resident_units": (ctypes.c_int, [_i32, _i32, _i32]),
    "lvamd_paged_prefill_waves_built": (ctypes.c_int, [_i32, _i32, _i32]),
    "lvamd_kv_compact": (
        ctypes.c_int,
        [_p, _p, _i32, _i64, _p, _p, _i64, _p, _i64, _p],
    ),
    "lvamd_kv_compact_static": (
        ctypes.c_int,
        [_p, _p, _i32, _i64, _p, _p, _i64, _p],
    ),
    "lvamd_kv_compact_ordered": (
        ctypes.c_int,
        [_p, _p, _i32, _i64, _p, _p, _p, _i64, _p],
    ),
    "lvamd_kv_compact_small": (
        ctypes.c_int,
        [_p, _p, _i32, _i64, _p, _p, _i64, _p],
    ),
    "lvamd_kv_compact_inline_pairs": (_i64, []),
    "lvamd_kv_block_copy_small": (
        ctypes.c_int,
        [_p, _p, _i32, _i64, _p, _p, _i64, _p],
    ),
    "lvamd_kv_block_copy_small_pairs": (_i64, []),
    "lvamd_kv_compact_workspace_size": (_i64, [_i64, _i32, _i64]),
    "lvamd_kv_block_copy": (
        ctypes.c_int,
        [_p, _p, _i32, _i64, _p, _p, _i64, _p],
    ),
    "lvamd_stage_upload": (ctypes.c_int, [_p, _p, _i64, _p, _p]),
    "lvamd_hbm_read_probe": (ctypes.c_int, [_p, _i64, _p, _i32, _p]),
}


class AttentionPlan(ctypes.Structure):
    """``lvamd_attention_plan``: one layer shape's launch facts in one step plan."""

    _fields_ = [
        ("pieces", _p), ("wave_first", _p), ("waves_per_head", _i32), ("col_tiles", _i32),
        ("part_acc", _p), ("part_ml", _p), ("num_partial_slots", _i64),
        ("jobs", _p), ("num_jobs", _i32), ("merge_columns", _i32), ("group_waves", _i32),
        ("units", _p), ("num_units", _i32), ("prefill_waves", _i32),
        ("prefill_part_acc", _p), ("prefill_part_ml", _p), ("num_prefill_partial_slots", _i64),
        ("prefill_jobs", _p), ("num_prefill_jobs", _i32), ("prefill_merge_columns", _i32),
        ("prefill_col_tiles", _i32), ("num_kv_heads", _i32),
        ("tables", _p), ("vis", _p), ("group", _i32), ("head_size", _i32), ("block_size", _i32), ("dtype", _i32),
    ]


def library_path() -> Path:
    return PACKAGE_DIR / LIB_NAME


HOST_MODULE = "_lvamd_host"


def host_path() -> Path:
    return PACKAGE_DIR / (HOST_MODULE + sysconfig.get_config_var("EXT_SUFFIX"))


@functools.lru_cache(maxsize=1)
def host():
    """The native host planner (``csrc/lvamd_host.cpp``), built next to the HIP library."""

    path = host_path()
    if not path.exists():
        raise errors.ExecutionNotReadyError(
            f"the host planner {path} is not built; run __graft_entry__.build() first"
        )
    spec = importlib.util.spec_from_file_location(HOST_MODULE, path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def header_functions() -> list[str]:
    """Names of every function the C header declares."""

    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lvamd_[a-z0-9_]+)\s*\(", text)))


@functools.lru_cache(maxsize=1)
def load() -> ctypes.CDLL:
    path = library_path()
    if not path.exists():
        raise errors.ExecutionNotReadyError(
            f"the HIP library {path} is not built; run __graft_entry__.build() first"
        )
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.lvamd_abi_version()
    if version != ABI_VERSION:
        raise errors.ExecutionNotReadyError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    return lib


# Column tiles per decode wave the library builds: 1, and 4 for narrow rows.
DECODE_COL_TILES = (1, 4)

_RESIDENT: dict[tuple, int] = {}


def resident_decode_waves(dtype_code: int, head_size: int, col_tiles: int = 1) -> int:
    """Decode waves the current GPU holds at once (cached per kernel)."""

    key = (dtype_code, head_size, col_tiles)
    found = _RESIDENT.get(key)
    if found is None:
        found = load().lvamd_paged_decode_resident_waves(dtype_code, head_size, col_tiles)
        check(min(found, 0), "lvamd_paged_decode_resident_waves")
        _RESIDENT[key] = found
    return found


@functools.lru_cache(maxsize=None)
def decode_tile_tokens(dtype_code: int, head_size: int, col_tiles: int = 1) -> int:
    """Tokens per decode-kernel tile for this kernel (the planner's unit)."""

    found = int(load().lvamd_paged_decode_tile_tokens(dtype_code, head_size, col_tiles))
    check(min(found, 0), "lvamd_paged_decode_tile_tokens")
    return found


def decode_split_groups(dtype_code: int, head_size: int) -> int:
    """Workgroups of the workgroup-split decode kernel the current GPU holds at once."""

    key = (dtype_code, head_size, "split")
    found = _RESIDENT.get(key)
    if found is None:
        found = int(load().lvamd_paged_decode_split_groups(dtype_code, head_size))
        check(min(found, 0), "lvamd_paged_decode_split_groups")
        _RESIDENT[key] = found
    return found


@functools.lru_cache(maxsize=None)
def decode_split_waves(dtype_code: int, head_size: int) -> int:
    """Waves per workgroup of the workgroup-split decode kernel."""

    found = int(load().lvamd_paged_decode_split_waves(dtype_code, head_size))
    check(min(found, 0), "lvamd_paged_decode_split_waves")
    return found


@functools.lru_cache(maxsize=None)
def decode_max_col_tiles(dtype_code: int, head_size: int) -> int:
    """The widest column-tile count a decode kernel is built with for this shape."""

    lib = load()
    for ctw in sorted(DECODE_COL_TILES, reverse=True):
        if lib.lvamd_paged_decode_tile_tokens(dtype_code, head_size, ctw) > 0:
            return ctw
    raise errors.ExecutionError(f"no decode kernel for dtype {dtype_code}, head size {head_size}")


@functools.lru_cache(maxsize=None)
def prefill_unit_columns(dtype_code: int, head_size: int) -> int:
    """Columns per prefill work unit, 0 when the prefill kernel does not cover the shape."""

    return int(load().lvamd_paged_prefill_unit_columns(dtype_code, head_size))


@functools.lru_cache(maxsize=None)
def prefill_key_tokens(dtype_code: int, head_size: int) -> int:
    """Keys per prefill tile (split-K key ranges start on multiples of it)."""

    found = int(load().lvamd_paged_prefill_key_tokens(dtype_code, head_size))
    check(min(found, 0), "lvamd_paged_prefill_key_tokens")
    return found


@functools.lru_cache(maxsize=None)
def xcd_count() -> int:
    """XCDs of the current GPU (each with its own L2)."""

    found = int(load().lvamd_xcd_count())
    check(min(found, 0), "lvamd_xcd_count")
    return found


def prefill_resident_units(dtype_code: int, head_size: int, waves: int = 4) -> int:
    """Prefill workgroups of ``waves`` waves the current GPU holds at once."""

    found = int(load().lvamd_paged_prefill_resident_units(dtype_code, head_size, waves))
    check(min(found, 0), "lvamd_paged_prefill_resident_units")
    return found


@functools.lru_cache(maxsize=None)
def prefill_waves_built(dtype_code: int, head_size: int, waves: int) -> bool:
    """Whether the prefill kernel is built with ``waves`` waves per workgroup."""

    return bool(load().lvamd_paged_prefill_waves_built(dtype_code, head_size, waves))


@functools.lru_cache(maxsize=1)
def attention_entry() -> int:
    """Address of ``lvamd_paged_attention``, for the host module's ``attend``
    (which calls it with plain integers)."""

    return ctypes.cast(load().lvamd_paged_attention, ctypes.c_void_p).value


def check(status: int, what: str) -> None:
    if status != 0:
        message = load().lvamd_status_string(status).decode()
        raise errors.ExecutionError(f"{what} failed: {message} (status {status})")
