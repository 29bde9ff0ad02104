"""Physical paged K/V pool on an MI355X, with HIP append, compact and block copy.

The contract is light-vllm's ``PagedKVCache`` (src/light_vllm/runtime/
execution/paged_cache.py:30-338): the config and its messages, the per-layer
layout ``[num_blocks, block_size, num_kv_heads, head_size]`` with separate K
and V tensors, ``layer`` / ``layer_spec`` / ``prepare_write`` /
``write_prepared`` / ``write`` / ``compact`` and their error messages.  The
data movement runs in the gfx950 kernels of ``liblvamd_hip.so`` (there is no
PyTorch fallback, and a cache on a non-GPU device is rejected); compact's
rules run in the native host planner, for one request or a whole step.

``hip_compact`` and ``hip_block_copy`` work on any cache object exposing the
reference's public surface (``config``, ``model_spec.layers``, ``layer(id)``),
so light-vllm's own ``PagedKVCache`` can use them unchanged.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from light_vllm_amd import errors, native
from light_vllm_amd.interfaces import AttentionLayerSpec, ModelKVCacheSpec
from light_vllm_amd.plan import Staging, current_stream

_DTYPE_CODES = {torch.float32: native.DTYPE_F32, torch.float16: native.DTYPE_F16, torch.bfloat16: native.DTYPE_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise errors.KVCacheError(f"HIP paged KV supports float32, float16 and bfloat16, not {dtype}") from exc


def _positive_int(value) -> bool:
    return type(value) is int and value > 0


@dataclass(frozen=True, slots=True)
class PagedKVCacheConfig:
    """Number and size of physical blocks, dtype and device of the pool.

    With a fixed block count the config is its own planner (``plan``)."""

    num_blocks: int
    block_size: int
    dtype: torch.dtype = torch.float32
    device: str | torch.device = "cpu"

    def __post_init__(self) -> None:
        for holds, message in (
            (_positive_int(self.num_blocks), "num_blocks must be a positive integer"),
            (_positive_int(self.block_size), "block_size must be a positive integer"),
            (self.dtype.is_floating_point, "KV cache dtype must be floating point"),
        ):
            if not holds:
                raise ValueError(message)
        object.__setattr__(self, "device", torch.device(self.device))

    def plan(self, model_spec: ModelKVCacheSpec) -> "PagedKVCacheConfig":
        return self


def kv_cache_bytes_per_block(model_spec: ModelKVCacheSpec, *, block_size: int, dtype: torch.dtype) -> int:
    """Bytes of one physical block across all layers: K and V rows of every
    layer's own kv-head shape, ``block_size`` tokens."""

    element = torch.empty((), dtype=dtype).element_size()
    row_elements = sum(spec.num_kv_heads * spec.head_size for spec in model_spec.layers)
    return 2 * row_elements * block_size * element


@dataclass(frozen=True, slots=True)
class PagedLayerCache:
    """One layer's K and V, each ``[block, offset, kv_head, head_size]``."""

    keys: Tensor
    values: Tensor


@dataclass(frozen=True, slots=True)
class PagedKVWriteMapping:
    """Physical write slots of one step, reused by every layer.

    ``slots`` holds the slots of the tokens that are written; when only some
    of the step's ``num_query_tokens`` tokens are, ``source_indices`` names
    them (token t of the update goes to ``slots[i]`` for
    ``source_indices[i] == t``)."""

    slots: Tensor
    num_query_tokens: int
    source_indices: Tensor | None = None


class _CacheState:
    """Per-cache launch state: device arrays of per-layer K and V base
    addresses grouped by row size (with their K and V addresses as ints),
    a staging ring for the index uploads, the compact workspace (grown on
    demand) and the compact kernel's inline pair limit."""

    def __init__(self, cache) -> None:
        device = cache.config.device
        groups: dict[int, list[tuple[int, int]]] = {}
        for spec in cache.model_spec.layers:
            layer = cache.layer(spec.layer_id)
            row_bytes = spec.num_kv_heads * spec.head_size * layer.keys.element_size()
            groups.setdefault(row_bytes, []).append((layer.keys.data_ptr(), layer.values.data_ptr()))
        # (row bytes, layers, [K addresses | V addresses] device table, its K
        # and V halves' addresses); the table is kept alive with its addresses.
        self.groups: list[tuple[int, int, Tensor, int, int]] = []
        for row_bytes, ptrs in groups.items():
            table = torch.tensor(ptrs, dtype=torch.int64).t().contiguous().to(device)
            self.groups.append((row_bytes, len(ptrs), table, table.data_ptr(), table.data_ptr() + 8 * len(ptrs)))
        self.inline_pairs = int(native.load().lvamd_kv_compact_inline_pairs())
        self.small_copies = int(native.load().lvamd_kv_block_copy_small_pairs())
        self.staging = Staging(device)
        self._device = device
        self._workspace: Tensor | None = None

    def workspace(self, nbytes: int) -> Tensor:
        if self._workspace is None or self._workspace.numel() < nbytes:
            self._workspace = torch.empty(nbytes, dtype=torch.uint8, device=self._device)
        return self._workspace


_CACHE_STATE: "weakref.WeakKeyDictionary[object, _CacheState]" = weakref.WeakKeyDictionary()


def _layer_pointers(cache) -> _CacheState:
    """Per-cache launch state, built on first use and dropped with the cache."""

    found = _CACHE_STATE.get(cache)
    if found is None:
        found = _CacheState(cache)
        _CACHE_STATE[cache] = found
    return found


def _require_gpu(cache) -> None:
    if cache.config.device.type != "cuda":
        raise errors.KVCacheError("the HIP paged KV path requires a GPU KV cache")


def hip_append(cache, layer_id: str, key: Tensor, value: Tensor, slots_ptr: int, num_tokens: int) -> None:
    """``flatK[slots[t]] = key[t]``, ``flatV[slots[t]] = value[t]`` on the current stream.

    ``slots_ptr`` is the device address of int64 slots, one per token
    (negative = skip), ``num_tokens`` of them.
    """

    layer = cache.layer(layer_id)
    spec = cache.layer_spec(layer_id)
    if key.stride(2) != 1 or value.stride(2) != 1:
        key = key.contiguous()
        value = value.contiguous()
    lib = native.load()
    status = lib.lvamd_kv_append(
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        layer.keys.data_ptr(), layer.values.data_ptr(),
        slots_ptr, num_tokens,
        spec.num_kv_heads, spec.head_size, dtype_code(key.dtype),
        current_stream(key.device),
    )
    native.check(status, "lvamd_kv_append")


def hip_append_rotary(cache, layer_id: str, query: Tensor, key: Tensor, value: Tensor,
                      rotary: tuple[Tensor, Tensor], slots_ptr: int, num_tokens: int) -> Tensor:
    """Rotate ``query`` and ``key`` (Qwen2's half rotation, rounded as
    apply_rotary's PyTorch path rounds it) and append: ``flatK[slots[t]] =
    rotate(key[t])``, ``flatV[slots[t]] = value[t]``; returns the rotated
    queries as a new tensor.  One kernel on the current stream.

    apply_rotary: src/light_vllm/modeling/models/_qwen2_kernels.py:205-245;
    append: src/light_vllm/runtime/execution/paged_cache.py:209-248.
    """

    spec = cache.layer_spec(layer_id)
    cosines, sines = rotary
    tokens = query.shape[0]
    for name, t in (("cosines", cosines), ("sines", sines)):
        if not isinstance(t, Tensor) or t.dim() != 2 or tuple(t.shape) != (tokens, spec.head_size):
            raise errors.KVCacheError(f"rotary {name} must have shape [{tokens}, {spec.head_size}]")
        if t.dtype != query.dtype or t.device != query.device:
            raise errors.KVCacheError(f"rotary {name} dtype and device must match the query")
    if cosines.stride(1) != 1:
        cosines = cosines.contiguous()
    if sines.stride(1) != 1:
        sines = sines.contiguous()
    if query.stride(2) != 1:
        query = query.contiguous()
    if key.stride(2) != 1 or value.stride(2) != 1:
        key = key.contiguous()
        value = value.contiguous()
    layer = cache.layer(layer_id)
    rotated = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    lib = native.load()
    status = lib.lvamd_kv_append_rotary(
        query.data_ptr(), query.stride(0), query.stride(1),
        rotated.data_ptr(), rotated.stride(0), rotated.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        cosines.data_ptr(), cosines.stride(0), sines.data_ptr(), sines.stride(0),
        layer.keys.data_ptr(), layer.values.data_ptr(), slots_ptr, num_tokens,
        spec.num_query_heads, spec.num_kv_heads, spec.head_size, dtype_code(query.dtype),
        current_stream(query.device),
    )
    native.check(status, "lvamd_kv_append_rotary")
    return rotated


# Compact rules by the native planner's code: (exception kind, message).
# The messages and the order in which the rules fire are light-vllm's
# (paged_cache.py:276-302); rule 10 is the batch rule of ``compact_many``.
_COMPACT_RULES = {
    1: ("value", "paged compact counts must be non-negative integers"),
    2: ("value", "reserved query tokens must cover every actual query"),
    3: ("value", "retained query indices must be non-negative integers"),
    4: ("value", "retained query indices must be unique"),
    5: ("kv", "retained query index exceeds the paged KV tail"),
    6: ("kv", "block table does not exactly cover the reserved query slots"),
    7: ("kv", "block table contains an invalid physical block"),
    8: ("kv", "block table aliases a physical block within one request"),
    9: ("kv", "readonly prefix blocks exceed the computed prefix"),
    10: ("kv", "compact requests of one step must not write the same slot"),
    11: ("type", "a compact request needs block_ids, num_computed_tokens, num_query_tokens, "
                 "num_reserved_query_tokens and retained_query_indices"),
}


def _compact_plan(config, requests, *, keep_equal: bool = False):
    """(moved per request, source slots, target slots) of compact requests,
    as int64 arrays; the first broken rule raises its error."""

    rule, _, moved, src, dst = native.host().compact_pairs(requests, config.num_blocks, config.block_size,
                                                           keep_equal)
    if rule:
        kind, message = _COMPACT_RULES[rule]
        if kind == "kv":
            raise errors.KVCacheError(message)
        raise (ValueError if kind == "value" else TypeError)(message)
    return np.frombuffer(moved, dtype=np.int64), np.frombuffer(src, dtype=np.int64), np.frombuffer(dst, dtype=np.int64)


def _compact_request(block_ids, **counts) -> dict:
    request = dict(counts)
    request["block_ids"] = block_ids
    return request


def compact_slots(config, block_ids: tuple[int, ...], **counts) -> tuple[tuple[int, ...], tuple[int, ...]]:
    """(source slots, target slots) of one compact request, src == dst pairs
    included: retained query i moves from logical position computed +
    retained[i] to computed + i.  Raises as ``compact`` does."""

    _, src, dst = _compact_plan(config, (_compact_request(block_ids, **counts),), keep_equal=True)
    return tuple(src.tolist()), tuple(dst.tolist())


def hip_compact(cache, block_ids: tuple[int, ...], **counts) -> int:
    """Move the retained query K/V to the contiguous formal tail of every layer.

    Returns the number of tokens whose slot changed (0 = nothing written).
    Pairs whose source equals their target are left out of the copy: such a
    slot is neither read nor written by any other pair (targets are unique and
    sources are unique), so the result is the same.
    """

    return hip_compact_many(cache, (_compact_request(block_ids, **counts),))[0]


def hip_compact_many(cache, requests) -> tuple[int, ...]:
    """``hip_compact`` for several requests of one step in a single launch.

    Each request is a dict of ``compact``'s keyword arguments with
    ``block_ids``; every request is validated by compact's rules, and the
    destinations must be unique across the batch (every source is read before
    any destination is written, as for one request).  Returns each request's
    moved-token count.
    """

    _require_gpu(cache)
    if not isinstance(requests, (list, tuple)):
        requests = tuple(requests)
    moved, src, dst = _compact_plan(cache.config, requests)
    if src.size:
        _launch_compact(cache, src, dst, moved)
    return tuple(moved.tolist())


# The longest group the one-pass compact takes: one thread moves its group's
# rows one batch of 16 after another, so a long group would serialise.
ORDERED_MAX_PAIRS = 64


def ordered_groups(moved: np.ndarray, src: np.ndarray, dst: np.ndarray) -> np.ndarray | None:
    """Group boundaries (int64, one group per request that moves anything)
    when the pairs may be moved in place in one pass, else None.

    The pass moves each group's pairs in order while the groups run side by
    side, so it is exact when every row that some pair writes is read only
    by earlier pairs of the same group: a destination equal to a source
    ``src[j]`` must be ``dst[i]`` with ``i > j`` in ``j``'s group.  Every
    request whose retained indices are strictly increasing (an accepted
    root-to-leaf path) meets this on its own rows: pair ``j`` reads position
    ``computed + retained[j]`` and writes ``computed + j``, and
    ``retained[j] >= j``.  Destinations are unique (compact's rules).
    """

    counts = moved[moved > 0]
    if counts.size == 0 or int(counts.max()) > ORDERED_MAX_PAIRS:
        return None
    starts = np.zeros(counts.size + 1, dtype=np.int64)
    np.cumsum(counts, out=starts[1:])
    order = np.argsort(dst, kind="stable")
    sorted_dst = dst[order]
    k = np.searchsorted(sorted_dst, src)
    k[k == sorted_dst.size] = 0
    hit = sorted_dst[k] == src
    if hit.any():
        reader = np.flatnonzero(hit)
        writer = order[k[hit]]
        group = np.repeat(np.arange(counts.size), counts)
        if np.any(writer <= reader) or np.any(group[writer] != group[reader]):
            return None
    return starts


def _launch_compact(cache, src: np.ndarray, dst: np.ndarray, moved: np.ndarray | None = None) -> None:
    pointers = _layer_pointers(cache)
    device = cache.config.device
    n = int(src.size)
    lib = native.load()
    stream = current_stream(device)
    if n <= pointers.inline_pairs:
        # A few pairs (a step's accepted tokens) ride in the kernel arguments.
        src = np.ascontiguousarray(src, dtype=np.int64)
        dst = np.ascontiguousarray(dst, dtype=np.int64)
        for row_bytes, num_layers, _, kptrs, vptrs in pointers.groups:
            native.check(lib.lvamd_kv_compact_small(kptrs, vptrs, num_layers, row_bytes, src.ctypes.data,
                                                    dst.ctypes.data, n, stream), "lvamd_kv_compact_small")
        return
    starts = ordered_groups(moved, src, dst) if moved is not None else None
    if starts is not None:
        # One pass, in place: [src | dst | group starts] in one upload.
        g = int(starts.size) - 1
        buf = pointers.staging.take(4 * n + 2 * (g + 1))
        buf[: 2 * n] = src.view(np.int32)
        buf[2 * n : 4 * n] = dst.view(np.int32)
        buf[4 * n : 4 * n + 2 * (g + 1)] = starts.view(np.int32)
        blob = pointers.staging.upload(buf[: 4 * n + 2 * (g + 1)])
        src_ptr = blob.data_ptr()
        for row_bytes, num_layers, _, kptrs, vptrs in pointers.groups:
            native.check(lib.lvamd_kv_compact_ordered(kptrs, vptrs, num_layers, row_bytes, src_ptr,
                                                      src_ptr + 8 * n, src_ptr + 16 * n, g, stream),
                         "lvamd_kv_compact_ordered")
        return
    # [src | dst] as int64 pairs of int32 words, in one pinned buffer and copy.
    buf = pointers.staging.take(4 * n)
    buf[: 2 * n] = src.view(np.int32)
    buf[2 * n : 4 * n] = dst.view(np.int32)
    blob = pointers.staging.upload(buf[: 4 * n])
    src_ptr = blob.data_ptr()
    dst_ptr = src_ptr + 8 * n
    for row_bytes, num_layers, _, kptrs, vptrs in pointers.groups:
        ws_bytes = lib.lvamd_kv_compact_workspace_size(n, num_layers, row_bytes)
        workspace = pointers.workspace(ws_bytes) if ws_bytes else None
        status = lib.lvamd_kv_compact(
            kptrs, vptrs, num_layers, row_bytes,
            src_ptr, dst_ptr, n, workspace.data_ptr() if workspace is not None else None, ws_bytes, stream,
        )
        native.check(status, "lvamd_kv_compact")


def hip_block_copy(cache, src_blocks, dst_blocks) -> None:
    """Copy-on-write: block ``dst_blocks[i]`` of every layer becomes a copy of ``src_blocks[i]``.

    No light-vllm counterpart (its prefix cache shares only complete read-only
    pages).  Sources and destinations must be disjoint and destinations unique.
    """

    _require_gpu(cache)
    src = tuple(src_blocks)
    dst = tuple(dst_blocks)
    if len(src) != len(dst):
        raise ValueError("block copy needs one destination per source")
    num_blocks = cache.config.num_blocks
    both = src + dst
    if both and (set(map(type, both)) != {int} or min(both) < 0 or max(both) >= num_blocks):
        raise errors.KVCacheError("block copy names an invalid physical block")
    if len(set(dst)) != len(dst):
        raise errors.KVCacheError("block copy writes the same physical block twice")
    if set(src) & set(dst):
        raise errors.KVCacheError("block copy sources and destinations must be disjoint")
    if not src:
        return
    pointers = _layer_pointers(cache)
    lib = native.load()
    stream = current_stream(cache.config.device)
    bs = cache.config.block_size
    if len(src) <= pointers.small_copies:
        # A step's few copies ride in the kernel arguments.
        src_a = np.asarray(src, dtype=np.int64)
        dst_a = np.asarray(dst, dtype=np.int64)
        for row_bytes, num_layers, _, kptrs, vptrs in pointers.groups:
            native.check(lib.lvamd_kv_block_copy_small(kptrs, vptrs, num_layers, row_bytes * bs, src_a.ctypes.data,
                                                       dst_a.ctypes.data, len(src), stream),
                         "lvamd_kv_block_copy_small")
        return
    blob, (src_off, dst_off) = pointers.staging.stage([np.asarray(src, dtype=np.int64).view(np.int32),
                                                       np.asarray(dst, dtype=np.int64).view(np.int32)])
    for row_bytes, num_layers, _, kptrs, vptrs in pointers.groups:
        status = lib.lvamd_kv_block_copy(
            kptrs, vptrs, num_layers, row_bytes * bs,
            blob.data_ptr() + 4 * src_off, blob.data_ptr() + 4 * dst_off, len(src), stream,
        )
        native.check(status, "lvamd_kv_block_copy")


class PagedKVCache:
    """Per-layer K/V pools shared by all requests, addressed by block id."""

    def __init__(self, model_spec: ModelKVCacheSpec, config: PagedKVCacheConfig) -> None:
        if config.device.type != "cuda":
            raise errors.KVCacheError("the HIP paged KV cache requires a GPU (cuda) device")
        dtype_code(config.dtype)
        self._model_spec = model_spec
        self._config = config
        self._layer_specs = {layer.layer_id: layer for layer in model_spec.layers}
        self._layers = {layer.layer_id: self._allocate_layer(layer) for layer in model_spec.layers}

    @property
    def config(self) -> PagedKVCacheConfig:
        return self._config

    @property
    def model_spec(self) -> ModelKVCacheSpec:
        return self._model_spec

    def layer_spec(self, layer_id: str) -> AttentionLayerSpec:
        try:
            return self._layer_specs[layer_id]
        except KeyError as exc:
            raise errors.KVCacheError(f"KV cache layer {layer_id!r} was not found") from exc

    def layer(self, layer_id: str) -> PagedLayerCache:
        try:
            return self._layers[layer_id]
        except KeyError as exc:
            raise errors.KVCacheError(f"KV cache layer {layer_id!r} was not found") from exc

    @torch.inference_mode()
    def prepare_write(self, slot_mapping: Tensor, *, validate: bool = True) -> PagedKVWriteMapping:
        """One step's slot mapping, normalised once for every layer's write
        (light-vllm: paged_cache.py:165-206).

        Negative entries mark tokens that are not written.  With ``validate``
        the written slots are checked in range and distinct, from one host
        copy of the mapping; metadata-proven mappings pass ``validate=False``
        and stay on the device untouched.
        """

        if slot_mapping.ndim != 1:
            raise errors.KVCacheError("slot mapping must have one entry per packed query token")
        if slot_mapping.device != self._config.device:
            raise errors.KVCacheError("slot mapping device must match the cache")
        num_tokens = slot_mapping.numel()
        if not validate:
            return PagedKVWriteMapping(slots=slot_mapping.to(torch.long), num_query_tokens=num_tokens)
        host = slot_mapping.to("cpu", torch.long).numpy()
        written = np.flatnonzero(host >= 0)
        chosen = host[written]
        if chosen.size:
            if int(chosen.max()) >= self._config.num_blocks * self._config.block_size:
                raise errors.KVCacheError("slot mapping contains an out-of-range physical slot")
            if np.unique(chosen).size != chosen.size:
                raise errors.KVCacheError("slot mapping must not write the same physical slot twice")
        device = self._config.device
        every = written.size == num_tokens
        return PagedKVWriteMapping(
            slots=torch.from_numpy(chosen).to(device),
            num_query_tokens=num_tokens,
            source_indices=None if every else torch.from_numpy(written).to(device),
        )

    @torch.inference_mode()
    def write_prepared(self, layer_id: str, key: Tensor, value: Tensor, mapping: PagedKVWriteMapping) -> None:
        """Write one layer's K/V through a prepared mapping (light-vllm:
        paged_cache.py:209-248) with the HIP append kernel, which takes one
        slot per token and skips negative ones."""

        self.layer(layer_id)
        spec = self.layer_spec(layer_id)
        cfg = self._config
        tail = (spec.num_kv_heads, spec.head_size)
        rules = (
            (lambda: key.ndim == 3 and tuple(key.shape[1:]) == tail,
             "paged KV update must have shape [tokens, kv_heads, head_size]"),
            (lambda: value.shape == key.shape, "paged K/V updates must have the same shape"),
            (lambda: mapping.num_query_tokens == key.shape[0], "slot mapping must have one entry per query token"),
            (lambda: key.dtype == cfg.dtype and key.device == cfg.device,
             "paged KV update dtype and device must match the cache"),
            (lambda: value.dtype == key.dtype and value.device == key.device,
             "paged K/V updates must use the same dtype and device"),
            (lambda: mapping.slots.device == cfg.device
             and (mapping.source_indices is None or mapping.source_indices.device == cfg.device),
             "prepared slot mapping device must match the cache"),
        )
        for holds, message in rules:
            if not holds():
                raise errors.KVCacheError(message)
        if mapping.slots.numel() == 0:
            return
        per_token = mapping.slots
        if mapping.source_indices is not None:
            per_token = torch.full((mapping.num_query_tokens,), -1, dtype=torch.long, device=cfg.device)
            per_token[mapping.source_indices] = mapping.slots
        per_token = per_token.contiguous()
        hip_append(self, layer_id, key, value, per_token.data_ptr(), per_token.numel())

    @torch.inference_mode()
    def write(self, layer_id: str, key: Tensor, value: Tensor, slot_mapping: Tensor) -> None:
        """Write the active tokens' K/V to their physical slots."""

        self.write_prepared(layer_id, key, value, self.prepare_write(slot_mapping))

    @torch.inference_mode()
    def compact(
        self,
        block_ids: tuple[int, ...],
        *,
        num_computed_tokens: int,
        num_query_tokens: int,
        num_reserved_query_tokens: int,
        retained_query_indices: tuple[int, ...],
        num_readonly_prefix_blocks: int = 0,
    ) -> int:
        """Move the accepted path to the contiguous formal tail of every layer
        (light-vllm: paged_cache.py:257-326); returns how many tokens moved."""

        return hip_compact(self, block_ids, num_computed_tokens=num_computed_tokens,
                           num_query_tokens=num_query_tokens, num_reserved_query_tokens=num_reserved_query_tokens,
                           retained_query_indices=retained_query_indices,
                           num_readonly_prefix_blocks=num_readonly_prefix_blocks)

    @torch.inference_mode()
    def compact_many(self, requests) -> tuple[int, ...]:
        """``compact`` for every request of a step in one launch (one dict of
        ``compact``'s arguments, with ``block_ids``, per request)."""

        return hip_compact_many(self, requests)

    @torch.inference_mode()
    def copy_blocks(self, src_blocks, dst_blocks) -> None:
        """Copy-on-write of whole blocks across every layer (no reference counterpart)."""

        hip_block_copy(self, src_blocks, dst_blocks)

    def _allocate_layer(self, spec: AttentionLayerSpec) -> PagedLayerCache:
        shape = (self._config.num_blocks, self._config.block_size, spec.num_kv_heads, spec.head_size)
        return PagedLayerCache(
            keys=torch.empty(shape, dtype=self._config.dtype, device=self._config.device),
            values=torch.empty(shape, dtype=self._config.dtype, device=self._config.device),
        )
