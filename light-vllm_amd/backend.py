"""The HIP paged-attention backend: ``create(cache, metadata) -> context``.

Drop-in for light-vllm's ``PagedAttentionBackend`` protocol
(src/light_vllm/runtime/execution/paged_attention.py:209-223).  A context is
created once per model step by ``PagedStepHandler.forward``
(src/light_vllm/runtime/execution/worker.py:286) and its ``forward`` is called
once per layer by the model (src/light_vllm/modeling/models/qwen2.py:417-423).

``create`` proves the step's block tables (light-vllm's rules and messages),
and builds the step plan for every layer shape of the cache in the native host
planner: slots, per-request records, flat tables, ancestor rows and the
decode / prefill work lists go to the GPU in one non-blocking copy.

``forward``:
1. validates shapes exactly as ``_validate_paged_attention_tensors``
   (paged_attention.py:226-247) plus the dtype/device rule of the Triton
   backend (triton_paged_attention.py:475-478);
2. attends with write-before-attend semantics: the stream-K decode kernel
   (short query runs) and the MFMA prefill kernel (long ones) read this
   step's K/V from the inputs and append their own requests' tokens to their
   pool slots themselves, and a merge kernel combines split partials; with
   ``rotary=`` one rotary-append launch writes the pool first.  Everything is on the current stream with no host
   synchronisation.
"""

from __future__ import annotations

import ctypes
import weakref

import torch
from torch import Tensor

from light_vllm_amd import errors, native
from light_vllm_amd.metadata import PagedAttentionMetadata
from light_vllm_amd.paged_cache import current_stream, dtype_code, hip_append_rotary
from light_vllm_amd.plan import (
    DECODE_MAX_COLUMNS, DECODE_MIN_UNITS_PER_WAVE, PREFILL_MIN_TILES, UNIT_TOKENS, LayerShapes, Staging, StepPlan,
)

# Head sizes the kernels are built for: multiples of 16 from 32 to 256.
SUPPORTED_HEAD_SIZES = tuple(range(32, 257, 16))


def validate_paged_attention_tensors(cache, metadata, layer_id: str, query: Tensor, key: Tensor, value: Tensor):
    """Shape checks shared by every backend (paged_attention.py:226-247).

    ``metadata`` is anything with ``num_query_tokens``: the step's
    ``PagedAttentionMetadata`` or its ``StepPlan`` (which holds the count).
    """

    layer_spec = cache.layer_spec(layer_id)
    rules = (
        (lambda: query.ndim == 3, "paged attention query must have three dimensions"),
        (lambda: query.shape[0] == key.shape[0] and value.shape == key.shape,
         "paged attention Q/K/V token dimensions must match"),
        (lambda: query.shape[0] == metadata.num_query_tokens,
         "paged attention metadata token count does not match query"),
        (lambda: tuple(query.shape[1:]) == (layer_spec.num_query_heads, layer_spec.head_size),
         "paged attention query shape does not match the layer spec"),
        (lambda: tuple(key.shape[1:]) == (layer_spec.num_kv_heads, layer_spec.head_size),
         "paged attention K/V shape does not match the layer spec"),
    )
    for holds, message in rules:
        if not holds():
            raise errors.KVCacheError(message)
    return layer_spec


class _Workspace:
    """Split-K partials, grown on demand and reused by every layer and step.

    Layers run in stream order on one stream, so one buffer serves them all.
    A buffer grows at least twofold, and the replaced ones stay allocated (a
    context created before the growth may still launch with their
    addresses), so together they hold less than the current one.
    """

    def __init__(self) -> None:
        self._buffer: Tensor | None = None
        self._retired: list[Tensor] = []

    def get(self, num_bytes: int, device: torch.device) -> Tensor:
        if self._buffer is None or self._buffer.numel() < num_bytes or self._buffer.device != device:
            if self._buffer is not None:
                self._retired.append(self._buffer)
            size = max(num_bytes, 2 * self._buffer.numel() if self._buffer is not None else 0, 1)
            self._buffer = torch.empty(size, dtype=torch.uint8, device=device)
        return self._buffer

    def ptr(self) -> int | None:
        return None if self._buffer is None else self._buffer.data_ptr()


def _rows_aligned(t: Tensor) -> bool:
    """Rows of 16-byte chunks: contiguous last dim, 16-byte aligned base and strides."""

    es = t.element_size()
    return t.stride(2) == 1 and t.data_ptr() % 16 == 0 and (t.stride(0) * es) % 16 == 0 and (
        t.stride(1) * es
    ) % 16 == 0


def _partial_layout(work, spec, prefill_columns: int, element_size: int) -> tuple[int, int, int, int]:
    """Byte sizes of a layer shape's split-K partials: (decode rows, decode
    (max, sum) pairs, prefill rows, prefill pairs).  A row is one column's
    normalised output in the pool's element type, a pair two fp32; every
    size is a multiple of 16 bytes (columns come in tiles of 16)."""

    dec = work.num_partial_slots * spec.num_kv_heads * 16 * work.col_tiles
    pre = work.num_prefill_partial_slots * spec.num_kv_heads * prefill_columns
    return dec * spec.head_size * element_size, dec * 8, pre * spec.head_size * element_size, pre * 8


class _LayerLaunch:
    """Launch facts shared by every layer of one shape in one step plan.

    Holds every kernel argument that does not depend on the layer's tensors,
    as argument tuples of the single-kernel entry points and as one
    ``lvamd_attention_plan`` (``plan_ptr``) for ``lvamd_paged_attention``, so
    a layer's ``forward`` only reads tensor pointers and strides.
    """

    __slots__ = ("work", "dtype", "decode_args", "merge_args", "prefill_args", "prefill_merge_args",
                 "workspace_ptr", "plan", "plan_ptr")

    def __init__(self, plan: StepPlan, work, spec, dtype: int, block_size: int, workspace_ptr: int | None,
                 prefill_columns: int, sizes: tuple[int, int, int, int]) -> None:
        group = spec.num_query_heads // spec.num_kv_heads
        self.work = work
        self.dtype = dtype
        self.workspace_ptr = workspace_ptr
        self.decode_args = self.merge_args = self.prefill_args = self.prefill_merge_args = None
        dec_rows, dec_pairs, pre_rows, pre_pairs = sizes
        part_acc = part_ml = pre_acc = pre_ml = None
        if dec_rows:
            part_acc = workspace_ptr
            part_ml = part_acc + dec_rows
        if pre_rows:
            pre_acc = workspace_ptr + dec_rows + dec_pairs
            pre_ml = pre_acc + pre_rows
        if work.waves_per_head:
            # lvamd_paged_decode arguments after the output strides, up to the scale.
            self.decode_args = (
                work.pieces_ptr, work.wave_first_ptr, work.waves_per_head, plan.tables_ptr, plan.vis_ptr,
                part_acc, part_ml, work.num_partial_slots,
                spec.num_kv_heads, group, spec.head_size, work.col_tiles, work.group_waves, block_size,
            )
        if work.num_jobs:
            # lvamd_paged_attention_merge arguments after the output strides, up to the stream.
            self.merge_args = (part_acc, part_ml) + (
                work.jobs_ptr, work.num_jobs, spec.num_kv_heads, group, spec.head_size, work.col_tiles,
                work.merge_columns, dtype,
            )
        if work.num_prefill_units:
            # lvamd_paged_prefill arguments after the output strides, up to the scale.
            self.prefill_args = (
                plan.tables_ptr, plan.vis_ptr, work.units_ptr, work.num_prefill_units,
                pre_acc, pre_ml, work.num_prefill_partial_slots,
                spec.num_kv_heads, group, spec.head_size, work.prefill_waves, block_size,
            )
        if work.num_prefill_jobs:
            self.prefill_merge_args = (pre_acc, pre_ml) + (
                work.prefill_jobs_ptr, work.num_prefill_jobs, spec.num_kv_heads, group, spec.head_size,
                prefill_columns // 16, work.prefill_merge_columns, dtype,
            )
        p = self.plan = native.AttentionPlan(
            pieces=work.pieces_ptr, wave_first=work.wave_first_ptr, waves_per_head=work.waves_per_head,
            col_tiles=work.col_tiles, part_acc=part_acc, part_ml=part_ml, num_partial_slots=work.num_partial_slots,
            jobs=work.jobs_ptr, num_jobs=work.num_jobs, merge_columns=work.merge_columns,
            group_waves=work.group_waves,
            units=work.units_ptr, num_units=work.num_prefill_units, prefill_waves=work.prefill_waves,
            prefill_part_acc=pre_acc, prefill_part_ml=pre_ml,
            num_prefill_partial_slots=work.num_prefill_partial_slots, prefill_jobs=work.prefill_jobs_ptr,
            num_prefill_jobs=work.num_prefill_jobs, prefill_merge_columns=work.prefill_merge_columns,
            prefill_col_tiles=max(prefill_columns // 16, 1), num_kv_heads=spec.num_kv_heads,
            tables=plan.tables_ptr, vis=plan.vis_ptr, group=group, head_size=spec.head_size, block_size=block_size,
            dtype=dtype,
        )
        self.plan_ptr = ctypes.addressof(p)


class _LayerStatic:
    """What the fast ``forward`` needs of one layer that stays fixed for a
    cache: its spec, shape key and place among the layers of that shape,
    pool addresses, dtype and device.  Built once per (backend, cache)."""

    __slots__ = ("spec", "shape", "index", "k_pool", "v_pool", "dtype", "device", "device_index", "element_size")

    def __init__(self, spec, index: int, layer, config, device_index: int) -> None:
        self.spec = spec
        self.shape = (spec.num_query_heads, spec.num_kv_heads, spec.head_size)
        self.index = index
        self.k_pool = layer.keys.data_ptr()
        self.v_pool = layer.values.data_ptr()
        self.dtype = config.dtype
        self.device = config.device
        self.device_index = device_index
        self.element_size = config.dtype.itemsize


_NOT_FAST = 1 << 30  # attend_tensors: a tensor rule of the fast path does not hold
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_NO_APPEND = (None, 0, 0, None, 0, 0)
# Per-XCD prefill order policies (the planner's kernel fact).
PREFILL_ORDERS = {"auto": 0, "grouped": 1, "plain": 2}


class HipPagedAttention:
    """Per-step context: writes each layer's K/V, then runs paged attention."""

    # forward accepts rotary=(cosines, sines): RoPE is applied inside the append.
    supports_rotary = True

    def __init__(self, backend: "HipPagedAttentionBackend", cache, plan: StepPlan) -> None:
        self._backend = backend
        self._cache = cache
        self._config = cache.config
        self._layer_ids: set[str] = set()
        self._plan = plan
        self._lib = backend._lib
        # The fast forward's facts: per layer the cache's fixed ones (pools,
        # shape, place among the layers of its shape), per layer shape this
        # step's (bound plan, output slab), bound at the shape's first layer.
        self._statics = backend.layer_statics(cache) if _raw_stream is not None else {}
        self._shape_bound: dict[tuple, tuple] = {}
        self._attend_tensors = backend._attend_tensors
        self._attend_fn = backend._attend_fn

    @property
    def layer_ids(self) -> frozenset[str]:
        return frozenset(self._layer_ids)

    @property
    def plan(self) -> StepPlan:
        return self._plan

    def forward(self, layer_id: str, query: Tensor, key: Tensor, value: Tensor, *, scale: float,
                rotary: tuple[Tensor, Tensor] | None = None) -> Tensor:
        """Append this layer's K/V, then attend (paged_attention.py:268-380).

        ``rotary=(cosines, sines)`` ([tokens, head_size] rows in the cache
        dtype, as Qwen2's ``_rotary_embeddings`` returns them) takes unrotated
        ``query``/``key`` and applies ``apply_rotary``'s half rotation
        (_qwen2_kernels.py:205-245) inside the append: one launch rotates the
        queries and writes the rotated keys and the values to their slots.
        The result equals ``apply_rotary`` followed by ``forward``.
        """

        if layer_id in self._layer_ids:
            raise errors.KVCacheError(f"paged attention layer {layer_id!r} ran more than once")
        self._layer_ids.add(layer_id)
        # The common case in one native call (the host module's
        # attend_tensors): it reads the tensors' dtype, device, shapes,
        # strides and pointers, and launches when every rule holds (the
        # layer's shapes, dtype and device, 16-byte rows); anything else, and
        # rotary, takes the general path, which raises the first broken
        # rule's message.
        static = self._statics.get(layer_id)
        if static is not None and rotary is None:
            bound = self._shape_bound.get(static.shape)
            if bound is None:
                bound = self._bind_shape(static)
            index = static.index
            status = self._attend_tensors(bound[0], static.k_pool, static.v_pool, bound[1] + index * bound[2],
                                          query, key, value, scale)
            if status == 0:
                return bound[3][index]
            if status != _NOT_FAST:
                native.check(status, "lvamd_paged_attention")
        return self._forward_general(layer_id, query, key, value, scale=scale, rotary=rotary)

    def _bind_shape(self, static) -> tuple:
        """The fast path's facts for the layers of one shape in this step:
        (the shape's facts for attend_tensors, the output slab's address,
        its bytes per layer, the per-layer output views).

        Outputs are views of one tensor per layer shape and step, made at the
        first layer of that shape (one allocation for the step's layers in
        place of one per layer); each layer's view is its own rows.  The
        bound launch stays alive with the context."""

        spec = static.spec
        launch = self._launch(spec)
        tokens = self._plan.num_tokens
        count = self._backend.shape_counts(self._cache)[static.shape]
        if count == 1:
            # One layer of this shape: its output is the slab (no views).
            slab = torch.empty((tokens, spec.num_query_heads, spec.head_size), dtype=static.dtype,
                               device=static.device)
            views = (slab,)
        else:
            slab = torch.empty((count, tokens, spec.num_query_heads, spec.head_size), dtype=static.dtype,
                               device=static.device)
            views = slab.unbind(0)
        facts = (
            self._attend_fn, launch.plan_ptr, spec.num_query_heads * spec.head_size, spec.head_size, static.dtype,
            static.device_index, static.element_size, tokens, spec.num_query_heads, spec.num_kv_heads,
            spec.head_size, _raw_stream,
        )
        bound = (facts, slab.data_ptr(), tokens * spec.num_query_heads * spec.head_size * static.element_size,
                 views, launch)
        self._shape_bound[static.shape] = bound
        return bound

    def _forward_general(self, layer_id: str, query: Tensor, key: Tensor, value: Tensor, *, scale: float,
                         rotary: tuple[Tensor, Tensor] | None) -> Tensor:
        """Every rule in the reference's order, then the launches for any
        row strides and for ``rotary``."""

        spec = validate_paged_attention_tensors(self._cache, self._plan, layer_id, query, key, value)
        config = self._config
        if query.device != config.device or query.dtype != config.dtype:
            raise errors.KVCacheError("HIP paged attention query dtype and device must match the KV cache")
        if key.dtype != config.dtype or value.dtype != config.dtype or key.device != config.device or (
            value.device != config.device
        ):
            raise errors.KVCacheError("paged KV update dtype and device must match the cache")
        if spec.head_size not in SUPPORTED_HEAD_SIZES:
            raise errors.KVCacheError(
                f"HIP paged attention supports head sizes {SUPPORTED_HEAD_SIZES}, not {spec.head_size}"
            )

        if not _rows_aligned(query):
            query = query.contiguous()
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
        launch = self._launch(spec)
        layer = self._cache.layer(layer_id)
        stream = current_stream(query.device)
        lib = self._lib
        plan = self._plan
        if rotary is not None:
            # The rotated queries go to a fresh buffer and the pool receives
            # the whole step's rotated K and V, so attention reads the pool.
            query = hip_append_rotary(self._cache, layer_id, query, key, value, rotary, plan.slots_ptr,
                                      plan.num_tokens)
            new_kv = _NO_APPEND
        else:
            # The decode and prefill kernels append their own requests'
            # tokens (fused append): they read this step's keys and values
            # from the inputs and write each token's row to its slot.
            if not _rows_aligned(key):
                key = key.contiguous()
            if not _rows_aligned(value):
                value = value.contiguous()
            new_kv = (key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0), value.stride(1))
        native.check(lib.lvamd_paged_attention(
            launch.plan_ptr, query.data_ptr(), query.stride(0), query.stride(1), *new_kv,
            layer.keys.data_ptr(), layer.values.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
            float(scale), stream,
        ), "lvamd_paged_attention")
        return out

    def decode_launch(
        self, layer_id: str, query: Tensor, out: Tensor, *, scale: float, key: Tensor | None = None,
        value: Tensor | None = None,
    ) -> "_DecodeLaunch | None":
        """The bound decode and merge launches of this layer (None if it has no decode rows).

        With ``key``/``value`` the launch also appends them (fused append);
        without, the pool must already hold this step's K/V.
        """

        launch = self._launch(self._cache.layer_spec(layer_id))
        if launch.decode_args is None:
            return None
        return _DecodeLaunch(self._lib, launch, self._cache.layer(layer_id), query, key, value, out, float(scale))

    def prefill(self, layer_id: str, query: Tensor, out: Tensor, *, scale: float) -> None:
        """Only the prefill kernel of this layer (the pool must hold the step's K/V)."""

        launch = self._launch(self._cache.layer_spec(layer_id))
        if launch.prefill_args is None:
            return
        layer = self._cache.layer(layer_id)
        stream = current_stream(query.device)
        o_args = (out.data_ptr(), out.stride(0), out.stride(1))
        native.check(self._lib.lvamd_paged_prefill(
            query.data_ptr(), query.stride(0), query.stride(1), *_NO_APPEND,
            layer.keys.data_ptr(), layer.values.data_ptr(), *o_args,
            *launch.prefill_args, float(scale), launch.dtype, stream,
        ), "lvamd_paged_prefill")
        if launch.prefill_merge_args is not None:
            m = launch.prefill_merge_args
            native.check(self._lib.lvamd_paged_attention_merge(m[0], m[1], *o_args, *m[2:], stream),
                         "lvamd_paged_attention_merge")

    def work_of(self, spec):
        """The work lists this step runs for layers of ``spec``'s shape."""

        return self._launch(spec).work

    def _launch(self, spec) -> _LayerLaunch:
        """The launch facts of this layer shape, bound once per plan."""

        backend = self._backend
        code = dtype_code(self._config.dtype)
        key = (spec.num_query_heads, spec.num_kv_heads, spec.head_size, code)
        plan = self._plan
        found = plan.launches.get(key)
        if found is not None and found.workspace_ptr is not None and found.workspace_ptr != backend.workspace.ptr():
            found = None  # the workspace (shared by all plans) was regrown since
        if found is None:
            work = plan.layer_work(backend.kernel_facts(spec, code, self._config.block_size))
            columns = backend.prefill_columns(code, spec.head_size)
            sizes = _partial_layout(work, spec, columns, self._config.dtype.itemsize)
            ptr = None
            if sum(sizes):
                ptr = backend.workspace.get(sum(sizes), self._config.device).data_ptr()
            found = _LayerLaunch(plan, work, spec, code, self._config.block_size, ptr, columns, sizes)
            plan.launches[key] = found
        return found


class _DecodeLaunch:
    """The decode and merge kernel launches of one layer, with bound arguments."""

    def __init__(self, lib, launch: _LayerLaunch, layer, query, key, value, out, scale) -> None:
        self.work = launch.work
        stream = current_stream(query.device)
        self._lib = lib
        if key is None:
            new_kv = _NO_APPEND
        else:
            new_kv = (key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0), value.stride(1))
        o_args = (out.data_ptr(), out.stride(0), out.stride(1))
        self._decode_args = (
            query.data_ptr(), query.stride(0), query.stride(1), *new_kv,
            layer.keys.data_ptr(), layer.values.data_ptr(), *o_args,
            *launch.decode_args, scale, launch.dtype, stream,
        )
        self._merge_args = None
        if launch.merge_args is not None:
            m = launch.merge_args
            self._merge_args = (m[0], m[1], *o_args, *m[2:], stream)

    def decode(self) -> None:
        native.check(self._lib.lvamd_paged_decode(*self._decode_args), "lvamd_paged_decode")

    def merge(self) -> None:
        if self._merge_args is not None:
            native.check(self._lib.lvamd_paged_attention_merge(*self._merge_args), "lvamd_paged_attention_merge")


class HipPagedAttentionBackend:
    """Creates one ``HipPagedAttention`` per model step.

    Construction fails with ``ExecutionNotReadyError`` when the HIP library or
    the host planner is missing, like the Triton backend without Triton
    (triton_paged_attention.py:566-570).  The step plan of the most recent
    metadata object is kept: metadata objects are immutable, so a second
    ``create`` with the same object (and a cache of the same geometry) reuses
    the validated, staged plan.  This package's metadata is recognised by its
    facts (the metadata object itself is not kept alive).
    """

    def __init__(
        self, *, use_prefill_kernel: bool = True, partition_tokens: int | None = None,
        decode_col_tiles: int | None = None, split_prefill: bool = True, prefill_waves: int | None = None,
        shared_prefix: bool = True, prefill_order: str = "auto", decode_workgroups: bool = True,
    ) -> None:
        """``use_prefill_kernel=False`` sends every request through the decode
        kernel; ``partition_tokens`` caps the tokens one decode wave handles (a
        tuning knob; by default the planner spreads the work over every
        resident wave); ``decode_col_tiles`` (1 or 4) fixes the decode kernel's
        column tiles per wave instead of the planner's per-step choice;
        ``split_prefill=False`` keeps every prefill unit's keys in one
        workgroup (no split-K partials); ``prefill_waves`` (4 or 8) fixes the
        prefill workgroup shape instead of the planner's per-step choice (8
        falls back to 4 where it is not built); ``shared_prefix=False`` turns
        off the shared-prefix spans (every prefill request then streams its
        whole prefix itself); ``prefill_order`` places each request's prefill
        units on one XCD (so they share its L2): ``"auto"`` when the
        planner's simulated packing of the resident workgroups is no slower,
        ``"grouped"`` always, ``"plain"`` never (heaviest first only);
        ``decode_workgroups=False`` keeps every decode step on stream-K
        shares (by default a latency-bound step, whose segments fit the
        resident workgroups, runs one segment per workgroup of eight waves,
        four for the widest rows, that combine their results in LDS, with no
        merge launch)."""

        native.load()
        native.host()
        if partition_tokens is not None and (partition_tokens <= 0 or partition_tokens % UNIT_TOKENS):
            raise ValueError(f"partition_tokens must be a positive multiple of {UNIT_TOKENS}")
        if decode_col_tiles is not None and decode_col_tiles not in native.DECODE_COL_TILES:
            raise ValueError(f"decode_col_tiles must be one of {native.DECODE_COL_TILES}")
        if prefill_waves not in (None, 4, 8):
            raise ValueError("prefill_waves must be 4 or 8")
        if prefill_order not in PREFILL_ORDERS:
            raise ValueError(f"prefill_order must be one of {tuple(PREFILL_ORDERS)}")
        self.workspace = _Workspace()
        self._use_prefill = use_prefill_kernel
        self._partition_tokens = partition_tokens
        self._col_tiles = decode_col_tiles
        self._split_prefill = split_prefill
        self._shared_prefix = shared_prefix
        self._prefill_waves = prefill_waves
        self._prefill_order = PREFILL_ORDERS[prefill_order]
        self._decode_workgroups = bool(decode_workgroups)
        self._staging: dict[torch.device, Staging] = {}
        self._facts: dict[tuple, tuple[int, ...]] = {}
        # cache -> kernel facts of its layer shapes (dropped with the cache).
        self._shapes: "weakref.WeakKeyDictionary[object, LayerShapes]" = weakref.WeakKeyDictionary()
        self._head_sizes_ok: "weakref.WeakSet[object]" = weakref.WeakSet()
        self._statics: "weakref.WeakKeyDictionary[object, dict]" = weakref.WeakKeyDictionary()
        self._shape_counts: "weakref.WeakKeyDictionary[object, dict]" = weakref.WeakKeyDictionary()
        # (geometry, metadata key, plan, weak reference to the cache) of the
        # most recent create().
        self._last: tuple[object, object, StepPlan, weakref.ref] | None = None
        # What every context's fast forward calls, looked up once.
        self._lib = native.load()
        self._attend_tensors = native.host().attend_tensors
        self._attend_fn = native.attention_entry()

    def prefill_columns(self, code: int, head_size: int) -> int:
        return native.prefill_unit_columns(code, head_size) if self._use_prefill else 0

    def kernel_facts(self, spec, code: int, block_size: int) -> tuple[int, ...]:
        """The library's figures for this layer shape (``plan.KERNEL_FACTS``
        order), queried once per shape and device."""

        key = (spec.num_query_heads, spec.num_kv_heads, spec.head_size, code, block_size, torch.cuda.current_device())
        found = self._facts.get(key)
        if found is None:
            d = spec.head_size
            group = spec.num_query_heads // spec.num_kv_heads
            columns = self.prefill_columns(code, d)
            max_ctw = native.decode_max_col_tiles(code, d)
            has4 = max_ctw >= 4
            key_tokens = native.prefill_key_tokens(code, d) if columns else 0
            wide = bool(columns) and native.prefill_waves_built(code, d, 8)
            found = (
                group, spec.num_kv_heads, block_size, columns, key_tokens, int(self._split_prefill),
                self._col_tiles or 0, self._prefill_waves or 0, max_ctw, int(wide),
                native.resident_decode_waves(code, d, 1), native.decode_tile_tokens(code, d, 1),
                native.resident_decode_waves(code, d, 4) if has4 else 0,
                native.decode_tile_tokens(code, d, 4) if has4 else 0,
                native.prefill_resident_units(code, d, 4) if columns else 0,
                native.prefill_resident_units(code, d, 8) if wide else 0,
                self._partition_tokens or 0, DECODE_MAX_COLUMNS, DECODE_MIN_UNITS_PER_WAVE, PREFILL_MIN_TILES,
                int(self._shared_prefix),
                native.xcd_count() if columns else 0, self._prefill_order,
                native.decode_split_groups(code, d) if self._decode_workgroups else 0,
                native.decode_split_waves(code, d),
            )
            self._facts[key] = found
        return found

    def layer_statics(self, cache) -> dict:
        """Per layer id, the cache's fixed facts for the fast forward (built
        once per cache); layers of unbuilt head sizes are left out."""

        found = self._statics.get(cache)
        if found is None:
            config = cache.config
            device = config.device
            index = device.index if device.index is not None else torch.cuda.current_device()
            seen: dict[tuple, int] = {}
            found = {}
            for spec in cache.model_spec.layers:
                if spec.head_size not in SUPPORTED_HEAD_SIZES:
                    continue
                shape = (spec.num_query_heads, spec.num_kv_heads, spec.head_size)
                position = seen.get(shape, 0)
                seen[shape] = position + 1
                found[spec.layer_id] = _LayerStatic(spec, position, cache.layer(spec.layer_id), config, index)
            self._statics[cache] = found
            self._shape_counts[cache] = seen
        return found

    def shape_counts(self, cache) -> dict:
        """Layers of each shape in the cache (after ``layer_statics``)."""

        return self._shape_counts[cache]

    def _check_head_sizes(self, cache) -> None:
        """A cache with a layer of an unbuilt head size is refused when the
        step starts (KVCacheError, checked once per cache), not at that
        layer's first forward.  The reference's Triton backend takes head
        sizes up to 256 (triton_paged_attention.py:475-478); the kernels here
        are built for SUPPORTED_HEAD_SIZES."""

        if cache in self._head_sizes_ok:
            return
        for spec in cache.model_spec.layers:
            if spec.head_size not in SUPPORTED_HEAD_SIZES:
                raise errors.KVCacheError(
                    f"HIP paged attention supports head sizes {SUPPORTED_HEAD_SIZES}, not {spec.head_size} "
                    f"(layer {spec.layer_id!r})"
                )
        self._head_sizes_ok.add(cache)

    def _cache_shapes(self, cache) -> LayerShapes:
        """Kernel facts of each distinct supported layer shape of ``cache``
        (looked up once per cache object)."""

        found = self._shapes.get(cache)
        if found is None:
            config = cache.config
            code = dtype_code(config.dtype)
            shapes = {(s.num_query_heads, s.num_kv_heads, s.head_size): s for s in cache.model_spec.layers}
            found = self._shapes[cache] = LayerShapes(
                self.kernel_facts(spec, code, config.block_size) for spec in shapes.values()
                if spec.head_size in SUPPORTED_HEAD_SIZES)
        return found

    def create(self, cache, metadata) -> HipPagedAttention:
        # This package's metadata is recognised by its facts object, which the
        # plan holds anyway: the metadata itself (a step's worth of tuples) is
        # not kept alive, so the caller frees it, not the next create().  The
        # same metadata on the same cache object takes the last plan with no
        # rule to re-check (the cache's configuration does not change).
        key = metadata.facts if isinstance(metadata, PagedAttentionMetadata) else metadata
        last = self._last
        if last is not None and last[1] is key and last[3]() is cache:
            return HipPagedAttention(self, cache, last[2])
        config = cache.config
        if config.device.type != "cuda":
            raise errors.KVCacheError("HIP paged attention requires a GPU KV cache")
        self._check_head_sizes(cache)
        shapes = self._cache_shapes(cache)
        # A plan is reusable by a cache of the same pool geometry, dtype and
        # layer shapes: its work lists were built from the kernel facts of
        # those shapes in that dtype.
        geometry = (config.num_blocks, config.block_size, config.device, config.dtype, shapes.keys)
        if last is not None and last[1] is key and last[0] == geometry:
            self._last = (geometry, key, last[2], weakref.ref(cache))
            return HipPagedAttention(self, cache, last[2])
        staging = self._staging.get(config.device)
        if staging is None:
            staging = self._staging[config.device] = Staging(config.device)
        # One native call validates, plans every layer shape of the cache and
        # stages it all; one copy uploads it.
        plan = StepPlan(metadata, block_size=config.block_size, device=config.device, num_blocks=config.num_blocks,
                        partition_tokens=self._partition_tokens, staging=staging, shapes=shapes)
        self._last = (geometry, key, plan, weakref.ref(cache))
        return HipPagedAttention(self, cache, plan)
