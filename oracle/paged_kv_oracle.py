"""CPU oracle of light-vllm's paged-KV path.  TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.  The HIP library has no CPU fallback and never calls into this file.

It restates, with numpy, the behaviour of the reference's PyTorch correctness
path (paths relative to light-vllm's source tree):

* ``linear_parents`` / ``append_draft_parents`` / ``semantic_positions`` /
  ``query_visibility``          src/light_vllm/runtime/execution/layout.py:13-55
* ``slot_mapping``              src/light_vllm/runtime/execution/paged_attention.py:110-136
* ``validate_block_tables``     src/light_vllm/runtime/execution/paged_attention.py:138-172
* ``visibility_tensor`` / ``request_indices``
                                src/light_vllm/runtime/execution/paged_attention.py:98-108, 174-186
* ``append``                    src/light_vllm/runtime/execution/paged_cache.py:165-248
* ``compact``                   src/light_vllm/runtime/execution/paged_cache.py:257-326
* ``paged_attention``           src/light_vllm/runtime/execution/paged_attention.py:268-380
                                (per query, per logical block, fp32 online softmax)
* ``dense_attention``           tests/test_paged_attention.py:74-81 (textbook
                                softmax, here in fp64 over the gathered keys)
* ``block_copy``                no reference function (copy-on-write of whole
                                blocks); its definition is the closed form below.
* ``rotary_half``               src/light_vllm/modeling/models/_qwen2_kernels.py:214-224
                                (apply_rotary's PyTorch path, with its rounding)
* ``kv_cache_bytes_per_block`` / ``planned_num_blocks``
                                src/light_vllm/runtime/execution/paged_cache.py:52-65, 98-114
                                (the capacity planner's arithmetic)

How each function is pinned (tests/test_oracle.py):
* slot mapping, validation, visibility, request indices, layouts and compact:
  the reference tests' known answers (tests/golden/reference_known_answers.json);
* append, compact, block copy: closed-form invariants (every untouched byte
  unchanged, moved rows byte-equal) on random pools;
* rotary_half: torch's own CPU arithmetic in the tensor dtype running the
  reference expression, closed forms (cos 1 / sin 0 is the identity, cos 0 /
  sin 1 the pure half swap), norm preservation, and planted mistakes;
* kv_cache_bytes_per_block / planned_num_blocks: known answers for the
  Qwen2.5 shapes (bytes written out by hand from the layer shapes) and a
  brute-force allocation count (blocks added until the budget is exceeded);
* paged_attention: the fp64 dense softmax on random inputs (GQA, tree masks,
  multi-block, shared prefix, lookahead), plus closed forms (one visible key
  gives that key's value; identical keys give the mean of the visible values),
  and planted mistakes in a copy of the oracle are shown to fail those checks.
"""

from __future__ import annotations

import math

import numpy as np


class OracleKVCacheError(RuntimeError):
    """Mirrors KVCacheError for the oracle's validation failures."""


# --------------------------------------------------------------------------- layouts
def linear_parents(num_queries: int) -> tuple[int, ...]:
    return tuple(i - 1 for i in range(num_queries))


def append_draft_parents(num_input_queries: int, draft_parents: tuple[int, ...]) -> tuple[int, ...]:
    parents = list(linear_parents(num_input_queries))
    for p in draft_parents:
        parents.append(num_input_queries - 1 if p == -1 else num_input_queries + p)
    return tuple(parents)


def semantic_positions(parents: tuple[int, ...], prefix_length: int) -> tuple[int, ...]:
    out: list[int] = []
    for p in parents:
        out.append(prefix_length if p == -1 else out[p] + 1)
    return tuple(out)


def query_visibility(parents: tuple[int, ...]) -> np.ndarray:
    """bool [q, q]: row i marks i and its ancestors."""

    q = len(parents)
    vis = np.zeros((q, q), dtype=bool)
    for i in range(q):
        vis[i, i] = True
        p = parents[i]
        while p != -1:
            vis[i, p] = True
            p = parents[p]
    return vis


def is_linear(parents: tuple[int, ...]) -> bool:
    return all(p == i - 1 for i, p in enumerate(parents))


def visibility_tensor(layouts: list[tuple[int, ...]]) -> tuple[np.ndarray, np.ndarray]:
    flat: list[bool] = []
    starts = [0]
    for parents in layouts:
        flat.extend(query_visibility(parents).reshape(-1).tolist())
        starts.append(len(flat))
    return np.asarray(flat, dtype=bool), np.asarray(starts, dtype=np.int32)


def request_indices(q_lens: list[int]) -> np.ndarray:
    return np.repeat(np.arange(len(q_lens)), q_lens).astype(np.int32)


# --------------------------------------------------------------------------- metadata
def _required_blocks(computed: int, reserved: int, block_size: int) -> int:
    return (computed + reserved + block_size - 1) // block_size


def slot_mapping(block_tables, computed, q_lens, reserved, block_size: int) -> np.ndarray:
    out: list[int] = []
    for table, c, q, res in zip(block_tables, computed, q_lens, reserved):
        need = _required_blocks(c, res, block_size)
        if len(table) < need:
            raise OracleKVCacheError("block table does not cover all scheduled tokens")
        if len(table) > need:
            raise OracleKVCacheError("block table contains unused physical blocks")
        for pos in range(c, c + q):
            out.append(table[pos // block_size] * block_size + pos % block_size)
    return np.asarray(out, dtype=np.int64)


def validate_block_tables(block_tables, computed, reserved, readonly, *, num_blocks: int, block_size: int) -> None:
    owners: dict[int, tuple[int, bool]] = {}
    for table, c, res, ro in zip(block_tables, computed, reserved, readonly):
        need = _required_blocks(c, res, block_size)
        if len(table) < need:
            raise OracleKVCacheError("block table does not cover all scheduled tokens")
        if len(table) > need:
            raise OracleKVCacheError("block table contains unused physical blocks")
        if any(b >= num_blocks for b in table):
            raise OracleKVCacheError("block table contains an out-of-range physical block")
        if ro > len(table) or ro * block_size > c:
            raise OracleKVCacheError("readonly prefix blocks exceed the computed prefix")
        if len(set(table)) != len(table):
            raise OracleKVCacheError("block table aliases a physical block within one request")
        for idx, b in enumerate(table):
            is_ro = idx < ro
            prev = owners.get(b)
            if prev is not None and (prev[0] != idx or not prev[1] or not is_ro):
                raise OracleKVCacheError("block tables alias a physical block across requests")
            owners[b] = (idx, is_ro)


# --------------------------------------------------------------------------- rotary
def _bits_to_f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    """Element bits (uint16 for bf16/f16, float32 for f32) as float32 values."""

    if dtype == "bf16":
        return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    if dtype == "f16":
        return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
    return np.asarray(bits, dtype=np.float32)


def _round_to(values: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to nearest-even in ``dtype``, returned as element bits."""

    values = np.asarray(values, dtype=np.float32)
    if dtype == "bf16":
        u = values.view(np.uint32).astype(np.uint64)
        rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        return np.where(np.isnan(values), np.uint16(0x7FC0), rounded)
    if dtype == "f16":
        return values.astype(np.float16).view(np.uint16)
    return values


def rotary_half(x: np.ndarray, cosines: np.ndarray, sines: np.ndarray, dtype: str) -> np.ndarray:
    """Qwen2's half rotation of x [T, H, D] by per-token cos/sin rows [T, D]
    (_qwen2_kernels.py:214-224): ``x * cos + cat(-x[D/2:], x[:D/2]) * sin``.

    Element bits in and out.  As in PyTorch's evaluation of that expression in
    the tensor dtype, each product is rounded to the dtype, then the float32
    sum of the two is rounded to the dtype.
    """

    xf = _bits_to_f32(x, dtype)
    c = _bits_to_f32(cosines, dtype)[:, None, :]
    s = _bits_to_f32(sines, dtype)[:, None, :]
    half = xf.shape[-1] // 2
    rotated = np.concatenate((-xf[..., half:], xf[..., :half]), axis=-1)
    first = _bits_to_f32(_round_to(xf * c, dtype), dtype)
    second = _bits_to_f32(_round_to(rotated * s, dtype), dtype)
    return _round_to(first + second, dtype)


# --------------------------------------------------------------------------- KV movement
def append(key_pool: np.ndarray, value_pool: np.ndarray, key: np.ndarray, value: np.ndarray, slots: np.ndarray) -> None:
    """flat[slot[t]] = row[t] for active (>= 0) slots; pools are [NB, bs, Hkv, D] of any dtype."""

    nb, bs = key_pool.shape[:2]
    flat_k = key_pool.reshape(nb * bs, *key_pool.shape[2:])
    flat_v = value_pool.reshape(nb * bs, *value_pool.shape[2:])
    slots = np.asarray(slots, dtype=np.int64)
    active = slots >= 0
    flat_k[slots[active]] = key[active]
    flat_v[slots[active]] = value[active]


def compact(
    pools: list[tuple[np.ndarray, np.ndarray]],
    block_ids: tuple[int, ...],
    *,
    num_computed_tokens: int,
    num_query_tokens: int,
    num_reserved_query_tokens: int,
    retained_query_indices: tuple[int, ...],
    num_readonly_prefix_blocks: int = 0,
    num_blocks: int,
    block_size: int,
) -> int:
    retained = tuple(retained_query_indices)
    counts = (num_computed_tokens, num_query_tokens, num_reserved_query_tokens, num_readonly_prefix_blocks)
    if any(type(v) is not int or v < 0 for v in counts):
        raise ValueError("paged compact counts must be non-negative integers")
    if num_reserved_query_tokens < num_query_tokens:
        raise ValueError("reserved query tokens must cover every actual query")
    if any(type(i) is not int or i < 0 for i in retained):
        raise ValueError("retained query indices must be non-negative integers")
    if len(set(retained)) != len(retained):
        raise ValueError("retained query indices must be unique")
    if any(i >= num_query_tokens for i in retained):
        raise OracleKVCacheError("retained query index exceeds the paged KV tail")
    if len(block_ids) != _required_blocks(num_computed_tokens, num_reserved_query_tokens, block_size):
        raise OracleKVCacheError("block table does not exactly cover the reserved query slots")
    if any(type(b) is not int or not 0 <= b < num_blocks for b in block_ids):
        raise OracleKVCacheError("block table contains an invalid physical block")
    if len(set(block_ids)) != len(block_ids):
        raise OracleKVCacheError("block table aliases a physical block within one request")
    if num_readonly_prefix_blocks * block_size > num_computed_tokens:
        raise OracleKVCacheError("readonly prefix blocks exceed the computed prefix")

    def slot(pos: int) -> int:
        return block_ids[pos // block_size] * block_size + pos % block_size

    src = [slot(num_computed_tokens + i) for i in retained]
    dst = [slot(num_computed_tokens + i) for i in range(len(retained))]
    if src == dst:
        return 0
    for kp, vp in pools:
        for pool in (kp, vp):
            flat = pool.reshape(pool.shape[0] * pool.shape[1], *pool.shape[2:])
            gathered = flat[src].copy()  # every source before any target
            flat[dst] = gathered
    return sum(s != d for s, d in zip(src, dst))


def block_copy(pools: list[tuple[np.ndarray, np.ndarray]], src_blocks, dst_blocks) -> None:
    """Closed form: block dst[i] := block src[i] in every layer, K and V."""

    for kp, vp in pools:
        for pool in (kp, vp):
            pool[list(dst_blocks)] = pool[list(src_blocks)]


# --------------------------------------------------------------------------- attention
def _visible_positions(computed: int, parents: tuple[int, ...]) -> list[list[int]]:
    vis = query_visibility(parents)
    prefix = list(range(computed))
    return [prefix + [computed + j for j in np.flatnonzero(vis[i])] for i in range(len(parents))]


def paged_attention(
    query: np.ndarray,
    key_pool: np.ndarray,
    value_pool: np.ndarray,
    block_tables,
    computed,
    layouts,
    *,
    scale: float,
) -> np.ndarray:
    """Per query token, per logical block, fp32 online softmax (reference order).

    query [T, Hq, D] float32; pools [NB, bs, Hkv, D] float32 (the bf16/fp16 values
    widened exactly, as the reference's .to(float32) does).  Returns fp32 [T, Hq, D].
    """

    query = np.asarray(query, dtype=np.float32)
    key_pool = np.asarray(key_pool, dtype=np.float32)
    value_pool = np.asarray(value_pool, dtype=np.float32)
    block_size = key_pool.shape[1]
    num_q_heads = query.shape[1]
    num_kv_heads = key_pool.shape[2]
    repeats = num_q_heads // num_kv_heads
    scale32 = np.float32(scale)
    out = np.zeros_like(query)
    token = 0
    for table, c, parents in zip(block_tables, computed, layouts):
        for positions in _visible_positions(c, tuple(parents)):
            q = query[token]
            m = np.full(num_q_heads, -np.inf, dtype=np.float32)
            s_run = np.zeros(num_q_heads, dtype=np.float32)
            acc = np.zeros_like(q)
            by_block: dict[int, list[int]] = {}
            for pos in positions:
                by_block.setdefault(pos // block_size, []).append(pos % block_size)
            for logical, offsets in by_block.items():
                blk = table[logical]
                keys = key_pool[blk, offsets]
                vals = value_pool[blk, offsets]
                if repeats > 1:
                    keys = np.repeat(keys, repeats, axis=1)
                    vals = np.repeat(vals, repeats, axis=1)
                scores = np.einsum("hd,thd->ht", q, keys) * scale32
                nxt = np.maximum(m, scores.max(axis=1))
                prev_scale = np.exp(m - nxt)
                weights = np.exp(scores - nxt[:, None])
                acc = acc * prev_scale[:, None] + np.einsum("ht,thd->hd", weights, vals)
                s_run = s_run * prev_scale + weights.sum(axis=1)
                m = nxt
            out[token] = acc / s_run[:, None]
            token += 1
    return out


def dense_attention(
    query: np.ndarray,
    key_pool: np.ndarray,
    value_pool: np.ndarray,
    block_tables,
    computed,
    layouts,
    *,
    scale: float,
) -> np.ndarray:
    """Textbook masked softmax in fp64 over every logical position of a request.

    Independent of ``paged_attention``'s position lists: the mask is built from
    the ancestor matrix directly (prefix columns all visible), and masked
    scores are -inf before one full softmax per query.
    """

    query = np.asarray(query, dtype=np.float64)
    block_size = key_pool.shape[1]
    num_q_heads, head_size = query.shape[1], query.shape[2]
    num_kv_heads = key_pool.shape[2]
    group = num_q_heads // num_kv_heads  # q head h reads kv head h // group
    out = np.zeros_like(query)
    start = 0
    for table, c, parents in zip(block_tables, computed, layouts):
        q_len = len(parents)
        length = c + q_len
        pos = np.arange(length)
        blocks = np.asarray(table)[pos // block_size]
        # [kv head, key, dim]; the query heads of a kv head are its group.
        keys = np.asarray(key_pool[blocks, pos % block_size], dtype=np.float64).transpose(1, 0, 2)
        vals = np.asarray(value_pool[blocks, pos % block_size], dtype=np.float64).transpose(1, 0, 2)
        mask = np.ones((q_len, length), dtype=bool)
        mask[:, c:] = query_visibility(tuple(parents))
        q = query[start : start + q_len].reshape(q_len, num_kv_heads, group, head_size).transpose(1, 0, 2, 3)
        q = q.reshape(num_kv_heads, q_len * group, head_size)
        scores = np.matmul(q, keys.transpose(0, 2, 1)).reshape(num_kv_heads, q_len, group, length) * float(scale)
        scores = np.where(mask[None, :, None, :], scores, -np.inf)
        scores -= scores.max(axis=3, keepdims=True)
        probs = np.exp(scores)
        probs /= probs.sum(axis=3, keepdims=True)
        o = np.matmul(probs.reshape(num_kv_heads, q_len * group, length), vals)  # [kv head, q x group, dim]
        out[start : start + q_len] = o.reshape(num_kv_heads, q_len, group, head_size).transpose(1, 0, 2, 3).reshape(
            q_len, num_q_heads, head_size)
        start += q_len
    return out


def visible_positions(computed: int, parents: tuple[int, ...]) -> list[list[int]]:
    """Logical positions each query of one request reads (paged_attention.py:188-206)."""

    return _visible_positions(computed, parents)


def softmax_scale(head_size: int) -> float:
    return 1.0 / math.sqrt(head_size)


def kv_cache_bytes_per_block(layers, *, block_size: int, element_size: int) -> int:
    """Bytes of one physical block over every layer: K and V rows of each
    layer's (num_kv_heads, head_size), ``block_size`` tokens
    (paged_cache.py:52-65).  ``layers``: (num_kv_heads, head_size) pairs."""

    per_token = sum(2 * hkv * d for hkv, d in layers)
    return block_size * per_token * element_size


def planned_num_blocks(free_bytes: int, memory_fraction: float, layers, *, block_size: int,
                       element_size: int) -> int:
    """Whole blocks in ``int(free_bytes * memory_fraction)`` bytes
    (CudaMemoryKVCachePlanner.plan, paged_cache.py:98-114); 0 means the
    planner raises KVCacheCapacityError."""

    budget = int(free_bytes * memory_fraction)
    return budget // kv_cache_bytes_per_block(layers, block_size=block_size, element_size=element_size)
