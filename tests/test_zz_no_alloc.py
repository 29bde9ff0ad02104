"""The allocation-free compact (``lvamd_kv_compact_static``) against the
workspace compact (``lvamd_kv_compact``), through the C ABI.

Both run on identical copies of the same pools; every byte of every layer's
K and V must agree, and the moved rows must equal the closed form (row
dst[i] holds what row src[i] held before the call, every other row is
unchanged).  Two calls in a row, the second with fewer pairs, so the second
runs over the scratch the first left behind.  The process's first call (the
static array's address lookup) is checked on its own, and the device's free
memory must not change across calls.  (The refusal of a call past the static
size happens before any HIP call and is tested on the CPU.)
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from light_vllm_amd import native

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")
LAYERS, BLOCKS, BS, HKV, D = 4, 64, 16, 4, 128  # rows of 1 KiB (bf16)


def _pools(seed: int):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    shape = (BLOCKS, BS, HKV, D)
    return [(torch.randn(shape, generator=gen, device=DEV).to(torch.bfloat16),
             torch.randn(shape, generator=gen, device=DEV).to(torch.bfloat16)) for _ in range(LAYERS)]


def _pointer_tables(pools):
    keys = torch.tensor([k.data_ptr() for k, _ in pools], dtype=torch.int64, device=DEV)
    values = torch.tensor([v.data_ptr() for _, v in pools], dtype=torch.int64, device=DEV)
    return keys, values


def _pairs(rng, n: int):
    slots = BLOCKS * BS
    dst = rng.permutation(slots)[:n]
    src = rng.integers(0, slots, size=n)  # sources may repeat and may be destinations
    return torch.tensor(src, device=DEV), torch.tensor(dst, device=DEV)


def _bits(pools):
    return [(k.view(torch.int16).cpu().numpy(), v.view(torch.int16).cpu().numpy()) for k, v in pools]


def _expected(before, src, dst):
    out = []
    for kb, vb in before:
        layer = []
        for pool in (kb, vb):
            flat = pool.reshape(BLOCKS * BS, HKV * D).copy()
            rows = flat[src.cpu().numpy()].copy()  # every source before any destination
            flat[dst.cpu().numpy()] = rows
            layer.append(flat.reshape(pool.shape))
        out.append(tuple(layer))
    return out


def test_static_compact_allocates_nothing() -> None:
    # The entry point's contract: no device allocation.  This file's first
    # test, so its first call is the process's first (nothing else calls the
    # static compact): the one that looks up the static array's device
    # address, checked against the closed form on its own.  Then the
    # device's free memory is read around two more calls (every tensor they
    # use made beforehand) and must not change.
    lib = native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    row_bytes = HKV * D * 2
    rng = np.random.default_rng(12)
    pools = _pools(6)
    ptrs = _pointer_tables(pools)
    calls = [_pairs(rng, n) for n in (300, 100, 33)]

    def run(src, dst):
        native.check(lib.lvamd_kv_compact_static(ptrs[0].data_ptr(), ptrs[1].data_ptr(), LAYERS, row_bytes,
                                                 src.data_ptr(), dst.data_ptr(), src.numel(), stream),
                     "lvamd_kv_compact_static")

    print("[gpu] no-alloc compact: first call, then free memory around two calls", file=sys.stderr, flush=True)
    before = _bits(pools)
    run(*calls[0])
    torch.cuda.synchronize()
    for (gk, gv), (ek, ev) in zip(_bits(pools), _expected(before, *calls[0])):
        np.testing.assert_array_equal(gk, ek)
        np.testing.assert_array_equal(gv, ev)
    before = _bits(pools)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info(DEV)
    run(*calls[1])
    run(*calls[2])
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info(DEV)
    assert free1 == free0, f"device free memory changed by {free0 - free1} bytes"
    expect = _expected(_expected(before, *calls[1]), *calls[2])
    for (gk, gv), (ek, ev) in zip(_bits(pools), expect):
        np.testing.assert_array_equal(gk, ek)
        np.testing.assert_array_equal(gv, ev)


def test_static_compact_matches_the_workspace_compact_on_two_calls() -> None:
    lib = native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    row_bytes = HKV * D * 2
    rng = np.random.default_rng(11)
    with_workspace, static = _pools(5), _pools(5)
    ws_ptrs, st_ptrs = _pointer_tables(with_workspace), _pointer_tables(static)
    for call, n in enumerate((600, 40)):  # both above the inline pair limit: staged through scratch
        print(f"[gpu] no-alloc compact call {call}: {n} pairs x {LAYERS} layers", file=sys.stderr, flush=True)
        assert n > lib.lvamd_kv_compact_inline_pairs()
        src, dst = _pairs(rng, n)
        before = _bits(static)
        ws_bytes = lib.lvamd_kv_compact_workspace_size(n, LAYERS, row_bytes)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        native.check(lib.lvamd_kv_compact(ws_ptrs[0].data_ptr(), ws_ptrs[1].data_ptr(), LAYERS, row_bytes,
                                          src.data_ptr(), dst.data_ptr(), n, workspace.data_ptr(), ws_bytes,
                                          stream), "lvamd_kv_compact")
        native.check(lib.lvamd_kv_compact_static(st_ptrs[0].data_ptr(), st_ptrs[1].data_ptr(), LAYERS, row_bytes,
                                                 src.data_ptr(), dst.data_ptr(), n, stream),
                     "lvamd_kv_compact_static")
        torch.cuda.synchronize()
        got, ref = _bits(static), _bits(with_workspace)
        for layer, ((gk, gv), (rk, rv), (ek, ev)) in enumerate(zip(got, ref, _expected(before, src, dst))):
            np.testing.assert_array_equal(gk, rk, err_msg=f"call {call} layer {layer} keys vs workspace compact")
            np.testing.assert_array_equal(gv, rv, err_msg=f"call {call} layer {layer} values vs workspace compact")
            np.testing.assert_array_equal(gk, ek, err_msg=f"call {call} layer {layer} keys vs closed form")
            np.testing.assert_array_equal(gv, ev, err_msg=f"call {call} layer {layer} values vs closed form")
