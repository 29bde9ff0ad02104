"""GPU: ``lvamd_kv_compact_small`` and ``lvamd_kv_block_copy_small`` (pairs
in the kernel arguments) through the C ABI, against the closed form and
against ``lvamd_kv_compact`` / ``lvamd_kv_block_copy`` with the same pairs in
device memory.

Compact: row dst[i] of every layer's K and V must hold what row src[i] held
before the call (sources may repeat and may be destinations: every source is
read before any destination is written); every other row is unchanged.
Block copy: block dst[i] becomes block src[i] (disjoint sets).  Row sizes
and layer counts cover each access width the kernels pick (16, 8, 4 and 2
bytes): the compact narrows its chunks until about 32 workgroups share the
call, so 16- and 8-byte chunks need many layers of wide rows (32 layers of
2048-byte rows, 16 layers of 2056-byte rows); three layers of 512-, 72- and
36-byte rows run 4-byte chunks, 18-byte rows 2-byte chunks.
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
LAYERS, SLOTS = 3, 512


def _pools(seed: int, row: int, layers: int = LAYERS):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    return [(torch.randint(-30000, 30000, (SLOTS, row), generator=gen, device=DEV, dtype=torch.int16),
             torch.randint(-30000, 30000, (SLOTS, row), generator=gen, device=DEV, dtype=torch.int16))
            for _ in range(layers)]


def _tables(pools):
    keys = torch.tensor([k.data_ptr() for k, _ in pools], dtype=torch.int64, device=DEV)
    values = torch.tensor([v.data_ptr() for _, v in pools], dtype=torch.int64, device=DEV)
    return keys, values


@pytest.mark.parametrize("layers,row", [(3, 256), (3, 36), (3, 18), (3, 9), (32, 1024), (16, 1028)])  # int16 elements
@pytest.mark.parametrize("n", (1, 7, 8, 9, 16, 17, 32))  # the kernel's 8 / 16 / 32-pair buckets
def test_small_compact_matches_the_closed_form_and_the_device_pair_compact(n, layers, row) -> None:
    print(f"[gpu] small compact n={n} layers={layers} row={2 * row} bytes", file=sys.stderr, flush=True)
    lib = native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    rng = np.random.default_rng(n * 1000 + row)
    dst = rng.permutation(SLOTS)[:n].astype(np.int64)
    src = rng.integers(0, SLOTS, size=n).astype(np.int64)
    small, device_pairs = _pools(row, row, layers), _pools(row, row, layers)
    before = [(k.cpu().numpy(), v.cpu().numpy()) for k, v in small]
    sk, sv = _tables(small)
    dk, dv = _tables(device_pairs)
    native.check(lib.lvamd_kv_compact_small(sk.data_ptr(), sv.data_ptr(), layers, 2 * row, src.ctypes.data,
                                            dst.ctypes.data, n, stream), "lvamd_kv_compact_small")
    src_d, dst_d = torch.tensor(src, device=DEV), torch.tensor(dst, device=DEV)
    native.check(lib.lvamd_kv_compact(dk.data_ptr(), dv.data_ptr(), layers, 2 * row, src_d.data_ptr(),
                                      dst_d.data_ptr(), n, None, 0, stream), "lvamd_kv_compact")
    torch.cuda.synchronize()
    for layer, ((gk, gv), (rk, rv), (bk, bv)) in enumerate(zip(small, device_pairs, before)):
        for got, ref, pool in ((gk, rk, bk), (gv, rv, bv)):
            expect = pool.copy()
            expect[dst] = pool[src]
            np.testing.assert_array_equal(got.cpu().numpy(), expect, err_msg=f"layer {layer}: closed form")
            np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy(), err_msg=f"layer {layer}: device pairs")


@pytest.mark.parametrize("row", (256, 18))  # int16 elements per block: 512 and 36 bytes
@pytest.mark.parametrize("n", (1, 9, 32))
def test_small_block_copy_matches_the_closed_form_and_the_device_pair_copy(n, row) -> None:
    print(f"[gpu] small block copy n={n} block={2 * row} bytes", file=sys.stderr, flush=True)
    lib = native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    rng = np.random.default_rng(n * 100 + row)
    perm = rng.permutation(SLOTS)
    src, dst = perm[:n].astype(np.int64), perm[n: 2 * n].astype(np.int64)
    small, device_pairs = _pools(row + 1, row), _pools(row + 1, row)
    before = [(k.cpu().numpy(), v.cpu().numpy()) for k, v in small]
    sk, sv = _tables(small)
    dk, dv = _tables(device_pairs)
    native.check(lib.lvamd_kv_block_copy_small(sk.data_ptr(), sv.data_ptr(), LAYERS, 2 * row, src.ctypes.data,
                                               dst.ctypes.data, n, stream), "lvamd_kv_block_copy_small")
    src_d, dst_d = torch.tensor(src, device=DEV), torch.tensor(dst, device=DEV)
    native.check(lib.lvamd_kv_block_copy(dk.data_ptr(), dv.data_ptr(), LAYERS, 2 * row, src_d.data_ptr(),
                                         dst_d.data_ptr(), n, stream), "lvamd_kv_block_copy")
    torch.cuda.synchronize()
    for layer, ((gk, gv), (rk, rv), (bk, bv)) in enumerate(zip(small, device_pairs, before)):
        for got, ref, pool in ((gk, rk, bk), (gv, rv, bv)):
            expect = pool.copy()
            expect[dst] = pool[src]
            np.testing.assert_array_equal(got.cpu().numpy(), expect, err_msg=f"layer {layer}: closed form")
            np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy(), err_msg=f"layer {layer}: device pairs")
