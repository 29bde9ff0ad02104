"""GPU parity of the fused rotary append.

``lvamd_kv_append_rotary`` must produce the rotated queries and the pool rows
of ``apply_rotary`` + append bit for bit against the oracle's ``rotary_half``
(itself pinned to torch's CPU arithmetic in the tensor dtype); every other
pool byte must be unchanged.  ``forward(..., rotary=(cos, sin))`` must then
attend over those rows within the attention tolerances (bf16 2e-2 / 2e-3,
fp16 3e-3 / 3e-4, fp32 1e-5 max-abs).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from light_vllm_amd import native
from oracle import paged_kv_oracle as O
from paged_cases import make_step, oracle_attention, tolerances

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")
ROPE_THETA = 1_000_000.0  # Qwen2.5's rope_theta
NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}
CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}


def _announce(name: str) -> None:
    print(f"[gpu] {name}", file=sys.stderr, flush=True)


def rope_rows(positions, d: int, dtype: torch.dtype):
    """cos/sin rows as Qwen2 builds them (qwen2.py:690-705): angles
    pos * theta^(-2i/d), both halves the same, rounded to the model dtype."""

    pos = torch.as_tensor(np.asarray(positions), dtype=torch.float32)
    freqs = 1.0 / (ROPE_THETA ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.outer(pos, freqs)
    emb = torch.cat((emb, emb), dim=-1)
    return emb.cos().to(dtype).to(DEV), emb.sin().to(dtype).to(DEV)


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.float32:
        return t.numpy().copy()
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def _call(q, q_out, k, v, cos, sin, kpool, vpool, slots, hq, hkv, d) -> int:
    lib = native.load()
    return lib.lvamd_kv_append_rotary(
        q.data_ptr(), q.stride(0), q.stride(1), q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
        k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
        cos.data_ptr(), cos.stride(0), sin.data_ptr(), sin.stride(0),
        kpool.data_ptr(), vpool.data_ptr(), slots.data_ptr(), slots.numel(),
        hq, hkv, d, CODES[q.dtype], torch.cuda.current_stream(DEV).cuda_stream,
    )


def _case(dtype, d, *, tokens=37, hq=12, hkv=2, nb=24, bs=16, seed=0, offset=0):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    width = (hq + 2 * hkv) * d
    # q, k, v as views of one fused projection (token stride = width), as the
    # model's qkv split produces them; ``offset`` shifts them off alignment.
    qkv = torch.randn(tokens * width + offset, generator=gen).to(dtype).to(DEV)
    qkv = qkv[offset:].view(tokens, width)
    q = qkv[:, : hq * d].view(tokens, hq, d)
    k = qkv[:, hq * d : (hq + hkv) * d].view(tokens, hkv, d)
    v = qkv[:, (hq + hkv) * d :].view(tokens, hkv, d)
    kpool = torch.randn((nb, bs, hkv, d), generator=gen).to(dtype).to(DEV)
    vpool = torch.randn((nb, bs, hkv, d), generator=gen).to(dtype).to(DEV)
    rng = np.random.default_rng(seed)
    slots = rng.permutation(nb * bs)[:tokens].astype(np.int64)
    slots[rng.choice(tokens, size=3, replace=False)] = -1  # inactive tokens
    cos, sin = rope_rows(rng.integers(0, 32768, size=tokens), d, dtype)
    return q, k, v, cos, sin, kpool, vpool, torch.from_numpy(slots).to(DEV)


def _expected(q, k, v, cos, sin, kpool, vpool, slots, dtype):
    name = NAMES[dtype]
    q_rot = O.rotary_half(_bits(q), _bits(cos), _bits(sin), name)
    k_rot = O.rotary_half(_bits(k), _bits(cos), _bits(sin), name)
    kp, vp = _bits(kpool), _bits(vpool)
    O.append(kp, vp, k_rot, _bits(v), slots.cpu().numpy())
    return q_rot, kp, vp


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("d", [48, 64, 80, 96, 112, 128, 160, 192, 240, 256])
def test_rotary_append_matches_oracle_bit_for_bit(dtype, d) -> None:
    _announce(f"rotary append {dtype} D={d}")
    q, k, v, cos, sin, kpool, vpool, slots = _case(dtype, d, seed=d)
    q_rot, kp, vp = _expected(q, k, v, cos, sin, kpool, vpool, slots, dtype)
    q_out = torch.empty(q.shape, dtype=dtype, device=DEV)
    assert _call(q, q_out, k, v, cos, sin, kpool, vpool, slots, q.shape[1], k.shape[1], d) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(q_out), q_rot)
    np.testing.assert_array_equal(_bits(kpool), kp)  # every other row unchanged
    np.testing.assert_array_equal(_bits(vpool), vp)


@pytest.mark.parametrize("dtype, offset", [(torch.bfloat16, 1), (torch.float16, 3), (torch.float32, 1)])
def test_rotary_append_in_place_and_unaligned_rows(dtype, offset) -> None:
    """Rows off 16-byte alignment take narrower accesses; query_out may alias
    the query."""

    _announce(f"rotary append in place {dtype} offset {offset}")
    q, k, v, cos, sin, kpool, vpool, slots = _case(dtype, 128, seed=5, offset=offset)
    q_rot, kp, vp = _expected(q, k, v, cos, sin, kpool, vpool, slots, dtype)
    assert _call(q, q, k, v, cos, sin, kpool, vpool, slots, q.shape[1], k.shape[1], 128) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(q), q_rot)
    np.testing.assert_array_equal(_bits(kpool), kp)
    np.testing.assert_array_equal(_bits(vpool), vp)


def _positions(metadata) -> np.ndarray:
    out = []
    for computed, layout in zip(metadata.num_computed_tokens, metadata.query_layouts):
        out.extend(O.semantic_positions(tuple(layout.parent_indices), computed))
    return np.asarray(out, dtype=np.int64)


CASES = {
    "decode_qwen7b": dict(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[700, 1500, 33, 2900, 260],
                          layouts=[(-1,)] * 5),
    "prefill_and_decode": dict(hq=14, hkv=2, d=64, bs=16, dtype=torch.float16, computed=[0, 300, 41],
                               layouts=[tuple(range(-1, 95)), (-1,), tuple(range(-1, 20))]),
    "tree_shared_prefix": dict(hq=12, hkv=2, d=128, bs=16, dtype=torch.bfloat16, computed=[160, 200, 171],
                               layouts=[(-1, 0, 0, 1, 1, 2, 3, 3, 5)] * 3, shared_prefix_blocks=8),
    "fp32_decode": dict(hq=14, hkv=2, d=64, bs=16, dtype=torch.float32, computed=[37, 128, 200, 511],
                        layouts=[(-1,)] * 4),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_forward_with_rotary_equals_rotate_then_attend(name) -> None:
    _announce(f"forward rotary {name}")
    case = dict(CASES[name])
    dtype = case["dtype"]
    step = make_step(seed=17, **case)
    lid = step.layer_ids[0]
    cos, sin = rope_rows(_positions(step.metadata), case["d"], dtype)
    q_rot = O.rotary_half(_bits(step.query), _bits(cos), _bits(sin), NAMES[dtype])
    k_rot = O.rotary_half(_bits(step.key), _bits(cos), _bits(sin), NAMES[dtype])
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale, rotary=(cos, sin))
    torch.cuda.synchronize()
    cfg = step.cache.config
    slots = step.metadata.slot_mapping(block_size=cfg.block_size, device=DEV)
    layer = step.cache.layer(lid)
    n = cfg.num_blocks * cfg.block_size
    hkv, d = step.key.shape[1:]
    np.testing.assert_array_equal(_bits(layer.keys.view(n, hkv, d).index_select(0, slots)), k_rot)
    np.testing.assert_array_equal(_bits(layer.values.view(n, hkv, d).index_select(0, slots)), _bits(step.value))
    q_rot_t = torch.from_numpy(q_rot.view(np.int16) if dtype != torch.float32 else q_rot)
    q_rot_t = q_rot_t.view(dtype) if dtype != torch.float32 else q_rot_t
    expect = oracle_attention(step, lid, query=q_rot_t)
    got = out.float().cpu().numpy()
    err = np.abs(got - expect)
    max_tol, mean_tol = tolerances(dtype)
    assert np.isfinite(got).all()
    assert err.max() <= max_tol, f"max-abs {err.max():.3e} > {max_tol}"
    assert err.mean() <= mean_tol, f"mean-abs {err.mean():.3e} > {mean_tol}"


def test_rotary_shape_errors() -> None:
    step = make_step(hq=4, hkv=2, d=64, bs=4, dtype=torch.bfloat16, computed=[5], layouts=[(-1,)], seed=3)
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    cos, sin = rope_rows([5], 64, torch.bfloat16)
    with pytest.raises(lv.KVCacheError, match="rotary cosines must have shape"):
        ctx.forward("layer0", step.query, step.key, step.value, scale=step.scale, rotary=(cos[:, :32], sin))
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    with pytest.raises(lv.KVCacheError, match="rotary sines dtype"):
        ctx.forward("layer0", step.query, step.key, step.value, scale=step.scale, rotary=(cos, sin.float()))


def _from_bits(bits: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    if dtype == torch.float32:
        return torch.from_numpy(bits).to(DEV)
    return torch.from_numpy(bits.view(np.int16)).view(dtype).to(DEV)


# Decode steps at the model's shape (the rotary append, then attention over
# the pool), against the fused-append attention step over rows rotated
# beforehand: the outputs and the pools must agree bit for bit.
ROTATED_CASES = {
    "c2_shape_bf16": dict(dtype=torch.bfloat16, seqs=64, lo=512, hi=4096, layout=(-1,), seed=5),
    "chain2_f16": dict(dtype=torch.float16, seqs=48, lo=200, hi=3000, layout=(-1, 0), seed=6),
    "short_bf16": dict(dtype=torch.bfloat16, seqs=96, lo=1, hi=300, layout=(-1,), seed=7),
}


@pytest.mark.parametrize("name", sorted(ROTATED_CASES))
def test_forward_with_rotary_bit_equals_attention_over_rotated_rows(name) -> None:
    """forward(..., rotary) must give the outputs and pool rows of forward over
    queries and keys rotated beforehand (the oracle's rotary_half, pinned bit
    for bit by the tests above), and leave every other pool byte unchanged."""

    _announce(f"rotary vs rotated rows {name}")
    c = ROTATED_CASES[name]
    dtype = c["dtype"]
    rng = np.random.default_rng(c["seed"])
    computed = rng.integers(c["lo"], c["hi"] + 1, size=c["seqs"]).tolist()
    case = dict(hq=28, hkv=4, d=128, bs=16, dtype=dtype, computed=computed, layouts=[c["layout"]] * c["seqs"])
    rotary = make_step(seed=c["seed"], **case)
    rotated = make_step(seed=c["seed"], **case)
    lid = rotary.layer_ids[0]
    cos, sin = rope_rows(_positions(rotary.metadata), 128, dtype)
    q_rot = _from_bits(O.rotary_half(_bits(rotary.query), _bits(cos), _bits(sin), NAMES[dtype]), dtype)
    k_rot = _from_bits(O.rotary_half(_bits(rotary.key), _bits(cos), _bits(sin), NAMES[dtype]), dtype)
    rl, dl = rotary.cache.layer(lid), rotated.cache.layer(lid)
    before_k, before_v = _bits(rl.keys), _bits(rl.values)
    ctx = lv.HipPagedAttentionBackend().create(rotary.cache, rotary.metadata)
    out_rotary = ctx.forward(lid, rotary.query, rotary.key, rotary.value, scale=rotary.scale, rotary=(cos, sin))
    ctx = lv.HipPagedAttentionBackend().create(rotated.cache, rotated.metadata)
    out_rotated = ctx.forward(lid, q_rot, k_rot, rotated.value, scale=rotated.scale)
    torch.cuda.synchronize()
    assert np.isfinite(out_rotary.float().cpu().numpy()).all()
    np.testing.assert_array_equal(_bits(out_rotary), _bits(out_rotated))
    # This step's slots hold the same rows in both caches; every other pool
    # byte is unchanged (the caches' unwritten rows differ between the two
    # allocations, so only the slots are compared across them).
    cfg = rotary.cache.config
    slots = rotary.metadata.slot_mapping(block_size=cfg.block_size, device=DEV)
    n = cfg.num_blocks * cfg.block_size
    for pool_r, pool_d, before in ((rl.keys, dl.keys, before_k), (rl.values, dl.values, before_v)):
        np.testing.assert_array_equal(_bits(pool_r.view(n, 4, 128).index_select(0, slots)),
                                      _bits(pool_d.view(n, 4, 128).index_select(0, slots)))
        keep = np.ones(n, dtype=bool)
        keep[slots.cpu().numpy()] = False
        np.testing.assert_array_equal(_bits(pool_r).reshape(n, -1)[keep], before.reshape(n, -1)[keep])
