"""The ctypes path of the eager calls (minivllm._ctypes_ops, used when the
_hip_ops extension cannot load) against the extension itself on the MI355X:
the same kernels on the same stream, so bit-identical outputs and KV writes,
and the same ValueError messages for invalid calls."""
from __future__ import annotations

import pytest
import torch

from minivllm import _ctypes_ops, _native
from minivllm.kv_block_pool import KVBlockPool

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _case(dtype, seed=0, B=5, H=8, D=128, S=16, N=64, L=2):
    g = torch.Generator().manual_seed(seed)
    pool = KVBlockPool(L, N, S, H, D, device=DEV, dtype=dtype)
    pool.k.copy_(torch.randn(pool.k.shape, generator=g).to(dtype))
    pool.v.copy_(torch.randn(pool.v.shape, generator=g).to(dtype))
    ctx = torch.tensor([1, 17, 100, 160, 33][:B])
    M = int(-(-ctx.max() // S))
    tables = torch.full((B, M), -1, dtype=torch.long)
    perm = torch.randperm(N, generator=g)
    used = 0
    for b in range(B):
        nb = int(-(-ctx[b] // S))
        tables[b, :nb] = perm[used:used + nb]
        used += nb
    qkv = torch.randn((B, 3, H, D), generator=g).to(dtype).to(DEV)
    return pool, tables.to(DEV), ctx.to(DEV), qkv


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_ctypes_path_is_bit_identical_to_the_extension(dtype):
    ext = _native._load_extension()
    print(f"  ctypes path against _hip_ops, {dtype}", flush=True)
    pool, tables, ctx, qkv = _case(dtype)
    q, k, v = qkv[:, 0], qkv[:, 1], qkv[:, 2]
    last = (ctx - 1).cpu()
    slots = (tables.cpu()[torch.arange(5), last // 16] * 16 + last % 16).to(DEV)
    slots[3] = -1
    twin = KVBlockPool(2, 64, 16, 8, 128, device=DEV, dtype=dtype)
    twin.k.copy_(pool.k)
    twin.v.copy_(pool.v)
    with torch.inference_mode():
        ext.kv_append(pool.k, pool.v, 1, k, v, slots)
        _ctypes_ops.kv_append(twin.k, twin.v, 1, k, v, slots)
        torch.cuda.synchronize()
        assert torch.equal(_bits(pool.k), _bits(twin.k)) and torch.equal(_bits(pool.v), _bits(twin.v))
        for split in (0, 32):
            a = ext.paged_decode(q, pool.k, pool.v, tables, ctx, 1, split)
            b = _ctypes_ops.paged_decode(q, pool.k, pool.v, tables, ctx, 1, split)
            torch.cuda.synchronize()
            assert torch.equal(_bits(a), _bits(b))
        row = tables[3]
        qc = torch.randn((40, 8, 128), generator=torch.Generator().manual_seed(3)).to(dtype).to(DEV)
        a = ext.paged_prefill(qc, pool.k, pool.v, row, 100, 1)
        b = _ctypes_ops.paged_prefill(qc, pool.k, pool.v, row, 100, 1)
        torch.cuda.synchronize()
        assert torch.equal(_bits(a), _bits(b))


def test_ctypes_path_raises_the_extension_messages():
    ext = _native._load_extension()
    pool, tables, ctx, qkv = _case(torch.bfloat16)
    q = qkv[:, 0]
    zero = KVBlockPool(1, 4, 0, 8, 128, device=DEV, dtype=torch.bfloat16)
    bad_calls = {
        "decode q rank": ("paged_decode", (q[0], pool.k, pool.v, tables, ctx, 1, 0)),
        "decode dtype": ("paged_decode", (q.float(), pool.k, pool.v, tables, ctx, 1, 0)),
        "decode layer": ("paged_decode", (q, pool.k, pool.v, tables, ctx, 2, 0)),
        "decode tables": ("paged_decode", (q, pool.k, pool.v, tables[:3], ctx, 1, 0)),
        "decode ctx dtype": ("paged_decode", (q, pool.k, pool.v, tables, ctx.float(), 1, 0)),
        "decode block size": ("paged_decode", (q, zero.k, zero.v, tables, ctx, 0, 0)),
        "append shapes": ("kv_append", (pool.k, pool.v, 1, q, q[:2], ctx)),
        "append heads": ("kv_append", (pool.k, pool.v, 1, q[:, :4], q[:, :4], ctx)),
        "append slots": ("kv_append", (pool.k, pool.v, 1, q, q, ctx[:2])),
        "prefill table": ("paged_prefill", (q, pool.k, pool.v, tables[0, :1], 100, 1)),
        "prefill start": ("paged_prefill", (q, pool.k, pool.v, tables[0], -1, 1)),
        "prefill block size": ("paged_prefill", (q, zero.k, zero.v, tables[0], 0, 0)),
    }
    for name, (fn, args) in bad_calls.items():
        with pytest.raises(ValueError) as want:
            getattr(ext, fn)(*args)
        with pytest.raises(ValueError) as got:
            getattr(_ctypes_ops, fn)(*args)
        assert str(got.value) == str(want.value), name
