"""Parity of the HIP KV append with the CPU oracle (MI355X): bit-exact.

The oracle (oracle.paged_decode.kv_append) writes row t to slot
slot_mapping[t] (block = slot // S, offset = slot % S) and skips slots < 0
or past the pool. On the GPU the whole pool is compared bytewise before and
after: exactly the named slots change, and they hold the new rows bit for
bit. The high-batch case (B=256, H=32, D=128, bf16, fragmented 32768-block
pool, 10% padding rows) then runs paged decode over the updated pool.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import _fixtures as fx
from minivllm import hip_paged_decode as hpd
from minivllm.kv_block_pool import KVBlockPool
from oracle import c_oracle
from oracle import paged_decode as ora

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bits(t: torch.Tensor) -> torch.Tensor:
    return t.view({2: torch.int16, 4: torch.int32}[t.element_size()])


def append(pool, layer, k, v, slots):
    print(f"  kv_append T={k.shape[0]} H={k.shape[1]} D={k.shape[2]} {k.dtype}->{pool.dtype} "
          f"strides={k.stride()} slots={slots.dtype}", flush=True)
    with torch.inference_mode():
        hpd.kv_append(pool, layer, k, v, slots)
    torch.cuda.synchronize()


def check_append(pool, before_k, before_v, layer, k_rows, v_rows, slots):
    """Changed slots == valid slots; their bytes == the oracle's."""
    S, N = pool.block_size, pool.num_blocks
    host_slots = slots.cpu().numpy()
    k_want, v_want = ora.kv_append(fx.to_numpy(before_k), fx.to_numpy(before_v), layer,
                                   fx.to_numpy(k_rows), fx.to_numpy(v_rows), host_slots)
    np.testing.assert_array_equal(fx.to_numpy(pool.k).view(np.uint8), k_want.view(np.uint8))
    np.testing.assert_array_equal(fx.to_numpy(pool.v).view(np.uint8), v_want.view(np.uint8))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_append_small_bit_exact(dtype):
    g = torch.Generator().manual_seed(1)
    L, N, S, H, D, T, layer = 3, 10, 16, 4, 64, 12, 2
    pool = KVBlockPool(L, N, S, H, D, device=DEV, dtype=dtype)
    pool.k.fill_(float("nan"))
    pool.v.fill_(float("nan"))
    before_k, before_v = pool.k.clone(), pool.v.clone()
    k = torch.randn(T, H, D, generator=g).to(dtype).to(DEV)
    v = torch.randn(T, H, D, generator=g).to(dtype).to(DEV)
    slots = torch.randperm(N * S, generator=g)[:T]
    slots[[0, 7]] = -1
    append(pool, layer, k, v, slots.to(DEV))
    check_append(pool, before_k, before_v, layer, k, v, slots)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("misaligned", [False, True])
def test_append_from_strided_qkv_view(dtype, misaligned):
    """k/v as column slices of a [T, 1, 3C] projection output (the model's layout)."""
    g = torch.Generator().manual_seed(2)
    T, H, D, S, N = 7, 8, 32, 16, 9
    C = H * D
    qkv = torch.randn(T, 1, 3 * C + 8, generator=g).to(dtype).to(DEV)  # rows 16-byte aligned
    base = 1 if misaligned else 0          # a 1-element shift forces the element path
    k = qkv[:, 0, base + C: base + 2 * C].view(T, H, D)
    v = qkv[:, 0, base + 2 * C: base + 3 * C].view(T, H, D)
    assert not k.is_contiguous()
    pool = KVBlockPool(1, N, S, H, D, device=DEV, dtype=dtype)
    pool.k.zero_()
    pool.v.zero_()
    before_k, before_v = pool.k.clone(), pool.v.clone()
    slots = torch.tensor([0, 17, 35, -1, 143, 50, 64], dtype=torch.int32)
    append(pool, 0, k, v, slots.to(DEV))
    check_append(pool, before_k, before_v, 0, k, v, slots)


def test_append_converts_f32_rows_into_bf16_pool_like_torch():
    g = torch.Generator().manual_seed(4)
    T, H, D, S, N = 6, 2, 40, 8, 5
    k = (torch.randn(T, H, D, generator=g) * 100).to(DEV)
    v = (torch.randn(T, H, D, generator=g) * 1e-3).to(DEV)
    pool = KVBlockPool(1, N, S, H, D, device=DEV, dtype=torch.bfloat16)
    pool.k.zero_()
    pool.v.zero_()
    slots = torch.tensor([3, 9, 39, 0, 20, 11], device=DEV)
    append(pool, 0, k, v, slots)
    blk, off = slots // S, slots % S
    assert torch.equal(bits(pool.k[0, blk, off]), bits(k.to(torch.bfloat16)))
    assert torch.equal(bits(pool.v[0, blk, off]), bits(v.to(torch.bfloat16)))


def test_negative_and_out_of_range_slots_write_nothing():
    T, H, D, S, N = 5, 4, 128, 16, 6
    pool = KVBlockPool(2, N, S, H, D, device=DEV, dtype=torch.bfloat16)
    pool.k.fill_(1.0)
    pool.v.fill_(2.0)
    before_k, before_v = pool.k.clone(), pool.v.clone()
    rows = torch.zeros(T, H, D, device=DEV, dtype=torch.bfloat16)
    slots = torch.tensor([-1, -5, N * S, N * S + 100, -(2**40)], device=DEV)
    append(pool, 1, rows, rows, slots)
    assert torch.equal(bits(pool.k), bits(before_k)) and torch.equal(bits(pool.v), bits(before_v))


def test_high_batch_append_then_decode():
    """B=256, H=32, D=128, bf16; ctx ~ U[128, 2048]; fragmented 32768-block pool;
    26 seeded rows (10%) carry slot -1. Append must be bit-exact over the whole
    pool; decode then attends ctx+1 tokens for appended rows, ctx for padded."""
    B, H, D, S, N = 256, 32, 128, 16, 32768
    g = torch.Generator().manual_seed(0)
    ctx = torch.randint(128, 2049, (B,), generator=g)
    perm = torch.randperm(N, generator=g)
    nblk_next = ctx // S + 1                       # blocks once position ctx is written
    M = int(nblk_next.max())
    tables = torch.full((B, M), -1, dtype=torch.int64)
    used = 0
    for b in range(B):
        n = int((ctx[b] + S - 1) // S)
        if ctx[b] % S == 0:
            n += 1                                 # position ctx opens a new block
        tables[b, :n] = perm[used: used + n]
        used += n
    slots = tables[torch.arange(B), ctx // S] * S + ctx % S
    pad = torch.randperm(B, generator=g)[: B // 10]
    slots[pad] = -1
    new_ctx = torch.where(slots >= 0, ctx + 1, ctx)

    gd = torch.Generator(device=DEV).manual_seed(1)
    pool = KVBlockPool(1, N, S, H, D, device=DEV, dtype=torch.bfloat16)
    pool.k.normal_(generator=gd)
    pool.v.normal_(generator=gd)
    before_k, before_v = pool.k.clone(), pool.v.clone()
    k_new = torch.randn((B, H, D), generator=gd, device=DEV).to(torch.bfloat16)
    v_new = torch.randn((B, H, D), generator=gd, device=DEV).to(torch.bfloat16)
    append(pool, 0, k_new, v_new, slots.to(DEV))

    # every byte outside the valid slots is unchanged; valid slots hold the rows
    valid = slots >= 0
    blk, off = (slots[valid] // S).to(DEV), (slots[valid] % S).to(DEV)
    for after, before, rows in ((pool.k, before_k, k_new), (pool.v, before_v, v_new)):
        changed = (bits(after) != bits(before)).any(dim=-1).any(dim=-1)[0]   # [N, S]
        expect = torch.zeros_like(changed)
        expect[blk, off] = True
        assert torch.equal(changed, expect)
        assert torch.equal(bits(after[0, blk, off]), bits(rows[valid.to(DEV)]))
    del before_k, before_v

    q = torch.randn((B, H, D), generator=gd, device=DEV).to(torch.bfloat16)
    w = fx.DecodeWorkload(q, pool, tables.to(DEV), new_ctx.to(DEV), 0, {})
    with torch.inference_mode():
        out = hpd.paged_attention_batch_hip(w.q, w.pool, w.tables, w.ctx, 0)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    want = c_oracle.paged_decode(*w.compact_host(), threads=fx.oracle_threads())
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-2)
