"""Seeded inputs for the paged-KV decode tests and the bench.

The small cases restate the reference tests' own recipes with the same seeds
and the same order of RNG draws, so the tensors equal the ones those tests
use:
  reference_case_2026   tests/test_paged_attention.py:12-47
  padding_case_11       tests/test_paged_attention_padding.py:12-32
  probe_case_2026       experiments/gpu_correctness_probe.py:35-56
  build_case            experiments/gpu_day6_fused_decode_ab.py:35-77
The large generators build the shapes of the benchmark workloads (random
block permutation of a big pool, ragged contexts, NaN in every slot past a
context).
"""
from __future__ import annotations

import math
import os

import numpy as np
import torch

from minivllm.kv_block_pool import KVBlockPool


# ------------------------------------------------------------ small cases

def reference_case_2026():
    """Pool L1 N4 S4 H2 D4 and q [2,2,4]; returns (pool, q, cases)."""
    torch.manual_seed(2026)
    pool = KVBlockPool(n_layer=1, num_blocks=4, block_size=4, n_head=2, head_dim=4, device="cpu")
    pool.k.copy_(torch.randn_like(pool.k))
    pool.v.copy_(torch.randn_like(pool.v))
    q = torch.randn(2, 2, 4)
    cases = [
        ("single_block_scaling", q[:1], torch.tensor([[2]]), torch.tensor([3])),
        ("cross_block_online_softmax", q[:1], torch.tensor([[0, 1]]), torch.tensor([6])),
        ("variable_lengths_padded_tables", q, torch.tensor([[0, 1], [2, -1]]), torch.tensor([6, 3])),
    ]
    return pool, q, cases


def padding_case_11():
    """NaN-poisoned pool with a mixed batch; returns (pool, q, tables, lengths)."""
    torch.manual_seed(11)
    pool = KVBlockPool(n_layer=1, num_blocks=3, block_size=4, n_head=2, head_dim=8)
    pool.k.fill_(float("nan"))
    pool.v.fill_(float("nan"))
    pool.k[0, 0, :2] = torch.randn(2, 2, 8)
    pool.v[0, 0, :2] = torch.randn(2, 2, 8)
    pool.k[0, 1, :4] = torch.randn(4, 2, 8)
    pool.v[0, 1, :4] = torch.randn(4, 2, 8)
    pool.k[0, 2, :1] = torch.randn(1, 2, 8)
    pool.v[0, 2, :1] = torch.randn(1, 2, 8)
    q = torch.randn(2, 2, 8)
    return pool, q, torch.tensor([[0, -1], [1, 2]]), torch.tensor([2, 5])


def probe_case_2026():
    """Varied lengths, cross-block, padded tables, NaN in unused KV."""
    torch.manual_seed(2026)
    k = torch.full((1, 4, 4, 2, 8), float("nan"))
    v = torch.full_like(k, float("nan"))
    for physical_block, valid_tokens in ((0, 4), (1, 2), (2, 3)):
        k[0, physical_block, :valid_tokens] = torch.randn(valid_tokens, 2, 8)
        v[0, physical_block, :valid_tokens] = torch.randn(valid_tokens, 2, 8)
    q = torch.randn(2, 2, 8)
    pool = KVBlockPool(n_layer=1, num_blocks=4, block_size=4, n_head=2, head_dim=8)
    pool.k.copy_(k)
    pool.v.copy_(v)
    return pool, q, torch.tensor([[0, 1], [2, -1]]), torch.tensor([6, 3])


def build_case(batch=2, length=128, heads=8, dim=32, block_size=16, layout="mixed",
               seed=20261030, scale=0.3):
    """Synthetic pre-filled paged KV on the CPU (float32, 2 layers, layer 1 used).

    Noncontiguous physical blocks from a seeded permutation, NaN in every
    unwritten slot, -1 table tails and a stride-2 q. Returns
    (q, pool, tables, lengths, layer).
    """
    g = torch.Generator(device="cpu").manual_seed(seed)
    if layout == "mixed":
        lengths = [max(1, length - (i % 4) * max(1, length // 7)) for i in range(batch)]
    elif layout == "fixed":
        lengths = [length] * batch
    else:
        raise ValueError("layout must be fixed/mixed")
    counts = [math.ceil(x / block_size) for x in lengths]
    n_phys = sum(counts) + 7
    layer = 1
    pool = KVBlockPool(2, n_phys, block_size, heads, dim, device="cpu", dtype=torch.float32)
    pool.k.fill_(float("nan"))
    pool.v.fill_(float("nan"))
    table = torch.full((batch, max(counts)), -1, dtype=torch.int64)
    order = torch.randperm(n_phys, generator=g).tolist()
    cur = 0
    for b, (length_b, blocks_b) in enumerate(zip(lengths, counts)):
        for logical in range(blocks_b):
            phys = order[cur]
            cur += 1
            table[b, logical] = phys
            valid = min(block_size, length_b - logical * block_size)
            pool.k[layer, phys, :valid] = torch.randn((valid, heads, dim), generator=g) * scale
            pool.v[layer, phys, :valid] = torch.randn((valid, heads, dim), generator=g) * scale
    q = torch.randn((batch, heads, 2 * dim), generator=g)[..., ::2].mul_(scale)
    return q, pool, table, torch.tensor(lengths, dtype=torch.int64), layer


# ------------------------------------------------------------ conversions

def to_numpy(t: torch.Tensor) -> np.ndarray:
    """Host numpy copy; bfloat16 becomes its uint16 bit patterns."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def pool_to_device(pool: KVBlockPool, device, dtype=None) -> KVBlockPool:
    """A copy of `pool` on `device` (optionally cast to `dtype`)."""
    dtype = dtype or pool.dtype
    out = KVBlockPool(pool.n_layer, pool.num_blocks, pool.block_size, pool.n_head, pool.head_dim,
                      device=device, dtype=dtype)
    out.k.copy_(pool.k.to(dtype))
    out.v.copy_(pool.v.to(dtype))
    return out


def oracle_threads() -> int:
    return max(1, min(16, len(os.sched_getaffinity(0))))


# ------------------------------------------------------ large workloads

class DecodeWorkload:
    """A paged decode-attention input of benchmark shape, resident on `device`."""

    def __init__(self, q, pool, tables, ctx, layer, meta):
        self.q, self.pool, self.tables, self.ctx, self.layer, self.meta = q, pool, tables, ctx, layer, meta

    def algorithmic_bytes(self) -> int:
        """Bytes the attention must move: valid K/V, q, out and the index reads.

        sum_b ctx_b*H*D*e*2 + B*H*D*(e_q + e_out) + sum_b ceil(ctx_b/S)*e_idx + B*e_idx
        """
        B, H, D = self.q.shape
        e = self.q.element_size()
        S = self.pool.block_size
        ctx = self.ctx.cpu().to(torch.int64)
        e_idx = self.tables.element_size()
        return int(ctx.sum()) * H * D * e * 2 + B * H * D * 2 * e + \
            int(((ctx + S - 1) // S).sum()) * e_idx + B * self.ctx.element_size()

    def compact_cpu(self) -> "DecodeWorkload":
        """The same workload on the CPU, its pool holding only the used blocks
        (tables remapped): the input of CPU baselines."""
        tables = self.tables.cpu()
        used = torch.unique(tables[tables >= 0])
        remap = torch.full((self.pool.num_blocks,), -1, dtype=torch.int64)
        remap[used] = torch.arange(used.numel())
        new_tables = torch.where(tables >= 0, remap[tables.clamp(min=0)], tables)
        dev_used = used.to(self.pool.k.device)
        L, N, S, H, D = self.pool.k.shape
        pool = KVBlockPool(1, used.numel(), S, H, D, dtype=self.pool.dtype)
        pool.k.copy_(self.pool.k[self.layer, dev_used][None])
        pool.v.copy_(self.pool.v[self.layer, dev_used][None])
        return DecodeWorkload(self.q.cpu(), pool, new_tables, self.ctx.cpu(), 0, dict(self.meta))

    def compact_host(self):
        """Host copies of only the used blocks (tables remapped) for the oracle."""
        tables = self.tables.cpu()
        used = torch.unique(tables[tables >= 0])
        remap = torch.full((self.pool.num_blocks,), -1, dtype=torch.int64)
        remap[used] = torch.arange(used.numel())
        new_tables = torch.where(tables >= 0, remap[tables.clamp(min=0)], tables)
        dev_used = used.to(self.pool.k.device)
        k = self.pool.k[self.layer, dev_used][None]
        v = self.pool.v[self.layer, dev_used][None]
        return (to_numpy(self.q), to_numpy(k), to_numpy(v), new_tables.numpy(),
                self.ctx.cpu().numpy(), 0)


def make_decode_workload(B, H, D, S, N, ctx_lo, ctx_hi, dtype, device, seed=0, fixed_ctx=None,
                         poison=True, table_width=None) -> DecodeWorkload:
    """Seeded decode input: ctx ~ U[ctx_lo, ctx_hi], blocks from randperm(N).

    Draws of the shape come from a CPU generator seeded `seed`; values (all
    N(0,1)) from a device generator seeded `seed + 1`. Slots past each
    context are NaN when `poison` (correctness runs).
    """
    g = torch.Generator(device="cpu").manual_seed(seed)
    if fixed_ctx is not None:
        ctx = torch.full((B,), int(fixed_ctx), dtype=torch.int64)
    else:
        ctx = torch.randint(ctx_lo, ctx_hi + 1, (B,), generator=g, dtype=torch.int64)
    nblk = (ctx + S - 1) // S
    M = table_width or int((max(ctx_hi, int(ctx.max())) + S - 1) // S)
    if int(nblk.sum()) > N:
        raise ValueError("pool too small for the drawn contexts")
    perm = torch.randperm(N, generator=g)
    tables = torch.full((B, M), -1, dtype=torch.int64)
    starts = torch.cumsum(nblk, 0) - nblk
    for b in range(B):
        tables[b, : nblk[b]] = perm[starts[b]: starts[b] + nblk[b]]
    gd = torch.Generator(device=device).manual_seed(seed + 1)
    pool = KVBlockPool(1, N, S, H, D, device=device, dtype=dtype)
    for t in (pool.k, pool.v):
        t.normal_(generator=gd)
    if poison:
        _poison_tails(pool, tables, ctx)
    q = torch.randn((B, H, D), generator=gd, device=device, dtype=torch.float32).to(dtype)
    meta = {"B": B, "H": H, "D": D, "S": S, "N": N, "ctx": [ctx_lo, ctx_hi] if fixed_ctx is None
            else fixed_ctx, "dtype": str(dtype).replace("torch.", ""), "seed": seed}
    return DecodeWorkload(q, pool, tables.to(device), ctx.to(device), 0, meta)


def _poison_tails(pool: KVBlockPool, tables: torch.Tensor, ctx: torch.Tensor) -> None:
    """NaN into every slot past each context and every block no table uses."""
    dev = pool.k.device
    S = pool.block_size
    used = torch.zeros(pool.num_blocks, dtype=torch.bool)
    used[tables[tables >= 0]] = True
    unused = (~used).nonzero().flatten().to(dev)
    nblk = (ctx + S - 1) // S
    last = tables[torch.arange(tables.shape[0]), nblk - 1].to(dev)
    n_last = (ctx - (nblk - 1) * S).to(dev)
    tail = torch.arange(S, device=dev)[None, :] >= n_last[:, None]            # [B, S]
    for t in (pool.k, pool.v):
        if unused.numel():
            t[0, unused] = float("nan")
        blocks = t[0, last]
        t[0, last] = torch.where(tail[:, :, None, None], torch.full_like(blocks, float("nan")), blocks)
