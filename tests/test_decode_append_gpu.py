"""The fused KV append + decode attention (mgi_paged_decode_append) on the
MI355X against the two separate calls it replaces: kv_append of the step's
rows, then paged decode over the updated pool (the reference's order in
KVCacheCausalSelfAttention.forward_decode_batch, minivllm/attention.py:370-416).

Both run on identical copies of one pool; the outputs and every byte of both
pools must be identical (the fused kernel writes a row's slot before its
wavefront reads the block, so attention sees the same pool). Rows cover the
decode step's cases: the slot of the sequence's last position (the fused
write), padding (slot -1), a slot in a block no table uses, a slot past the
pool, and a sequence with no context whose row still lands. Both splits of
the fast kernel (even, partitions), every dtype, the lane layouts of head
dims 8 to 256, and the shapes that take the separate append kernel
(generic-path head dims, rows of another dtype, a strided head dim) are
checked; then the high-batch step at full size (B=256, 32 heads, bf16,
contexts 128-2048, a fragmented 32768-block pool, 10 % padding rows).
"""
from __future__ import annotations

import pytest
import torch

from minivllm import hip_paged_decode as hpd
from minivllm.kv_block_pool import KVBlockPool

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bits(t: torch.Tensor) -> torch.Tensor:
    return t.view({2: torch.int16, 4: torch.int32}[t.element_size()])


def step_case(B, H, D, S, ctx_lo, ctx_hi, dtype, seed, kinds=("tail", "pad", "free", "out", "empty")):
    """A decode step: contexts (with the new token) ~ U[ctx_lo, ctx_hi],
    scattered tables, and per row a slot kind drawn from `kinds`:
    tail  -- the slot of the sequence's last position (what decode writes)
    pad   -- -1 (skipped)
    free  -- a slot in a block no table uses
    out   -- a slot past the pool (skipped)
    empty -- context 0 and a slot in a block no table uses"""
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (B,), generator=g)
    kind = [kinds[int(i)] for i in torch.randint(0, len(kinds), (B,), generator=g)]
    kind[0] = "tail"
    for b in range(B):
        if kind[b] == "empty":
            ctx[b] = 0
    nblk = (ctx + S - 1) // S
    M = max(1, int(nblk.max()))
    n_free = B + 3
    N = int(nblk.sum()) + n_free
    perm = torch.randperm(N, generator=g)
    tables = torch.full((B, M), -1, dtype=torch.int64)
    used = 0
    for b in range(B):
        n = int(nblk[b])
        tables[b, :n] = perm[used:used + n]
        used += n
    free_blocks = perm[used:]
    slots = torch.empty(B, dtype=torch.int64)
    for b in range(B):
        c = int(ctx[b])
        if kind[b] == "tail":
            slots[b] = tables[b, (c - 1) // S] * S + (c - 1) % S
        elif kind[b] == "pad":
            slots[b] = -1
        elif kind[b] == "out":
            slots[b] = N * S + int(torch.randint(0, 5, (1,), generator=g))
        else:  # free, empty: distinct blocks, any offset
            slots[b] = free_blocks[b % len(free_blocks)] * S + int(torch.randint(0, S, (1,), generator=g))
    gd = torch.Generator(device=DEV).manual_seed(seed + 1)
    pool = KVBlockPool(2, N, S, H, D, device=DEV, dtype=dtype)
    pool.k.normal_(generator=gd)
    pool.v.normal_(generator=gd)
    q = torch.randn((B, H, D), generator=gd, device=DEV).to(dtype)
    kv = torch.randn((B, 2, H, D), generator=gd, device=DEV).to(dtype)
    return dict(q=q, pool=pool, tables=tables.to(DEV), ctx=ctx.to(DEV), slots=slots.to(DEV),
                k=kv[:, 0], v=kv[:, 1], kinds=kind)


def copy_pool(pool: KVBlockPool) -> KVBlockPool:
    p = KVBlockPool(pool.n_layer, pool.num_blocks, pool.block_size, pool.n_head, pool.head_dim, device=DEV,
                    dtype=pool.dtype)
    p.k.copy_(pool.k)
    p.v.copy_(pool.v)
    return p


def run_both(c, layer=1, split_tokens=0, k=None, v=None):
    k = c["k"] if k is None else k
    v = c["v"] if v is None else v
    print(f"  fused append+decode B={c['q'].shape[0]} H={c['q'].shape[1]} D={c['q'].shape[2]} "
          f"S={c['pool'].block_size} {c['q'].dtype} k{tuple(k.stride())} {k.dtype} split={split_tokens}",
          flush=True)
    sep, fused = copy_pool(c["pool"]), copy_pool(c["pool"])
    with torch.inference_mode():
        hpd.kv_append(sep, layer, k, v, c["slots"])
        out_sep = hpd.paged_attention_batch_hip(c["q"], sep, c["tables"], c["ctx"], layer,
                                                split_tokens=split_tokens)
        out_fused = hpd.paged_attention_batch_append_hip(c["q"], fused, c["tables"], c["ctx"], layer, k, v,
                                                         c["slots"], split_tokens=split_tokens)
    torch.cuda.synchronize()
    return out_sep, out_fused, sep, fused


def assert_identical(out_sep, out_fused, sep, fused):
    assert torch.isfinite(out_fused.float()).all()
    assert torch.equal(bits(out_fused), bits(out_sep))
    assert torch.equal(bits(fused.k), bits(sep.k))
    assert torch.equal(bits(fused.v), bits(sep.v))


CASES = [
    # B, H, D, S, ctx_lo, ctx_hi, split_tokens -- even split, partitions, one
    # partition, and the lane layouts (D 8 .. 256, full and partial head groups)
    (7, 8, 128, 16, 1, 300, 0),
    (7, 8, 128, 16, 1, 300, 64),
    (33, 4, 64, 32, 1, 700, 0),
    (64, 32, 128, 16, 512, 4096, 0),
    (3, 2, 256, 16, 1, 40, 0),
    (20, 6, 96, 16, 1, 400, 0),
    (5, 3, 8, 8, 1, 90, 0),
    (300, 4, 128, 16, 1, 64, 0),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("B,H,D,S,lo,hi,split", CASES)
def test_fused_matches_append_then_decode(dtype, B, H, D, S, lo, hi, split):
    c = step_case(B, H, D, S, lo, hi, dtype, seed=B + D)
    assert_identical(*run_both(c, split_tokens=split))


def test_every_row_kind_lands_in_the_fused_write():
    """All rows the decode case: their slots hold the new rows afterwards, and
    nothing else in the pool changed."""
    c = step_case(40, 8, 128, 16, 1, 500, torch.bfloat16, seed=3, kinds=("tail",))
    before_k = c["pool"].k.clone()
    out_sep, out_fused, sep, fused = run_both(c)
    assert_identical(out_sep, out_fused, sep, fused)
    S = fused.block_size
    blk, off = c["slots"] // S, c["slots"] % S
    assert torch.equal(bits(fused.k[1, blk, off]), bits(c["k"]))
    changed = (bits(fused.k) != bits(before_k)).any(dim=-1).any(dim=-1)
    assert int(changed.sum()) == 40 and not bool(changed[0].any())


@pytest.mark.parametrize("variant", ["generic_head_dim", "f32_rows_into_bf16", "strided_head_dim"])
def test_shapes_taking_the_separate_append_kernel(variant):
    """Shapes the fused write does not take run the append kernel first, with
    the same result as the two calls."""
    if variant == "generic_head_dim":
        c = step_case(9, 4, 24, 16, 1, 200, torch.bfloat16, seed=5)
        assert_identical(*run_both(c))
    elif variant == "f32_rows_into_bf16":
        c = step_case(9, 4, 128, 16, 1, 200, torch.bfloat16, seed=6)
        g = torch.Generator(device=DEV).manual_seed(9)
        k = torch.randn(c["k"].shape, generator=g, device=DEV)
        v = torch.randn(c["v"].shape, generator=g, device=DEV)
        assert_identical(*run_both(c, k=k, v=v))
    else:
        c = step_case(9, 4, 128, 16, 1, 200, torch.bfloat16, seed=7)
        kt = c["k"].transpose(1, 2).contiguous().transpose(1, 2)   # head dim stride H
        vt = c["v"].transpose(1, 2).contiguous().transpose(1, 2)
        assert kt.stride(2) != 1
        assert_identical(*run_both(c, k=kt, v=vt))


@pytest.mark.parametrize("dtype,split", [(torch.bfloat16, 0), (torch.float32, 0), (torch.bfloat16, 64)],
                         ids=["bf16_even", "f32_even", "bf16_partitions"])
def test_int32_tables_lengths_and_slots(dtype, split):
    """int32 block tables, context lengths and slot mapping (the fused write
    reads the slot of a tail row and of a row with no blocks through the
    same index loads as the attention)."""
    c = step_case(21, 8, 128, 16, 1, 400, dtype, seed=17)
    for key in ("tables", "ctx", "slots"):
        c[key] = c[key].to(torch.int32)
    assert "empty" in c["kinds"] and "pad" in c["kinds"]
    assert_identical(*run_both(c, split_tokens=split))


def test_rows_from_a_fused_qkv_view():
    """The model's layout: k and v are views of one [B, 3, H, D] projection
    (row stride 3 H D), q a third view."""
    c = step_case(16, 8, 128, 16, 1, 600, torch.bfloat16, seed=11)
    g = torch.Generator(device=DEV).manual_seed(12)
    qkv = torch.randn((16, 3, 8, 128), generator=g, device=DEV).to(torch.bfloat16)
    c["q"] = qkv[:, 0]
    assert_identical(*run_both(c, k=qkv[:, 1], v=qkv[:, 2]))


def test_repeated_fused_steps_match_repeated_separate_steps():
    """Three decode steps in a row on one pool (each step's context one longer,
    its slot the next position): the pools and outputs stay identical."""
    B, H, D, S = 24, 8, 128, 16
    c = step_case(B, H, D, S, 100, 900, torch.bfloat16, seed=13, kinds=("tail",))
    sep, fused = copy_pool(c["pool"]), copy_pool(c["pool"])
    tables, ctx = c["tables"].clone(), c["ctx"].clone()
    g = torch.Generator(device=DEV).manual_seed(14)
    for step in range(3):
        ctx = ctx + 1
        cpu_t, cpu_c = tables.cpu(), ctx.cpu()
        if int(((cpu_c + S - 1) // S).max()) > cpu_t.shape[1]:
            break
        ok = cpu_t[torch.arange(B), (cpu_c - 1) // S] >= 0
        slots = torch.where(ok, cpu_t[torch.arange(B), ((cpu_c - 1) // S).clamp(max=cpu_t.shape[1] - 1)] * S
                            + (cpu_c - 1) % S, torch.full_like(cpu_c, -1)).to(DEV)
        kv = torch.randn((B, 2, H, D), generator=g, device=DEV).to(torch.bfloat16)
        q = torch.randn((B, H, D), generator=g, device=DEV).to(torch.bfloat16)
        with torch.inference_mode():
            hpd.kv_append(sep, 1, kv[:, 0], kv[:, 1], slots)
            o1 = hpd.paged_attention_batch_hip(q, sep, tables, ctx, 1)
            o2 = hpd.paged_attention_batch_append_hip(q, fused, tables, ctx, 1, kv[:, 0], kv[:, 1], slots)
        torch.cuda.synchronize()
        print(f"  step {step}", flush=True)
        assert_identical(o1, o2, sep, fused)


def test_high_batch_step_full_size():
    """B=256, H=32, D=128, bf16; contexts 128-2048 before the step; a
    fragmented 32768-block pool; 26 seeded rows (10 %) carry slot -1. The
    fused step against the append kernel then decode: outputs and both whole
    pools bit-identical."""
    B, H, D, S, N = 256, 32, 128, 16, 32768
    g = torch.Generator().manual_seed(0)
    ctx = torch.randint(128, 2049, (B,), generator=g)
    perm = torch.randperm(N, generator=g)
    M = int((ctx // S + 1).max())
    tables = torch.full((B, M), -1, dtype=torch.int64)
    used = 0
    for b in range(B):
        n = int(ctx[b] // S + 1)
        tables[b, :n] = perm[used:used + n]
        used += n
    slots = tables[torch.arange(B), ctx // S] * S + ctx % S
    pad = torch.randperm(B, generator=g)[: B // 10]
    slots[pad] = -1
    new_ctx = torch.where(slots >= 0, ctx + 1, ctx)
    gd = torch.Generator(device=DEV).manual_seed(1)
    pool = KVBlockPool(1, N, S, H, D, device=DEV, dtype=torch.bfloat16)
    pool.k.normal_(generator=gd)
    pool.v.normal_(generator=gd)
    q = torch.randn((B, H, D), generator=gd, device=DEV).to(torch.bfloat16)
    kv = torch.randn((B, 2, H, D), generator=gd, device=DEV).to(torch.bfloat16)
    c = dict(q=q, pool=pool, tables=tables.to(DEV), ctx=new_ctx.to(DEV), slots=slots.to(DEV),
             k=kv[:, 0], v=kv[:, 1])
    out_sep, out_fused, sep, fused = run_both(c, layer=0)
    del c["pool"], pool
    assert_identical(out_sep, out_fused, sep, fused)
