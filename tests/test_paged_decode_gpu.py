"""Parity of the HIP paged decode attention with the CPU oracle (MI355X).

Tolerances: fp32 within 1e-5 (rtol and atol, as the reference
tests pair them, tests/test_paged_attention.py:32); bf16 within 2e-2 and
fp16 within 2e-3 (its output rounding is 2^-11 relative) against the oracle
evaluated in double on the same 16-bit inputs; large logits 5e-4
(tests/test_triton_paged_decode.py:66-71). Small cases check every element;
benchmark-size cases check the C oracle on the drawn workload plus
size-independent properties: block-placement invariance (bit-exact),
partition-size invariance, single-token contexts (bit-exact) and finiteness
with NaN in every slot past a context.
"""
from __future__ import annotations

import math

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
F32_TOL = dict(rtol=1e-5, atol=1e-5)
BF16_TOL = dict(rtol=2e-2, atol=2e-2)
F16_TOL = dict(rtol=2e-3, atol=2e-3)


def tol_for(dtype):
    return {torch.float32: F32_TOL, torch.float16: F16_TOL}.get(dtype, BF16_TOL)


def hip(q, pool, tables, lens, layer, **kw):
    print(f"  hip decode B={q.shape[0]} H={q.shape[1]} D={q.shape[2]} S={pool.block_size} "
          f"dtype={q.dtype} kw={kw}", flush=True)
    with torch.inference_mode():
        out = hpd.paged_attention_batch_hip(q.to(DEV), pool, tables.to(DEV), lens.to(DEV), layer, **kw)
    torch.cuda.synchronize()
    assert out.dtype == q.dtype and tuple(out.shape) == tuple(q.shape)
    return out.float().cpu().numpy()


def oracle_args(q, pool, tables, lens, layer):
    return (fx.to_numpy(q), fx.to_numpy(pool.k), fx.to_numpy(pool.v), tables.cpu().numpy(),
            lens.cpu().numpy(), layer)


# ------------------------------------------------ reference test fixtures

@pytest.mark.parametrize("case", [0, 1, 2])
def test_reference_unit_cases(case):
    pool, _, cases = fx.reference_case_2026()
    _, q, tables, lens = cases[case]
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, 0)
    want = ora.paged_attention_online_v1(*oracle_args(q, pool, tables, lens, 0))
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, **F32_TOL)


@pytest.mark.parametrize("make", [fx.padding_case_11, fx.probe_case_2026])
def test_nan_pool_cases(make):
    pool, q, tables, lens = make()
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, 0)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ora.dense_gold(*oracle_args(q, pool, tables, lens, 0)), **F32_TOL)


@pytest.mark.parametrize("bs,length,batch,dim", [
    (16, 1, 1, 32), (16, 15, 2, 32), (16, 16, 2, 32), (16, 17, 4, 32), (16, 65, 4, 32),
    (16, 129, 4, 32), (16, 257, 2, 32), (8, 37, 3, 16), (32, 129, 3, 64), (16, 33, 2, 48)])
def test_kernel_matches_oracle_reference_grid(bs, length, batch, dim):
    """The GPU grid of tests/test_triton_paged_decode.py:51-64 (8 heads, scale 0.3)."""
    q, pool, tables, lens, layer = fx.build_case(batch, length, 8, dim, bs, "mixed", scale=0.3)
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ora.dense_gold(*oracle_args(q, pool, tables, lens, layer)), **F32_TOL)


@pytest.mark.parametrize("batch,length", [(1, 1), (1, 15), (1, 16), (2, 17), (4, 33), (4, 64), (4, 65),
                                          (2, 128), (4, 129), (2, 256), (4, 257)])
def test_kernel_matches_reference_fused_decode_grid(batch, length):
    """The correctness grid of experiments/gpu_day6_fused_decode_ab.py:171-181
    (8 heads, head_dim 32, block 16, mixed lengths, seed 20261030 + B + L)
    against the dense closed form, at that script's 2e-4 and at 1e-5."""
    q, pool, tables, lens, layer = fx.build_case(batch, length, 8, 32, 16, "mixed", seed=20261030 + batch + length)
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer)
    want = ora.dense_gold(*oracle_args(q, pool, tables, lens, layer))
    np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-4)
    np.testing.assert_allclose(got, want, **F32_TOL)


def test_large_logits_stable():
    q, pool, tables, lens, layer = fx.build_case(2, 65, 4, 32, 16, "mixed", scale=8.0)
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ora.dense_gold(*oracle_args(q, pool, tables, lens, layer)),
                               rtol=5e-4, atol=5e-4)


# ------------------------------------------------------- shape / path sweep

def _small_case(B, H, D, S, ctx, dtype, seed, N=None, layers=2, layer=1):
    g = torch.Generator().manual_seed(seed)
    nblk = [(c + S - 1) // S for c in ctx]
    N = N or sum(nblk) + 5
    M = max(max(nblk), 1)
    pool = KVBlockPool(layers, N, S, H, D, dtype=dtype)
    pool.k.copy_(torch.randn(pool.k.shape, generator=g).to(dtype))
    pool.v.copy_(torch.randn(pool.v.shape, generator=g).to(dtype))
    perm = torch.randperm(N, generator=g)
    tables = torch.full((B, M), -1, dtype=torch.int64)
    used = 0
    for b in range(B):
        tables[b, : nblk[b]] = perm[used: used + nblk[b]]
        # NaN past the context in the last block
        if ctx[b] % S:
            last = int(perm[used + nblk[b] - 1])
            pool.k[layer, last, ctx[b] % S:] = float("nan")
            pool.v[layer, last, ctx[b] % S:] = float("nan")
        used += nblk[b]
    q = torch.randn((B, H, D), generator=g).to(dtype)
    return q, pool, tables, torch.tensor(ctx, dtype=torch.int64), layer


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
@pytest.mark.parametrize("S,H", [(16, 32), (8, 3), (32, 5)])
@pytest.mark.parametrize("split", [0, 16, 48, 256])
def test_fast_path_shapes(dtype, D, S, H, split):
    ctx = [1, S - 1, S, 3 * S + 1, 300, 513]
    q, pool, tables, lens, layer = _small_case(len(ctx), H, D, S, ctx, dtype, seed=D + S + H + split)
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer, split_tokens=split)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ora.dense_gold(*oracle_args(q, pool, tables, lens, layer)),
                               **tol_for(dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,S", [(4, 4), (12, 5), (100, 16), (8, 1), (300, 3), (64, 4), (64, 12)])
def test_generic_path_shapes(dtype, D, S):
    ctx = [1, 7, 40, 65]
    q, pool, tables, lens, layer = _small_case(len(ctx), 3, D, S, ctx, dtype, seed=D * 7 + S)
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer)
    assert np.isfinite(got).all()
    tol = F32_TOL if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
    np.testing.assert_allclose(got, ora.dense_gold(*oracle_args(q, pool, tables, lens, layer)), **tol)


@pytest.mark.parametrize("split", [0, 64], ids=["auto", "partitions"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_int32_indices_and_strided_q(dtype, split):
    ctx = [5, 77, 190]
    q, pool, tables, lens, layer = _small_case(3, 8, 128, 16, ctx, dtype, seed=11)
    wide = torch.randn(3, 8, 256).to(dtype)
    wide[..., ::2] = q
    q_strided = wide[..., ::2]
    assert q_strided.stride(-1) == 2
    # a table wider than one partition, so the automatic split divides the work
    wide_tables = torch.nn.functional.pad(tables, (0, 40 - tables.shape[1]), value=-1)
    assert (split == 0) == (hpd._native.lib().mgi_paged_decode_balanced_waves(3, 8, 128, 16, 40, split) > 0)
    got = hip(q_strided, fx.pool_to_device(pool, DEV), wide_tables.int(), lens.int(), layer,
              split_tokens=split)
    np.testing.assert_allclose(got, ora.dense_gold(*oracle_args(q, pool, tables, lens, layer)),
                               **tol_for(dtype))


def test_zero_context_row_gives_zeros():
    q, pool, tables, lens, layer = _small_case(3, 4, 64, 16, [9, 40, 3], torch.float32, seed=5)
    lens[1] = 0
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer)
    assert (got[1] == 0).all()
    keep = [0, 2]
    want = ora.dense_gold(*oracle_args(q[keep], pool, tables[keep], lens[keep], layer))
    np.testing.assert_allclose(got[keep], want, **F32_TOL)


def test_out_of_range_table_entries_inside_context_are_masked():
    q, pool, tables, lens, layer = _small_case(2, 4, 128, 16, [64, 64], torch.float32, seed=9)
    bad = tables.clone()
    bad[0, 1] = pool.num_blocks + 3
    bad[1, 2] = -1
    got = hip(q, fx.pool_to_device(pool, DEV), bad, lens, layer, split_tokens=32)
    want = c_oracle.paged_decode(*oracle_args(q, pool, bad, lens, layer))
    np.testing.assert_allclose(got, want, **F32_TOL)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_single_token_context_returns_value_row_exactly(dtype):
    q, pool, tables, lens, layer = _small_case(4, 32, 128, 16, [1, 1, 1, 1], dtype, seed=3)
    dpool = fx.pool_to_device(pool, DEV)
    with torch.inference_mode():
        out = hpd.paged_attention_batch_hip(q.to(DEV), dpool, tables.to(DEV), lens.to(DEV), layer)
    want = dpool.v[layer, tables[:, 0].to(DEV), 0]
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(out.view(bits), want.view(bits))


# ------------------------------------------------- benchmark-size parity

def _check_against_c_oracle(w, dtype, seqs=None):
    with torch.inference_mode():
        out = hpd.paged_attention_batch_hip(w.q, w.pool, w.tables, w.ctx, w.layer)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    if seqs is not None:
        sub = fx.DecodeWorkload(w.q[seqs], w.pool, w.tables[seqs], w.ctx[seqs], w.layer, w.meta)
        got = got[seqs]
    else:
        sub = w
    args = list(sub.compact_host())
    if dtype == torch.float16:  # exact in float32; the C oracle takes float32 or bfloat16 bits
        args[:3] = [np.asarray(x, dtype=np.float32) for x in args[:3]]
    want = c_oracle.paged_decode(*args, threads=fx.oracle_threads())
    np.testing.assert_allclose(got, want, **tol_for(dtype))
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_decode_microbench_shape_matches_oracle(dtype):
    """B=64, H=32, D=128, S=16, ctx ~ U[512, 4096], 20k-block permuted pool."""
    print(f"  workload B=64 H=32 D=128 ctx U[512,4096] N=20000 {dtype}", flush=True)
    w = fx.make_decode_workload(64, 32, 128, 16, 20000, 512, 4096, dtype, DEV, seed=0)
    _check_against_c_oracle(w, dtype)


def test_decode_microbench_invariances():
    w = fx.make_decode_workload(64, 32, 128, 16, 20000, 512, 4096, torch.float32, DEV, seed=1)
    with torch.inference_mode():
        base = hpd.paged_attention_batch_hip(w.q, w.pool, w.tables, w.ctx, w.layer)
        # partition size only changes the order of the merge
        for split in (64, 512, 1024, 4096):
            print(f"  split_tokens={split}", flush=True)
            other = hpd.paged_attention_batch_hip(w.q, w.pool, w.tables, w.ctx, w.layer,
                                                  split_tokens=split)
            torch.testing.assert_close(other, base, **F32_TOL)
        # physical placement of blocks does not enter the arithmetic: bit-exact
        g = torch.Generator(device=DEV).manual_seed(5)
        perm = torch.randperm(w.pool.num_blocks, generator=g, device=DEV)
        inv = torch.argsort(perm)
        moved = KVBlockPool(1, w.pool.num_blocks, 16, 32, 128, device=DEV, dtype=torch.float32)
        moved.k.copy_(w.pool.k[:, perm])
        moved.v.copy_(w.pool.v[:, perm])
        tables2 = torch.where(w.tables >= 0, inv[w.tables.clamp(min=0)], w.tables)
        again = hpd.paged_attention_batch_hip(w.q, moved, tables2, w.ctx, w.layer)
    assert torch.equal(again.view(torch.int32), base.view(torch.int32))


# (own share in 16ths, ticket claims per wave) of the balanced split: the
# library's default, no second tier, nearly everything by ticket, and half.
TIERS = [None, (16, 0), (1, 16), (8, 64)]


def _set_tiers(monkeypatch, tiers):
    if tiers is not None:
        monkeypatch.setenv("MINIVLLM_HIP_BAL_TIER1", str(tiers[0]))
        monkeypatch.setenv("MINIVLLM_HIP_BAL_TIER2", str(tiers[1]))


@pytest.mark.parametrize("tiers", TIERS)
@pytest.mark.parametrize("B", [7, 200, 1000])
def test_balanced_split_with_empty_and_one_token_contexts(B, tiers, monkeypatch):
    """The automatic split spreads every sequence's blocks over the waves'
    own claims and the ticket claims (several sequences per claim, several
    claims per sequence); rows with no context are zeros and one-token rows
    return their value row."""
    _set_tiers(monkeypatch, tiers)
    print(f"  tiers={tiers}", flush=True)
    S, H, D, M = 16, 4, 64, 80
    g = torch.Generator().manual_seed(B)
    choices = torch.tensor([0, 1, 2, 15, 16, 17, 300, 1000, M * S])
    ctx = choices[torch.randint(len(choices), (B,), generator=g)]
    ctx[0], ctx[-1] = 0, M * S
    N = int(((ctx + S - 1) // S).sum()) + 8
    print(f"  balanced split B={B} N={N}", flush=True)
    q, pool, tables, lens, layer = _small_case(B, H, D, S, ctx.tolist(), torch.float32, seed=B, N=N)
    assert tables.shape[1] <= M
    tables = torch.nn.functional.pad(tables, (0, M - tables.shape[1]), value=-1)
    assert hpd._native.lib().mgi_paged_decode_workspace_bytes(B, H, D, S, M, 0) > 0
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer)
    want = c_oracle.paged_decode(*oracle_args(q, pool, tables, lens, layer))
    np.testing.assert_allclose(got, want, **F32_TOL)
    assert (got[ctx.numpy() == 0] == 0).all()


@pytest.mark.parametrize("B", [4096, 4100])
def test_largest_balanced_batch_and_the_partition_fallback(B):
    """The balanced split holds the batch's block prefix sums in LDS, 4096
    sequences at most (64 per lane of its scan); one more row takes the
    partition split. Both against the C oracle. At this batch the library
    splits only tables wider than one 2048-token partition, so the table
    has 130 blocks and a few contexts fill it."""
    S, H, D, M = 16, 4, 64, 130
    g = torch.Generator().manual_seed(B)
    choices = torch.tensor([0, 1, 15, 16, 17, 40, 200, M * S])
    ctx = choices[torch.randint(len(choices), (B,), generator=g)]
    N = int(((ctx + S - 1) // S).sum()) + 8
    q, pool, tables, lens, layer = _small_case(B, H, D, S, ctx.tolist(), torch.float32, seed=B, N=N)
    tables = torch.nn.functional.pad(tables, (0, M - tables.shape[1]), value=-1)
    waves = hpd._native.lib().mgi_paged_decode_balanced_waves(B, H, D, S, M, 0)
    assert (waves > 0) == (B <= 4096), waves
    print(f"  B={B} balanced waves per head group {waves}", flush=True)
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer)
    want = c_oracle.paged_decode(*oracle_args(q, pool, tables, lens, layer))
    np.testing.assert_allclose(got, want, **F32_TOL)
    assert (got[ctx.numpy() == 0] == 0).all()


@pytest.mark.parametrize("tiers", [None, (1, 16)])
def test_balanced_split_ignores_stale_workspace(tiers, monkeypatch):
    """The workspace is used as found: NaN bytes, zeros, or ticket counters
    left at 1 give the same output, bit for bit, as a fresh workspace."""
    _set_tiers(monkeypatch, tiers)
    print(f"  stale workspace tiers={tiers} B=64 H=32 D=128 bf16 ctx U[512,1024]", flush=True)
    w = fx.make_decode_workload(64, 32, 128, 16, 5000, 512, 1024, torch.bfloat16, DEV, seed=3,
                                poison=False, table_width=64)
    lib = hpd._native.lib()
    B, H, D = w.q.shape
    L, N, S = w.pool.k.shape[:3]
    M = w.tables.shape[1]
    assert lib.mgi_paged_decode_balanced_waves(B, H, D, S, M, 0) > 0
    ws_bytes = int(lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, 0))

    def call(ws):
        out = torch.empty_like(w.q)
        st = lib.mgi_paged_decode(
            out.data_ptr(), hpd._native.strides(out), w.q.data_ptr(), hpd._native.strides(w.q),
            w.pool.k.data_ptr(), w.pool.v.data_ptr(), hpd._native.strides(w.pool.k),
            hpd._native.strides(w.pool.v), hpd._native.DTYPE_CODES[w.q.dtype],
            w.tables.data_ptr(), hpd._native.strides(w.tables), hpd._native.ITYPE_CODES[w.tables.dtype],
            w.ctx.data_ptr(), w.ctx.stride(0), hpd._native.ITYPE_CODES[w.ctx.dtype],
            B, H, D, S, N, M, L, int(w.layer), 1.0 / math.sqrt(D), 0, ws.data_ptr(), ws_bytes,
            hpd._native.stream_handle(DEV))
        hpd._native.check(st)
        torch.cuda.synchronize()
        return out

    base = hpd.paged_attention_batch_hip(w.q, w.pool, w.tables, w.ctx, w.layer)
    torch.cuda.synchronize()
    assert torch.isfinite(base.float()).all()
    n_groups = H // 4
    for name in ("nan", "zero", "one"):
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        if name == "nan":
            ws.fill_(0xFF)
        elif name == "zero":
            ws.zero_()
        else:
            ws.fill_(0xFF)
            ws[ws_bytes - 4 * n_groups:].view(torch.int32).fill_(1)
        for rep in range(2):  # the second call finds the first call's counters
            got = call(ws)
            assert torch.equal(got.view(torch.int16), base.view(torch.int16)), (name, rep)


@pytest.mark.parametrize("split", [0, 256], ids=["auto", "partitions"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_few_sequences_many_partials(dtype, split):
    """Few (sequence, head group) pairs with many partials each: the merge
    runs several wavefronts per workgroup (B=3, 4 heads, contexts of 5k-12k
    tokens split over hundreds of claims or 256-token partitions)."""
    ctx = [5001, 12000, 7777]
    q, pool, tables, lens, layer = _small_case(3, 4, 128, 16, ctx, dtype, seed=31)
    got = hip(q, fx.pool_to_device(pool, DEV), tables, lens, layer, split_tokens=split)
    want = c_oracle.paged_decode(*oracle_args(q, pool, tables, lens, layer))
    np.testing.assert_allclose(got, want, **tol_for(dtype))


def test_long_context_split_decode():
    """B=8, H=32, D=128, bf16, ctx ~ U[32768, 131072] over a 65536-block pool."""
    print("  workload B=8 ctx U[32768,131072] N=65536 bf16", flush=True)
    w = fx.make_decode_workload(8, 32, 128, 16, 65536, 32768, 131072, torch.bfloat16, DEV, seed=0,
                                poison=False)
    base = _check_against_c_oracle(w, torch.bfloat16)   # all 8 sequences
    with torch.inference_mode():
        for split in (256, 512, 1024, 2048):
            print(f"  split_tokens={split}", flush=True)
            other = hpd.paged_attention_batch_hip(w.q, w.pool, w.tables, w.ctx, w.layer,
                                                  split_tokens=split)
            torch.testing.assert_close(other.float(), base.float(), **BF16_TOL)


# ------------------------------------------------------------ any finite scale

@pytest.mark.parametrize("scale", [-0.3, 0.0], ids=["neg", "zero"])
@pytest.mark.parametrize("split", [0, 64], ids=["balanced", "partitions"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_any_finite_scale_matches_c_oracle(dtype, split, scale):
    """mgi_paged_decode with a negative or zero scale (the torch wrapper
    always passes 1/sqrt(D)) against the C oracle: the kernels scale scores
    before taking maxima, so any finite scale is exact."""
    B, H, D, S = 24, 8, 128, 16
    g = torch.Generator().manual_seed(41)
    ctx = torch.randint(0, 600, (B,), generator=g).tolist()
    q, pool, tables, lens, layer = _small_case(B, H, D, S, ctx, dtype, seed=41)
    dpool = fx.pool_to_device(pool, DEV)
    qd, td, ld = q.to(DEV), tables.to(DEV), lens.to(DEV)
    lib = hpd._native.lib()
    L, N = dpool.k.shape[:2]
    M = td.shape[1]
    ws_bytes = int(lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, split))
    ws = torch.full((max(ws_bytes, 4) // 4,), float("nan"), device=DEV)
    out = torch.full_like(qd, float("nan"))
    print(f"  hip decode scale={scale} split={split} B={B} H={H} D={D} dtype={dtype}", flush=True)
    hpd._native.check(lib.mgi_paged_decode(
        out.data_ptr(), hpd._native.strides(out), qd.data_ptr(), hpd._native.strides(qd),
        dpool.k.data_ptr(), dpool.v.data_ptr(), hpd._native.strides(dpool.k), hpd._native.strides(dpool.v),
        hpd._native.DTYPE_CODES[dtype], td.data_ptr(), hpd._native.strides(td), hpd._native.ITYPE_CODES[td.dtype],
        ld.data_ptr(), ld.stride(0), hpd._native.ITYPE_CODES[ld.dtype],
        B, H, D, S, N, M, L, layer, float(scale), split, ws.data_ptr(), ws_bytes, hpd._native.stream_handle(DEV)))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    want = c_oracle.paged_decode(*oracle_args(q, pool, tables, lens, layer), scale=scale)
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, want, **tol_for(dtype))


@pytest.mark.parametrize("split", [0, 64], ids=["balanced", "partitions"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_strided_outputs_match_contiguous(dtype, split):
    """mgi_paged_decode writes through any output strides: a head-major view,
    an odd row stride and an element stride of 2 give the contiguous output
    bit for bit, and the columns between the elements stay untouched."""
    B, H, D, S = 16, 8, 128, 16
    g = torch.Generator().manual_seed(43)
    ctx = torch.randint(1, 900, (B,), generator=g).tolist()
    q, pool, tables, lens, layer = _small_case(B, H, D, S, ctx, dtype, seed=43)
    dpool = fx.pool_to_device(pool, DEV)
    qd, td, ld = q.to(DEV), tables.to(DEV), lens.to(DEV)
    lib = hpd._native.lib()
    L, N = dpool.k.shape[:2]
    M = td.shape[1]
    ws_bytes = int(lib.mgi_paged_decode_workspace_bytes(B, H, D, S, M, split))
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=DEV)

    def call(out):
        print(f"  hip decode split={split} dtype={dtype} out strides={tuple(out.stride())}", flush=True)
        hpd._native.check(lib.mgi_paged_decode(
            out.data_ptr(), hpd._native.strides(out), qd.data_ptr(), hpd._native.strides(qd),
            dpool.k.data_ptr(), dpool.v.data_ptr(), hpd._native.strides(dpool.k),
            hpd._native.strides(dpool.v), hpd._native.DTYPE_CODES[dtype], td.data_ptr(),
            hpd._native.strides(td), hpd._native.ITYPE_CODES[td.dtype], ld.data_ptr(), ld.stride(0),
            hpd._native.ITYPE_CODES[ld.dtype], B, H, D, S, N, M, L, layer, 1.0 / math.sqrt(D), split,
            ws.data_ptr(), ws_bytes, hpd._native.stream_handle(DEV)))
        torch.cuda.synchronize()
        return out

    bits = torch.int32 if dtype == torch.float32 else torch.int16
    base = call(torch.full_like(qd, float("nan")))
    head_major = call(torch.full((H, B, D), float("nan"), device=DEV, dtype=dtype).permute(1, 0, 2))
    wide = torch.full((B, H, D + 5), float("nan"), device=DEV, dtype=dtype)
    odd = call(wide[..., :D])
    strided = torch.full((B, H, 2 * D), float("nan"), device=DEV, dtype=dtype)
    every_other = call(strided[..., ::2])
    for got in (head_major, odd, every_other):
        assert torch.equal(got.contiguous().view(bits), base.view(bits))
    assert torch.isnan(wide[..., D:]).all() and torch.isnan(strided[..., 1::2]).all()
    want = c_oracle.paged_decode(*oracle_args(q, pool, tables, lens, layer))
    np.testing.assert_allclose(base.float().cpu().numpy(), want, **tol_for(dtype))
