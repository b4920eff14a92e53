"""Pins the CPU oracle before it is trusted as the HIP kernels' checker.

Each oracle function is checked against
  * the reference tests' own fixtures and tolerances (seeded recipes restated
    in _fixtures.py): tests/test_paged_attention.py:26-47 (1e-5),
    tests/test_paged_attention_padding.py:12-32 (NaN pool, 1e-5),
    tests/test_triton_paged_decode.py:13-33 (8 (S, ctx) pairs, 1e-5);
  * closed forms: dense softmax attention, ctx = 1 -> V[0], identical keys ->
    mean(V), partition merge == unsplit;
  * invariances: physical block placement, partition size;
  * library routines: torch index_put_ for the KV write, torch's float ->
    bfloat16 cast for the rounding;
and planted mistakes (a dropped rescale, a wrong scale, a wrong head, an
off-by-one mask) must fail those same checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import _fixtures as fx
from oracle import c_oracle
from oracle import paged_decode as ora

TOL = dict(rtol=1e-5, atol=1e-5)


def np_pool(pool):
    return fx.to_numpy(pool.k), fx.to_numpy(pool.v)


# ----------------------------------------------------- reference fixtures

@pytest.mark.parametrize("case", [0, 1, 2])
def test_reference_unit_cases(case):
    pool, _, cases = fx.reference_case_2026()
    name, q, tables, lengths = cases[case]
    k, v = np_pool(pool)
    args = (q.numpy(), k, v, tables.numpy(), lengths.numpy(), 0)
    online = ora.paged_attention_online_v1(*args)
    ref = ora.paged_attention_reference(*args)
    dense = ora.dense_gold(*args)
    assert np.isfinite(online).all(), name
    np.testing.assert_allclose(online, ref, **TOL)
    np.testing.assert_allclose(online, dense, **TOL)


def test_nan_in_unwritten_slots_is_never_read():
    pool, q, tables, lengths = fx.padding_case_11()
    k, v = np_pool(pool)
    args = (q.numpy(), k, v, tables.numpy(), lengths.numpy(), 0)
    online = ora.paged_attention_online_v1(*args)
    assert np.isfinite(online).all()
    np.testing.assert_allclose(online, ora.paged_attention_reference(*args), **TOL)
    np.testing.assert_allclose(online, ora.dense_gold(*args), **TOL)


def test_probe_case():
    pool, q, tables, lengths = fx.probe_case_2026()
    k, v = np_pool(pool)
    args = (q.numpy(), k, v, tables.numpy(), lengths.numpy(), 0)
    online = ora.paged_attention_online_v1(*args)
    assert np.isfinite(online).all()
    np.testing.assert_allclose(online, ora.dense_gold(*args), **TOL)


@pytest.mark.parametrize("bs,context", [(8, 17), (16, 1), (16, 15), (16, 16), (16, 17), (16, 31),
                                        (16, 65), (16, 129)])
def test_dense_matches_online_for_ragged_blocks(bs, context):
    q, pool, tables, lens, layer = fx.build_case(3, context, 4, 8, bs, "mixed")
    k, v = np_pool(pool)
    args = (q.numpy(), k, v, tables.numpy(), lens.numpy(), layer)
    dense = ora.dense_gold(*args)
    np.testing.assert_allclose(dense, ora.paged_attention_online_v1(*args), **TOL)
    assert np.isfinite(dense).all()


@pytest.mark.parametrize("batch,length", [(1, 1), (1, 15), (1, 16), (2, 17), (4, 33), (4, 64), (4, 65),
                                          (2, 128), (4, 129), (2, 256), (4, 257)])
def test_online_matches_torch_softmax_on_the_fused_decode_grid(batch, length):
    """The correctness grid of experiments/gpu_day6_fused_decode_ab.py:171-181
    (8 heads, head_dim 32, block 16, seed 20261030 + B + L): the oracle's
    online recurrence against torch.softmax over each row's gathered tokens
    (float64), the library routine the reference's dense_gold uses."""
    q, pool, tables, lens, layer = fx.build_case(batch, length, 8, 32, 16, "mixed", seed=20261030 + batch + length)
    k, v = np_pool(pool)
    online = ora.paged_attention_online_v1(q.numpy(), k, v, tables.numpy(), lens.numpy(), layer)
    for b in range(batch):
        n = int(lens[b])
        blocks = tables[b, :-(-n // 16)]
        keys = pool.k[layer, blocks].reshape(-1, 8, 32)[:n].double()
        vals = pool.v[layer, blocks].reshape(-1, 8, 32)[:n].double()
        w = torch.softmax(torch.einsum("hd,thd->ht", q[b].double(), keys) / 32 ** 0.5, dim=-1)
        np.testing.assert_allclose(online[b], torch.einsum("ht,thd->hd", w, vals).numpy(), rtol=1e-9, atol=1e-9)


def test_build_case_has_nontrivial_mapping_nan_padding_and_strided_q():
    q, pool, tables, lens, layer = fx.build_case(4, 65, 8, 32, 16, "mixed")
    assert tables.shape[0] == 4 and bool((tables == -1).any())
    assert bool(torch.isnan(pool.k).any())
    assert q.stride(-1) != 1
    k, v = np_pool(pool)
    assert np.isfinite(ora.dense_gold(q.numpy(), k, v, tables.numpy(), lens.numpy(), layer)).all()


# ------------------------------------------------------------ closed forms

def _random_case(seed, B=3, H=4, D=16, S=4, N=40, ctx=(1, 9, 23)):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((1, N, S, H, D))
    v = rng.standard_normal((1, N, S, H, D))
    q = rng.standard_normal((B, H, D))
    M = max((c + S - 1) // S for c in ctx)
    perm = rng.permutation(N)
    tables = np.full((B, M), -1, np.int64)
    used = 0
    for b, c in enumerate(ctx):
        nb = (c + S - 1) // S
        tables[b, :nb] = perm[used: used + nb]
        used += nb
    return q, k, v, tables, np.array(ctx, np.int64)


def test_single_token_context_returns_its_value_row():
    q, k, v, tables, _ = _random_case(1)
    ctx = np.ones(3, np.int64)
    out = ora.paged_attention_online_v1(q, k, v, tables, ctx, 0)
    for b in range(3):
        np.testing.assert_array_equal(out[b], v[0, tables[b, 0], 0])


def test_identical_keys_average_the_values():
    q, k, v, tables, ctx = _random_case(2)
    for b in range(3):
        for j in range((ctx[b] + 3) // 4):
            k[0, tables[b, j]] = k[0, tables[b, 0], 0]
    out = ora.paged_attention_online_v1(q, k, v, tables, ctx, 0)
    for b in range(3):
        _, vals = ora.gather_tokens(k, v, tables, int(ctx[b]), b, 0)
        np.testing.assert_allclose(out[b], vals.mean(axis=0), rtol=1e-12, atol=1e-12)


def test_dense_gold_matches_textbook_softmax():
    q, k, v, tables, ctx = _random_case(3)
    out = ora.dense_gold(q, k, v, tables, ctx, 0)
    for b in range(3):
        keys, vals = ora.gather_tokens(k, v, tables, int(ctx[b]), b, 0)
        for h in range(4):
            s = keys[:, h] @ q[b, h] / math.sqrt(16)
            w = torch.softmax(torch.from_numpy(s), dim=0).numpy()
            np.testing.assert_allclose(out[b, h], w @ vals[:, h], rtol=1e-12, atol=1e-12)


def test_block_placement_does_not_change_the_result():
    q, k, v, tables, ctx = _random_case(4)
    perm = np.random.default_rng(5).permutation(k.shape[1])
    inv = np.argsort(perm)
    k2, v2 = k[:, perm], v[:, perm]            # block i moves to position inv[i]
    tables2 = np.where(tables >= 0, inv[np.maximum(tables, 0)], -1)
    a = ora.paged_attention_online_v1(q, k, v, tables, ctx, 0)
    b = ora.paged_attention_online_v1(q, k2, v2, tables2, ctx, 0)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("P", [1, 4, 7, 16, 64])
def test_partition_merge_equals_unsplit(P):
    q, k, v, tables, ctx = _random_case(6, ctx=(5, 33, 60))
    dense = ora.dense_gold(q, k, v, tables, ctx, 0)
    for b, (ms, ls, Os) in enumerate(ora.partition_partials(q, k, v, tables, ctx, 0, P)):
        np.testing.assert_allclose(ora.merge_partials(ms, ls, Os), dense[b], rtol=1e-12, atol=1e-12)


# ----------------------------------------------------- planted mistakes

def _mutant_online(q, k, v, tables, ctx, layer, bug):
    """online_v1 restated with one planted mistake; must fail the pinning checks."""
    q = ora.as_float(q)
    B, H, D = q.shape
    S = k.shape[2]
    sc = 1.0 / D if bug == "scale" else 1.0 / math.sqrt(D)
    out = np.zeros((B, H, D))
    for b in range(B):
        m, l, O = np.full(H, -np.inf), np.zeros(H), np.zeros((H, D))
        c = int(ctx[b]) - (1 if bug == "off_by_one" else 0)
        for j in range((c + S - 1) // S):
            n = min(S, c - j * S)
            keys = k[layer, tables[b, j], :n]
            if bug == "head":
                keys = np.roll(keys, 1, axis=1)
            s = np.einsum("hd,thd->ht", q[b], keys) * sc
            mn = np.maximum(m, s.max(-1))
            alpha = np.ones(H) if bug == "no_rescale" else np.exp(m - mn)
            p = np.exp(s - mn[:, None])
            ln = alpha * l + p.sum(-1)
            O = (alpha[:, None] * l[:, None] * O + np.einsum("ht,thd->hd", p, v[layer, tables[b, j], :n])) / ln[:, None]
            m, l = mn, ln
        out[b] = O
    return out


@pytest.mark.parametrize("bug", ["scale", "head", "no_rescale", "off_by_one"])
def test_planted_mistakes_are_rejected(bug):
    q, pool, tables, lens, layer = fx.build_case(3, 65, 4, 8, 16, "mixed", scale=1.0)
    k, v = np_pool(pool)
    args = (q.numpy(), k, v, tables.numpy(), lens.numpy(), layer)
    dense = ora.dense_gold(*args)
    with np.errstate(all="ignore"):
        bad = _mutant_online(*args, bug)
    assert not np.allclose(bad, dense, **TOL), bug
    # the faithful restatement passes the same check
    np.testing.assert_allclose(ora.paged_attention_online_v1(*args), dense, **TOL)


# ------------------------------------------------------------- C oracle

def test_c_oracle_matches_numpy_f32_and_bf16():
    q, pool, tables, lens, layer = fx.build_case(4, 129, 8, 32, 16, "mixed")
    k, v = np_pool(pool)
    qn = np.ascontiguousarray(q.numpy())
    args = (qn, k, v, tables.numpy(), lens.numpy(), layer)
    want = ora.paged_attention_online_v1(*args)
    np.testing.assert_allclose(c_oracle.paged_decode(*args, acc_double=True, threads=2), want,
                               rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(c_oracle.paged_decode(*args, acc_double=False), want, **TOL)
    # bfloat16 bit patterns, NaN tails included
    kb, vb = ora.f32_to_bf16_bits(k), ora.f32_to_bf16_bits(v)
    qb = ora.f32_to_bf16_bits(qn)
    argsb = (qb, kb, vb, tables.numpy(), lens.numpy(), layer)
    np.testing.assert_allclose(c_oracle.paged_decode(*argsb, threads=3),
                               ora.dense_gold(*argsb), rtol=1e-6, atol=1e-6)


# ------------------------------------------------------------ KV append

def test_kv_append_matches_index_put_bitwise():
    g = torch.Generator().manual_seed(7)
    L, N, S, H, D, T = 2, 12, 4, 3, 8, 9
    pool_k = torch.randn(L, N, S, H, D, generator=g)
    pool_v = torch.randn(L, N, S, H, D, generator=g)
    pool_k.view(torch.int32)[0, 3] = 0x7FC00001            # NaN payloads stay untouched
    k_new = torch.randn(T, H, D, generator=g)
    v_new = torch.randn(T, H, D, generator=g)
    k_new.view(torch.int32)[2, 1, 3] = 0x7FA5A5A5           # a NaN payload row is copied bit for bit
    slots = torch.randperm(N * S, generator=g)[:T]
    slots[[1, 5]] = -1
    layer = 1
    want_k, want_v = pool_k.clone(), pool_v.clone()
    keep = slots >= 0
    blk, off = slots[keep] // S, slots[keep] % S
    want_k[layer, blk, off] = k_new[keep]
    want_v[layer, blk, off] = v_new[keep]
    got_k, got_v = ora.kv_append(pool_k.numpy(), pool_v.numpy(), layer, k_new.numpy(), v_new.numpy(),
                                 slots.numpy())
    np.testing.assert_array_equal(got_k.view(np.uint32), want_k.numpy().view(np.uint32))
    np.testing.assert_array_equal(got_v.view(np.uint32), want_v.numpy().view(np.uint32))


def test_kv_append_skips_out_of_range_slots():
    k = np.zeros((1, 2, 2, 1, 2), np.float32)
    rows = np.ones((3, 1, 2), np.float32)
    got, _ = ora.kv_append(k, k, 0, rows, rows, np.array([-1, 4, 99]))
    assert not got.any()


def test_bf16_rounding_matches_torch_cast():
    g = torch.Generator().manual_seed(3)
    x = torch.cat([torch.randn(4096, generator=g) * 10,
                   torch.tensor([0.0, -0.0, 1e-40, -1e-40, 3.4e38, float("inf"), -float("inf"),
                                 1.00390625, 1.01171875, 65504.0])])
    got = ora.f32_to_bf16_bits(x.numpy())
    want = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(got, want)
    back = ora.bf16_bits_to_f32(got)
    np.testing.assert_array_equal(back, x.to(torch.bfloat16).float().numpy())
    assert ora.f32_to_bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0
