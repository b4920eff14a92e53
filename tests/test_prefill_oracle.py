"""Pinning of the prefill oracle (oracle.paged_decode.paged_prefill) on the CPU.

The oracle computes a chunk's causal attention as one dense softmax over the
gathered tokens. It is checked against:
  * the per-block online recurrence of the decode oracle, run once per query
    row with context_length = start + i + 1 -- the reference's own per-token
    prefill loop (minivllm/attention.py:269-299), whose decode oracle is
    pinned by the reference's golden cases;
  * torch's scaled_dot_product_attention on the CPU (a library routine), with
    is_causal for start 0 and an absolute-position mask otherwise;
  * the decode closed form for a one-row chunk, block-placement invariance,
    and NaN in never-visible slots;
  * planted mistakes (an off-by-one mask, a chunk-relative mask, a read past
    the chunk), each of which must be rejected.
Chunk patterns are the reference's prefix test cases
(tests/test_prefill_prefix_sdpa_v2.py:52-64): block size 4, head_dim 8, and a
non-monotonic physical allocation.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import paged_decode as ora

PIECES = ([5, 7, 19], [1, 1, 9], [16, 1, 15], [8, 8, 8, 8], [3, 5, 4, 16, 11],
          [16, 16, 16, 16], [64, 32, 32])


def _interleaved_table(n_blocks, n_used):
    """The reference test's allocation: even blocks first, then odd ones."""
    perm = list(range(n_blocks))[::2] + list(range(n_blocks))[1::2]
    return np.asarray(perm[:n_used], dtype=np.int64)


def _case(total, S=4, H=4, D=8, N=64, L=2, layer=1, seed=0):
    rng = np.random.default_rng(seed)
    k = np.full((L, N, S, H, D), np.nan)
    v = np.full((L, N, S, H, D), np.nan)
    n_used = -(-total // S)
    table = _interleaved_table(N, n_used)
    for j in range(total):
        k[layer, table[j // S], j % S] = rng.standard_normal((H, D))
        v[layer, table[j // S], j % S] = rng.standard_normal((H, D))
    return k, v, table, layer, rng


def _per_row_reference(q, k, v, table, start, layer):
    T = q.shape[0]
    tables = np.repeat(table[None, :], T, axis=0)
    ctx = start + np.arange(T) + 1
    return ora.paged_attention_reference(q, k, v, tables, ctx, layer)


@pytest.mark.parametrize("pieces", PIECES, ids=lambda p: "-".join(map(str, p)))
def test_chunks_match_the_per_token_online_loop(pieces):
    k, v, table, layer, rng = _case(sum(pieces))
    start = 0
    for T in pieces:
        q = rng.standard_normal((T, 4, 8))
        got = ora.paged_prefill(q, k, v, table, start, layer)
        want = _per_row_reference(q, k, v, table, start, layer)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
        assert np.isfinite(got).all()
        start += T


@pytest.mark.parametrize("start,T", [(0, 1), (0, 37), (13, 1), (13, 29), (40, 24)])
def test_matches_torch_sdpa_with_absolute_positions(start, T):
    k, v, table, layer, rng = _case(start + T, S=4, H=3, D=16)
    q = rng.standard_normal((T, 3, 16))
    got = ora.paged_prefill(q, k, v, table, start, layer)
    keys, vals = ora.gather_tokens(k, v, table[None, :], start + T, 0, layer)
    qt = torch.from_numpy(q).permute(1, 0, 2)[None]
    kt = torch.from_numpy(keys).permute(1, 0, 2)[None]
    vt = torch.from_numpy(vals).permute(1, 0, 2)[None]
    if start == 0:
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True)
    else:
        mask = torch.arange(start + T)[None, :] <= (start + torch.arange(T))[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
    np.testing.assert_allclose(got, ref[0].permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-12)


def test_one_row_chunk_is_a_decode_step():
    k, v, table, layer, rng = _case(23, S=4)
    q = rng.standard_normal((1, 4, 8))
    got = ora.paged_prefill(q, k, v, table, 22, layer)
    want = ora.dense_gold(q, k, v, table[None, :], np.array([23]), layer)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_first_row_of_a_fresh_sequence_returns_its_value():
    k, v, table, layer, rng = _case(9, S=4)
    q = rng.standard_normal((9, 4, 8)) * 5
    got = ora.paged_prefill(q, k, v, table, 0, layer)
    np.testing.assert_array_equal(got[0], v[layer, table[0], 0])


def test_block_placement_does_not_change_the_result():
    k, v, table, layer, rng = _case(30, S=4)
    q = rng.standard_normal((10, 4, 8))
    base = ora.paged_prefill(q, k, v, table, 20, layer)
    perm = np.random.default_rng(5).permutation(k.shape[1])
    k2, v2 = np.empty_like(k), np.empty_like(v)
    k2[:, perm], v2[:, perm] = k, v
    np.testing.assert_allclose(ora.paged_prefill(q, k2, v2, perm[table], 20, layer), base,
                               rtol=1e-12, atol=1e-12)


def _mutant(q, k, v, table, start, layer, bug):
    """paged_prefill with one planted mistake."""
    T, H, D = q.shape
    ctx = start + T + (1 if bug == "reads_past_chunk" else 0)
    keys, vals = ora.gather_tokens(k, v, table[None, :], ctx, 0, layer)
    scores = np.einsum("ihd,jhd->hij", q, keys) / math.sqrt(D)
    pos = (0 if bug == "chunk_relative_mask" else start) + np.arange(T)
    j = np.arange(ctx)[None, :]
    visible = j < pos[:, None] if bug == "strict_mask" else j <= pos[:, None]
    if bug == "reads_past_chunk":
        visible = j <= pos[:, None] + 1
    with np.errstate(invalid="ignore"):
        scores = np.where(visible[None], scores, -np.inf)
        scores -= scores.max(axis=-1, keepdims=True)
        w = np.exp(scores)
        w /= w.sum(axis=-1, keepdims=True)
        return np.einsum("hij,jhd->ihd", w, vals)


@pytest.mark.parametrize("bug", ["strict_mask", "chunk_relative_mask", "reads_past_chunk"])
def test_planted_mistakes_are_rejected(bug):
    k, v, table, layer, rng = _case(40, S=4)
    # Slot 40 (one past the chunk) holds data, so a read past the chunk shows.
    k[layer, _interleaved_table(64, 11)[10], 0] = rng.standard_normal((4, 8))
    v[layer, _interleaved_table(64, 11)[10], 0] = rng.standard_normal((4, 8))
    table = _interleaved_table(64, 11)
    q = rng.standard_normal((12, 4, 8))
    want = _per_row_reference(q, k, v, table, 28, layer)
    np.testing.assert_allclose(ora.paged_prefill(q, k, v, table, 28, layer), want, rtol=1e-12)
    bad = _mutant(q, k, v, table, 28, layer, bug)
    assert not np.allclose(np.nan_to_num(bad, nan=1e9), want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("bad", [[3], [0], [1, 4]], ids=["middle", "first", "two"])
def test_invalid_table_entries_mask_their_tokens(bad):
    """Entries outside [0, N) mask their block's tokens; a row that sees none is
    zero. Pinned by the C decode oracle (an independent restatement that skips
    such blocks) run once per query row at context start + i + 1."""
    k, v, table, layer, rng = _case(30, S=4)
    table = table.copy()
    for j in bad:
        table[j] = -1 if j % 2 == 0 else k.shape[1] + 3
    q = rng.standard_normal((14, 4, 8)).astype(np.float32)
    got = ora.paged_prefill(q, k, v, table, 16, layer)
    T = q.shape[0]
    want = c_oracle.paged_decode(q, k.astype(np.float32), v.astype(np.float32),
                                 np.repeat(table[None, :], T, axis=0), 16 + np.arange(T) + 1, layer)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    if 0 in bad:
        start0 = ora.paged_prefill(q, k, v, table, 0, layer)
        assert np.all(start0[:4] == 0.0)          # rows 0..3 see only the masked block 0
