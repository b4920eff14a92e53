"""The lock-step harness itself, on the CPU (tests/_e2e.Lockstep).

The HIP entry points are patched with the PyTorch path (index_put_ KV write
and online_v1), so the two runtimes compute the same bits, and a difference
is planted in the "hip" runtime's greedy tokens or attention output:
  * a token changed at an allowed tie is replaced by the reference's, the
    event is recorded, and every later decode row and every live sequence's
    KV stays in the checks (both runtimes end with the same streams);
  * the same change where ties are not allowed fails the step;
  * an attention output moved past the logit bound fails the step.
online_v1_fp32 (the fp32-accumulating reference of the bf16 lock step) is
checked against online_v1 on a float32 copy of the pool.
"""
from __future__ import annotations

import math
from unittest.mock import patch

import pytest
import torch

import _e2e
from minivllm import hip_paged_decode
from minivllm.attention import write_kv_rows
from minivllm.kv_block_pool import KVBlockPool
from minivllm.paged_attention_batch import paged_attention_batch_online_v1

SPEC = _e2e.RuntimeSpec(n_requests=6, prompt_mean=24, prompt_cap=64, output_len=6, n_embd=64, n_head=2,
                        n_layer=2, vocab=128, max_running=6, token_budget=64, seed=1)


def _cpu_kv_append(pool, layer_idx, k, v, slot_mapping):
    write_kv_rows(pool, layer_idx, k, v, slot_mapping, use_hip=False)


def _cpu_attention(q, pool, block_tables, context_lengths, layer_idx, *, split_tokens=0):
    return paged_attention_batch_online_v1(q=q, pool=pool, block_tables=block_tables,
                                           context_lengths=context_lengths, layer_idx=layer_idx)


def _fused(attention):
    """A CPU stand-in for the fused append + attention call built from the two
    stand-ins, in the two calls' order."""
    def call(q, pool, block_tables, context_lengths, layer_idx, k, v, slot_mapping, *, split_tokens=0):
        _cpu_kv_append(pool, layer_idx, k, v, slot_mapping)
        return attention(q, pool, block_tables, context_lengths, layer_idx)
    return call


def _lockstep(**criterion) -> _e2e.Lockstep:
    model = _e2e.make_model(SPEC, torch.device("cpu"), torch.float32)
    return _e2e.Lockstep(SPEC, model, _e2e.make_prompts(SPEC), torch.device("cpu"), torch.float32,
                         **criterion)


def _plant_token(ls: _e2e.Lockstep, at_call: int) -> dict:
    """Changes row 0's greedy token in the hip runtime's decode call number
    ``at_call`` (1-based); returns a record of what was planted."""
    inner = ls.hip.rt.runner.decode_batch
    planted = {"calls": 0}

    def decode_batch(sequences):
        logits, tokens = inner(sequences)
        planted["calls"] += 1
        if planted["calls"] == at_call:
            tokens = list(tokens)
            tokens[0] = (tokens[0] + 1) % SPEC.vocab
            planted["seq_id"] = sequences[0].seq_id
        return logits, tokens

    ls.hip.rt.runner.decode_batch = decode_batch
    return planted


def _run(ls: _e2e.Lockstep) -> None:
    with torch.inference_mode():
        while not ls.finished:
            ls.step()
            assert ls.stats["steps"] < 500


@patch.object(hip_paged_decode, "paged_attention_batch_hip", _cpu_attention)
@patch.object(hip_paged_decode, "kv_append", _cpu_kv_append)
@patch.object(hip_paged_decode, "paged_attention_batch_append_hip", _fused(_cpu_attention))
def test_forced_tie_keeps_every_row_in_the_checks():
    ls = _lockstep(logit_tol=(2e-5, 2e-4), tie_margin=1e9, kv_tol=(2e-5, 2e-4))
    planted = _plant_token(ls, at_call=3)
    _run(ls)
    ls.finish_checks()
    assert [sid for _, sid, _, _ in ls.forced] == [planted["seq_id"]]
    assert ls.stats["decode_rows_checked"] == ls.stats["decode_rows"] > 0
    # Same arithmetic in both runtimes once the token is forced back.
    assert ls.stats["max_logit_abs"] == 0.0 and ls.stats["max_kv_abs"] == 0.0
    for x in ls.ref.seqs:
        y = ls.hip.by_id[x.seq_id]
        assert x.generated_tokens == y.generated_tokens and x.last_token == y.last_token


@patch.object(hip_paged_decode, "paged_attention_batch_hip", _cpu_attention)
@patch.object(hip_paged_decode, "kv_append", _cpu_kv_append)
@patch.object(hip_paged_decode, "paged_attention_batch_append_hip", _fused(_cpu_attention))
def test_token_difference_outside_a_tie_fails():
    ls = _lockstep(logit_tol=(2e-5, 2e-4), tie_margin=0.0, kv_tol=(2e-5, 2e-4))
    _plant_token(ls, at_call=2)
    with pytest.raises(AssertionError, match="differs at reference top-2 margin"):
        _run(ls)


def _shifted_attention(q, pool, block_tables, context_lengths, layer_idx, *, split_tokens=0):
    out = _cpu_attention(q, pool, block_tables, context_lengths, layer_idx)
    return out + 0.05 * out.abs().amax()


@patch.object(hip_paged_decode, "paged_attention_batch_hip", _shifted_attention)
@patch.object(hip_paged_decode, "kv_append", _cpu_kv_append)
@patch.object(hip_paged_decode, "paged_attention_batch_append_hip", _fused(_shifted_attention))
def test_attention_error_past_the_bound_fails():
    ls = _lockstep(logit_tol=(2e-5, 2e-4), tie_margin=1e9, kv_tol=(2e-5, 2e-4))
    with pytest.raises(AssertionError, match="decode logits differ"):
        _run(ls)


def test_online_v1_fp32_is_online_v1_on_a_float32_copy():
    g = torch.Generator().manual_seed(5)
    L, N, S, H, D, B = 2, 24, 4, 3, 16, 3
    pool = KVBlockPool(L, N, S, H, D, device="cpu", dtype=torch.bfloat16)
    pool.k.copy_(torch.randn(pool.k.shape, generator=g))
    pool.v.copy_(torch.randn(pool.v.shape, generator=g))
    ctx = torch.tensor([1, 9, 17])
    tables = torch.full((B, 5), -1, dtype=torch.long)
    perm = torch.randperm(N, generator=g)
    used = 0
    for b in range(B):
        nb = -(-int(ctx[b]) // S)
        tables[b, :nb] = perm[used:used + nb]
        used += nb
    q = torch.randn((B, H, D), generator=g).to(torch.bfloat16)
    got = _e2e.online_v1_fp32(q, pool, tables, ctx, 1)
    assert got.dtype == torch.bfloat16
    f32 = KVBlockPool(L, N, S, H, D, device="cpu", dtype=torch.float32)
    f32.k.copy_(pool.k.float())
    f32.v.copy_(pool.v.float())
    want = paged_attention_batch_online_v1(q=q.float(), pool=f32, block_tables=tables, context_lengths=ctx,
                                           layer_idx=1)
    assert torch.equal(got, want.to(torch.bfloat16))
    # Closed form: dense softmax attention over each sequence's gathered tokens.
    for b in range(B):
        n = int(ctx[b])
        blocks = tables[b, :-(-n // S)]
        keys = f32.k[1, blocks].reshape(-1, H, D)[:n]
        vals = f32.v[1, blocks].reshape(-1, H, D)[:n]
        w = torch.softmax(torch.einsum("hd,thd->ht", q[b].float(), keys) / math.sqrt(D), dim=-1)
        dense = torch.einsum("ht,thd->hd", w, vals)
        torch.testing.assert_close(got[b].float(), dense, atol=2e-2, rtol=2e-2)
