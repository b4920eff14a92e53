"""Backend routing on the GPU, restating
tests/test_decode_backend_integration.py:31-65 of the reference for the HIP
backend: with the append and attention as two calls (fused_decode_append
off), the attention entry point is patched (at
minivllm.hip_paged_decode.paged_attention_batch_hip, where the model imports
it at call time) with a stand-in that checks the new token's K/V are already
in the pool -- written by the real kv_append kernel -- and then runs the
PyTorch online-softmax attention. Logits and the written KV must then be
bit-identical to the reference backend's (atol = rtol = 0): the append is a
bitwise copy to the same slots, the reference writes with index_put_. The
default route, the fused call, must match the two calls bit for bit.
"""
from __future__ import annotations

from unittest.mock import patch

import pytest
import torch

from minivllm.decode_batch_metadata import DecodeBatchMetadata
from minivllm.kv_block_pool import KVBlockPool
from minivllm.model import MiniGPT
from minivllm.paged_attention_batch import paged_attention_batch_online_v1

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("backend", ["hip", "triton_v0"])
def test_route_appends_kv_before_attention_and_logits_identical(backend, dtype):
    print(f"  routing backend={backend} dtype={dtype}", flush=True)
    torch.manual_seed(10)
    model = MiniGPT(n_embd=16, n_head=4, vocab_size=32, block_size=32, dropout=0.0, n_layer=2)
    model = model.eval().to(device=DEV, dtype=dtype)
    for block in model.blocks:
        block.attn.fused_decode_append = False
    inputs = torch.tensor([[1], [2]], dtype=torch.long, device=DEV)
    meta = DecodeBatchMetadata(positions=torch.tensor([0, 0], device=DEV),
                               context_lengths=torch.tensor([1, 1], device=DEV),
                               block_tables=torch.tensor([[1], [0]], dtype=torch.long, device=DEV),
                               slot_mapping=torch.tensor([16, 0], dtype=torch.long, device=DEV))

    def make_pool():
        pool = KVBlockPool(n_layer=2, num_blocks=2, block_size=16, n_head=4, head_dim=4, device=DEV,
                           dtype=dtype)
        pool.k.fill_(float("nan"))
        pool.v.fill_(float("nan"))
        return pool

    pool0, pool1 = make_pool(), make_pool()
    calls = []

    def stand_in(q, pool, block_tables, context_lengths, layer_idx):
        calls.append(layer_idx)
        # Row 0 wrote slot 16 (block 1, offset 0), row 1 slot 0 (block 0).
        assert torch.isfinite(pool.k[layer_idx, 1, 0].float()).all()
        assert torch.isfinite(pool.v[layer_idx, 0, 0].float()).all()
        return paged_attention_batch_online_v1(q, pool, block_tables, context_lengths, layer_idx)

    with torch.inference_mode():
        model.set_decode_attention_backend("reference")
        expected = model.decode_batch(inputs, meta, pool0)
        model.set_decode_attention_backend(backend)
        with patch("minivllm.hip_paged_decode.paged_attention_batch_hip", side_effect=stand_in):
            actual = model.decode_batch(inputs, meta, pool1)
    torch.cuda.synchronize()
    assert calls == [0, 1]
    torch.testing.assert_close(expected, actual, atol=0, rtol=0)
    torch.testing.assert_close(pool0.k[:, 1, 0], pool1.k[:, 1, 0], atol=0, rtol=0)
    torch.testing.assert_close(pool0.v[:, 0, 0], pool1.v[:, 0, 0], atol=0, rtol=0)
    # Nothing else was written: every other slot still holds NaN.
    for pool in (pool1,):
        written = torch.zeros(pool.k.shape[1:3], dtype=torch.bool, device=DEV)
        written[1, 0] = written[0, 0] = True
        assert torch.isnan(pool.k.float()[:, ~written]).all()


def test_unpatched_hip_route_matches_reference_within_tolerance():
    """The same step through the real HIP attention kernel: the KV bit-identical,
    the logits within the fp32 attention tolerance of the reference tests."""
    torch.manual_seed(10)
    model = MiniGPT(n_embd=16, n_head=4, vocab_size=32, block_size=32, dropout=0.0, n_layer=2).eval().to(DEV)
    inputs = torch.tensor([[1], [2]], dtype=torch.long, device=DEV)
    meta = DecodeBatchMetadata(positions=torch.tensor([0, 0], device=DEV),
                               context_lengths=torch.tensor([1, 1], device=DEV),
                               block_tables=torch.tensor([[1], [0]], dtype=torch.long, device=DEV),
                               slot_mapping=torch.tensor([16, 0], dtype=torch.long, device=DEV))
    pools = []
    for backend in ("reference", "hip"):
        pool = KVBlockPool(n_layer=2, num_blocks=2, block_size=16, n_head=4, head_dim=4, device=DEV)
        pool.k.fill_(float("nan"))
        pool.v.fill_(float("nan"))
        model.set_decode_attention_backend(backend)
        with torch.inference_mode():
            pools.append((pool, model.decode_batch(inputs, meta, pool)))
    (p0, ref), (p1, got) = pools
    torch.testing.assert_close(got, ref, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(p0.k[:, 1, 0], p1.k[:, 1, 0], atol=0, rtol=0)
    torch.testing.assert_close(p0.v[:, 0, 0], p1.v[:, 0, 0], atol=0, rtol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_route_matches_two_calls_bit_for_bit(dtype):
    """The default HIP route (the append inside the attention launch) against
    the two calls, on a head dim the fused write takes (128): three decode
    steps of 6 sequences over cached contexts, one of them padding; logits and
    every pool byte identical at every step."""
    torch.manual_seed(3)
    model = MiniGPT(n_embd=256, n_head=2, vocab_size=64, block_size=512, dropout=0.0, n_layer=2)
    model = model.eval().to(device=DEV, dtype=dtype)
    model.set_decode_attention_backend("hip")
    B, S, N, M = 6, 16, 128, 20
    g = torch.Generator().manual_seed(4)
    ctx0 = torch.randint(20, 300, (B,), generator=g)
    perm = torch.randperm(N, generator=g)
    tables = perm[:B * M].view(B, M).clone()
    pools = []
    for fused in (False, True):
        pool = KVBlockPool(n_layer=2, num_blocks=N, block_size=S, n_head=2, head_dim=128, device=DEV, dtype=dtype)
        gd = torch.Generator(device=DEV).manual_seed(5)
        pool.k.normal_(generator=gd)
        pool.v.normal_(generator=gd)
        pools.append(pool)
    for step in range(3):
        pos = ctx0 + step
        slots = tables[torch.arange(B), pos // S] * S + pos % S
        slots[2] = -1   # a padding row: no write, attention over its cached context
        ctx = torch.where(slots >= 0, pos + 1, pos)
        meta = DecodeBatchMetadata(positions=pos.to(DEV), context_lengths=ctx.to(DEV),
                                   block_tables=tables.to(DEV), slot_mapping=slots.to(DEV))
        inputs = torch.randint(0, 64, (B, 1), generator=g).to(DEV)
        outs = []
        for fused, pool in zip((False, True), pools):
            for block in model.blocks:
                block.attn.fused_decode_append = fused
            with torch.inference_mode():
                outs.append(model.decode_batch(inputs, meta, pool))
        torch.cuda.synchronize()
        print(f"  fused route step {step} {dtype}", flush=True)
        assert torch.equal(outs[0], outs[1])
        assert torch.equal(pools[0].k, pools[1].k) and torch.equal(pools[0].v, pools[1].v)
