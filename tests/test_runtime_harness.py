"""The host harness around the decode path (CPU): block manager, scheduler,
runtime loop and model-level backend routing.

Pinned by the reference's own known answers:
  * tests/test_block_manager.py:8-52 (slot identities, LIFO reuse);
  * scripts/release_smoke.py:84-94 -- (iterations, preemptions, repeated KV
    tokens) = conservative (27, 0, 0) / recompute (27, 3, 44) for the
    "baseline" workload on 2 blocks, and (34, 0, 0) / (32, 0, 0) for
    "mixed_short" on 3 blocks, with identical tokens under both policies
    (experiments/bench_preemption.py:39-110, 218-220);
  * tests/test_auto_preemption.py:151-194 (40 seeded random cases with
    check_invariants every step; recompute == conservative tokens);
  * tests/test_decode_backend_integration.py:19-76 (routing, KV written
    before attention, bit-identical logits, no silent CPU fallback).
"""
from __future__ import annotations

import random
from unittest.mock import patch

import pytest
import torch

from minivllm.block_manager import BlockManager
from minivllm.decode_batch_metadata import DecodeBatchMetadata
from minivllm.kv_block_pool import KVBlockPool
from minivllm.mini_runtime import MiniRuntime
from minivllm.model import MiniGPT
from minivllm.model_runner import ModelRunner
from minivllm.paged_attention_batch import paged_attention_batch_online_v1
from minivllm.scheduler import Scheduler
from minivllm.sequence import SequenceState, Status


def request(name, prompt, n_out):
    return SequenceState(seq_id=name, prompt_tokens=list(prompt), max_tokens=len(prompt) + n_out)


# ---------------------------------------------------------- block manager

def test_block_manager_cross_block_multi_request_and_reuse():
    manager = BlockManager(num_blocks=5, block_size=4)
    a, b, c, d = (SequenceState(seq_id=n, prompt_tokens=[i] * L, max_tokens=12)
                  for n, i, L in (("A", 1, 7), ("B", 2, 4), ("C", 3, 8), ("D", 4, 9)))
    seqs = [a, b, c, d]
    assert manager.num_new_blocks_needed(a, 3) == 1
    slots = manager.reserve_slots(a, 3)
    a.length += 3
    manager.check_invariants(seqs)
    assert manager.num_new_blocks_needed(a, 1) == 0
    slots += manager.reserve_slots(a, 1)
    a.length += 1
    assert len(a.block_table) == 1
    assert manager.num_new_blocks_needed(a, 3) == 1
    slots += manager.reserve_slots(a, 3)
    a.length += 3
    assert len(a.block_table) == 2
    assert [manager.logical_to_slot(a, p) for p in range(len(slots))] == slots
    manager.check_invariants(seqs)
    manager.reserve_slots(b, 4)
    b.length += 4
    assert set(a.block_table).isdisjoint(b.block_table)
    released = set(manager.free(a))
    assert len(released) == 2
    manager.check_invariants(seqs)
    manager.reserve_slots(c, 8)
    c.length += 8
    assert set(c.block_table) == released
    assert manager.num_new_blocks_needed(d, 9) == 3
    assert not manager.can_reserve(d, 9)


def test_initial_order_then_lifo_reuse():
    m = BlockManager(num_blocks=4, block_size=2)
    s = request("x", [1], 1)
    assert m.reserve_slots(s, 6) == [0, 1, 2, 3, 4, 5]   # blocks 0, 1, 2 in order
    s.length = 6
    m.free(s)                                             # pushes 0, 1, 2 back
    t = request("y", [1], 1)
    assert m.reserve_append_slot(t)[0] == 2               # last released, first reused


# ----------------------------------------------- preemption known counts

class CountingRunner:
    """Counts repeated KV positions independently of the runtime's records."""

    def __init__(self, inner):
        self.inner, self.high, self.repeated = inner, {}, 0
        self.prefill_tokens = self.decode_tokens = 0

    def _track(self, seq, start, end):
        prev = self.high.get(seq.seq_id, 0)
        self.repeated += max(0, min(end, prev) - start)
        self.high[seq.seq_id] = max(prev, end)

    def prefill_chunk(self, seq, start_pos, num_tokens):
        out = self.inner.prefill_chunk(seq, start_pos, num_tokens)
        self._track(seq, start_pos, start_pos + num_tokens)
        self.prefill_tokens += num_tokens
        return out

    def decode_batch(self, sequences):
        starts = [(s, s.length) for s in sequences]
        out = self.inner.decode_batch(sequences)
        for s, st in starts:
            self._track(s, st, st + 1)
        self.decode_tokens += len(sequences)
        return out


WORKLOADS = {
    "baseline": [("A", 16, 8), ("B", 16, 8), ("C", 12, 6), ("D", 16, 5)],
    "mixed_short": [("A", 4, 32), ("B", 4, 2), ("C", 4, 2), ("D", 4, 2)],
}


def run_workload(model, profile, policy, num_blocks):
    manager = BlockManager(num_blocks=num_blocks, block_size=16)
    rt = MiniRuntime.__new__(MiniRuntime)
    rt.block_manager = manager
    rt.scheduler = Scheduler(manager, max_running=4, max_num_batched_tokens=64, preemption_policy=policy)
    pool = KVBlockPool(n_layer=1, num_blocks=num_blocks, block_size=16, n_head=2, head_dim=8)
    rt.runner = CountingRunner(ModelRunner(model, pool, manager))
    rt.iteration, rt.records = 0, []
    seqs = [SequenceState(seq_id=n, prompt_tokens=[((i + j) % 31) + 1 for j in range(p)],
                          max_tokens=p + o) for i, (n, p, o) in enumerate(WORKLOADS[profile])]
    for s in seqs:
        rt.add_request(s)
    with torch.inference_mode():
        for _ in range(200):
            if all(s.status == Status.FINISHED for s in seqs):
                break
            rt.step()
            manager.check_invariants(seqs)
    assert all(s.status == Status.FINISHED for s in seqs)
    assert not manager.block_owner and len(manager.free_blocks) == num_blocks
    summary = rt.metrics_summary()
    assert summary["preemptions"] == rt.scheduler.num_preemptions
    assert summary["repeated_kv_tokens"] == rt.runner.repeated
    assert summary["prefill_tokens"] == rt.runner.prefill_tokens
    assert summary["decode_tokens"] == rt.runner.decode_tokens
    assert sum(len(s.generated_tokens) for s in seqs) == sum(s.max_tokens - s.prompt_length for s in seqs)
    return (rt.iteration, rt.scheduler.num_preemptions, rt.runner.repeated), {s.seq_id: s.generated_tokens
                                                                              for s in seqs}


@pytest.fixture(scope="module")
def preemption_model():
    torch.set_num_threads(1)
    torch.manual_seed(2026)
    return MiniGPT(n_embd=16, n_head=2, vocab_size=64, block_size=256, dropout=0.0, n_layer=1).eval()


@pytest.mark.parametrize("profile,blocks,expected", [
    ("baseline", 2, {"conservative": (27, 0, 0), "recompute": (27, 3, 44)}),
    ("mixed_short", 3, {"conservative": (34, 0, 0), "recompute": (32, 0, 0)}),
])
def test_release_smoke_known_counts(preemption_model, profile, blocks, expected):
    counts, tokens = {}, {}
    for policy in ("conservative", "recompute"):
        counts[policy], tokens[policy] = run_workload(preemption_model, profile, policy, blocks)
    assert counts == expected
    assert tokens["conservative"] == tokens["recompute"]


# --------------------------------------------------- scheduler stress

class FakeRunner:
    def __init__(self, manager):
        self.manager = manager

    def prefill_chunk(self, seq, start_pos, num_tokens):
        assert seq.length == seq.prompt_pos == start_pos
        self.manager.reserve_slots(seq, num_tokens)
        seq.length += num_tokens
        return torch.zeros((1, num_tokens, 16))

    def decode_batch(self, sequences):
        for seq in sequences:
            self.manager.reserve_append_slot(seq)
            seq.length += 1
        return torch.zeros((len(sequences), 16)), [0] * len(sequences)


def cpu_runtime(policy, num_blocks=2, block_size=4, max_running=2, token_budget=8, model=None):
    rt = MiniRuntime.__new__(MiniRuntime)
    manager = BlockManager(num_blocks=num_blocks, block_size=block_size)
    rt.block_manager = manager
    rt.scheduler = Scheduler(manager, max_running, token_budget, preemption_policy=policy)
    if model is None:
        rt.runner = FakeRunner(manager)
    else:
        pool = KVBlockPool(n_layer=1, num_blocks=num_blocks, block_size=block_size, n_head=2, head_dim=8)
        pool.k.fill_(float("nan"))
        pool.v.fill_(float("nan"))
        rt.runner = ModelRunner(model, pool, manager)
    rt.iteration, rt.records = 0, []
    return rt


def test_deterministic_multi_request_stress():
    for case in range(40):
        rng = random.Random(2026 + case)
        bs = rng.choice((2, 3, 4, 8))
        blocks = rng.choice((2, 3, 4, 5, 6))
        rt = cpu_runtime("recompute", num_blocks=blocks, block_size=bs, max_running=rng.randint(1, 4),
                         token_budget=rng.randint(1, 12))
        seqs = []
        for n in range(rng.randint(2, 5)):
            prompt_len = rng.randint(1, bs * blocks - 1)
            out_len = rng.randint(1, bs * blocks - prompt_len)
            seq = request(chr(65 + n), [1] * prompt_len, out_len)
            rt.add_request(seq)
            seqs.append(seq)
        for _ in range(400):
            if all(s.status == Status.FINISHED for s in seqs):
                break
            rt.step()
            rt.block_manager.check_invariants(seqs)
        else:
            pytest.fail(f"case {case} did not finish")
        assert rt.block_manager.block_owner == {}


def test_real_tiny_model_recompute_matches_conservative():
    torch.manual_seed(2026)
    model = MiniGPT(n_embd=16, n_head=2, vocab_size=32, block_size=64, dropout=0.0, n_layer=1).eval()
    base, pre = cpu_runtime("conservative", model=model), cpu_runtime("recompute", model=model)
    data = [("A", [1, 5, 3, 7]), ("B", [2, 6, 4, 8])]
    bs = [request(n, p, 3) for n, p in data]
    ps = [request(n, p, 3) for n, p in data]
    for s in bs:
        base.add_request(s)
    for s in ps:
        pre.add_request(s)
    with torch.inference_mode():
        for rt, seqs in ((base, bs), (pre, ps)):
            for _ in range(25):
                if all(s.status == Status.FINISHED for s in seqs):
                    break
                rt.step()
    assert pre.scheduler.num_preemptions > 0
    assert [s.generated_tokens for s in bs] == [s.generated_tokens for s in ps]


# ------------------------------------------------------ decode metadata

def test_decode_metadata_semantics():
    torch.manual_seed(0)
    model = MiniGPT(n_embd=16, n_head=2, vocab_size=32, block_size=64, n_layer=1).eval()
    manager = BlockManager(num_blocks=8, block_size=4)
    pool = KVBlockPool(1, 8, 4, 2, 8)
    runner = ModelRunner(model, pool, manager)
    a, b = request("a", [1, 2, 3, 4, 5], 4), request("b", [7, 8], 4)
    manager.reserve_slots(a, 5)
    a.length, a.last_token = 5, 9
    manager.reserve_slots(b, 2)
    b.length, b.last_token = 2, 11
    ids, meta = runner._prepare_decode_batch([a, b])
    assert ids.tolist() == [[9], [11]]
    assert meta.positions.tolist() == [5, 2]
    assert meta.context_lengths.tolist() == [6, 3]
    assert meta.block_tables.tolist() == [a.block_table, b.block_table + [-1]]
    assert meta.slot_mapping.tolist() == [a.block_table[1] * 4 + 1, b.block_table[0] * 4 + 2]
    for t in (meta.positions, meta.context_lengths, meta.block_tables, meta.slot_mapping):
        assert t.dtype == torch.int64


# ------------------------------------------------------ backend routing

def _model():
    torch.manual_seed(10)
    return MiniGPT(n_embd=16, n_head=4, vocab_size=32, block_size=32, dropout=0.0, n_layer=2).eval()


def test_default_backend_and_validation():
    model = _model()
    assert all(b.attn.decode_attention_backend == "reference" for b in model.blocks)
    with pytest.raises(ValueError, match="decode backend"):
        model.set_decode_attention_backend("unknown")
    for name in ("hip", "triton_v0"):
        model.set_decode_attention_backend(name)
        assert all(b.attn.decode_attention_backend == name for b in model.blocks)
    model.set_prefill_fastpath_mode("sdpa_v2")
    assert all(b.attn.decode_attention_backend == "triton_v0" for b in model.blocks)


def test_hip_route_writes_kv_before_attention_and_matches_reference_bitwise():
    """The reference's routing test (two calls: the KV write, then the backend)
    on the HIP route with fused_decode_append off."""
    model = _model()
    for block in model.blocks:
        block.attn.fused_decode_append = False
    inputs = torch.tensor([[1], [2]], dtype=torch.long)
    meta = DecodeBatchMetadata(positions=torch.tensor([0, 0]), context_lengths=torch.tensor([1, 1]),
                               block_tables=torch.tensor([[1], [0]], dtype=torch.long),
                               slot_mapping=torch.tensor([16, 0], dtype=torch.long))

    def make_pool():
        pool = KVBlockPool(n_layer=2, num_blocks=2, block_size=16, n_head=4, head_dim=4)
        pool.k.fill_(float("nan"))
        pool.v.fill_(float("nan"))
        return pool

    pool0, pool1 = make_pool(), make_pool()
    calls = []

    def fake_append(pool, layer_idx, k, v, slot_mapping):
        calls.append(("append", layer_idx))
        keep = slot_mapping >= 0
        pool.k[layer_idx, slot_mapping[keep] // 16, slot_mapping[keep] % 16] = k[keep]
        pool.v[layer_idx, slot_mapping[keep] // 16, slot_mapping[keep] % 16] = v[keep]

    def fake_attention(q, pool, block_tables, context_lengths, layer_idx):
        calls.append(("attn", layer_idx))
        assert torch.isfinite(pool.k[layer_idx, 1, 0]).all() and torch.isfinite(pool.v[layer_idx, 0, 0]).all()
        return paged_attention_batch_online_v1(q, pool, block_tables, context_lengths, layer_idx)

    with torch.inference_mode():
        model.set_decode_attention_backend("reference")
        expected = model.decode_batch(inputs, meta, pool0)
        model.set_decode_attention_backend("hip")
        with patch("minivllm.hip_paged_decode.kv_append", side_effect=fake_append), \
                patch("minivllm.hip_paged_decode.paged_attention_batch_hip", side_effect=fake_attention):
            actual = model.decode_batch(inputs, meta, pool1)
    assert calls == [("append", 0), ("attn", 0), ("append", 1), ("attn", 1)]
    torch.testing.assert_close(expected, actual, atol=0, rtol=0)
    torch.testing.assert_close(pool0.k[:, 1, 0], pool1.k[:, 1, 0], atol=0, rtol=0)
    torch.testing.assert_close(pool0.v[:, 0, 0], pool1.v[:, 0, 0], atol=0, rtol=0)


def test_fused_hip_route_passes_the_step_rows_and_matches_reference_bitwise():
    """The default HIP route makes one call per layer with the step's q, k, v
    and slot mapping (a stand-in does the write and the reference attention):
    logits and KV bit-identical to the reference backend."""
    model = _model()
    inputs = torch.tensor([[1], [2]], dtype=torch.long)
    meta = DecodeBatchMetadata(positions=torch.tensor([0, 0]), context_lengths=torch.tensor([1, 1]),
                               block_tables=torch.tensor([[1], [0]], dtype=torch.long),
                               slot_mapping=torch.tensor([16, 0], dtype=torch.long))
    pools = []
    for _ in range(2):
        pool = KVBlockPool(n_layer=2, num_blocks=2, block_size=16, n_head=4, head_dim=4)
        pool.k.fill_(float("nan"))
        pool.v.fill_(float("nan"))
        pools.append(pool)
    calls = []

    def fake_fused(q, pool, block_tables, context_lengths, layer_idx, k, v, slot_mapping):
        calls.append(layer_idx)
        assert q.shape == k.shape == v.shape == (2, 4, 4) and slot_mapping is meta.slot_mapping
        pool.k[layer_idx, slot_mapping // 16, slot_mapping % 16] = k
        pool.v[layer_idx, slot_mapping // 16, slot_mapping % 16] = v
        return paged_attention_batch_online_v1(q, pool, block_tables, context_lengths, layer_idx)

    with torch.inference_mode():
        model.set_decode_attention_backend("reference")
        expected = model.decode_batch(inputs, meta, pools[0])
        model.set_decode_attention_backend("hip")
        with patch("minivllm.hip_paged_decode.paged_attention_batch_append_hip", side_effect=fake_fused):
            actual = model.decode_batch(inputs, meta, pools[1])
    assert calls == [0, 1]
    torch.testing.assert_close(expected, actual, atol=0, rtol=0)
    torch.testing.assert_close(pools[0].k[:, 1, 0], pools[1].k[:, 1, 0], atol=0, rtol=0)


@pytest.mark.parametrize("backend", ["hip", "triton_v0"])
def test_hip_backend_on_cpu_never_falls_back(backend):
    model = _model()
    model.set_decode_attention_backend(backend)
    pool = KVBlockPool(n_layer=2, num_blocks=1, block_size=16, n_head=4, head_dim=4)
    meta = DecodeBatchMetadata(positions=torch.tensor([0]), context_lengths=torch.tensor([1]),
                               block_tables=torch.tensor([[0]]), slot_mapping=torch.tensor([0]))
    with torch.inference_mode(), pytest.raises((RuntimeError, ValueError)):
        model.decode_batch(torch.tensor([[1]]), meta, pool)


def test_reference_backend_skips_padding_slots():
    model = _model()
    pool = KVBlockPool(n_layer=2, num_blocks=2, block_size=16, n_head=4, head_dim=4)
    pool.k.fill_(7.0)
    pool.v.fill_(7.0)
    before = pool.k.clone()
    meta = DecodeBatchMetadata(positions=torch.tensor([0, 0]), context_lengths=torch.tensor([1, 1]),
                               block_tables=torch.tensor([[1], [0]]), slot_mapping=torch.tensor([16, -1]))
    with torch.inference_mode():
        model.decode_batch(torch.tensor([[1], [2]]), meta, pool)
    assert torch.equal(pool.k[:, 0], before[:, 0])            # padded row wrote nothing
    assert not torch.equal(pool.k[:, 1, 0], before[:, 1, 0])  # the other row did


def test_pack_decode_metadata_matches_row_by_row_construction():
    from minivllm.decode_graphs import metadata_views, pack_decode_metadata

    rng = random.Random(5)
    B, B_pad, M = 5, 8, 12
    tables = [[rng.randrange(100) for _ in range(rng.randint(1, M))] for _ in range(B)]
    tokens = [rng.randrange(50) for _ in range(B)]
    positions = [rng.randrange(1, 200) for _ in range(B)]
    slots = [rng.randrange(1600) for _ in range(B)]
    buf = pack_decode_metadata(tokens, positions, slots, tables, B_pad, M)
    ids, meta = metadata_views(buf, B_pad, M)
    assert ids[:, 0].tolist() == tokens + [0] * (B_pad - B)
    assert meta.positions.tolist() == positions + [0] * (B_pad - B)
    assert meta.context_lengths.tolist() == [p + 1 for p in positions] + [0] * (B_pad - B)
    assert meta.slot_mapping.tolist() == slots + [-1] * (B_pad - B)
    want = [t + [-1] * (M - len(t)) for t in tables] + [[-1] * M] * (B_pad - B)
    assert meta.block_tables.tolist() == want
