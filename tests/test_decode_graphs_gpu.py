"""Captured decode steps (minivllm.decode_graphs) on the MI355X.

Every replay is checked against the eager step at the same shapes, several
times, with eager work and synchronizations between replays; end-to-end
token streams with graphs enabled must equal the eager ones.
"""
from __future__ import annotations

import pytest
import torch

import _e2e
from minivllm.decode_graphs import DecodeGraphs, metadata_views, pack_decode_metadata
from minivllm.kv_block_pool import KVBlockPool
from minivllm.model import MiniGPT

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _model(dtype, n_embd=512, n_head=4, n_layer=2, vocab=1000, block_size=512):
    torch.manual_seed(7)
    m = MiniGPT(n_embd=n_embd, n_head=n_head, vocab_size=vocab, block_size=block_size, n_layer=n_layer)
    m = m.eval().to(device=DEV, dtype=dtype)
    m.set_decode_attention_backend("hip")
    return m


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_replays_match_eager_bitwise(dtype):
    model = _model(dtype)
    S, N, M = 16, 96, 32
    pool = KVBlockPool(model.n_layer, N, S, 4, 128, device=DEV, dtype=dtype)
    g = torch.Generator(device=DEV).manual_seed(1)
    pool.k.normal_(generator=g)
    pool.v.normal_(generator=g)
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(2)).tolist()
    lengths = [5, 100, 257, 31]              # tokens already cached per sequence
    tables, used = [], 0
    for L in lengths:
        n = L // S + 1
        tables.append(perm[used:used + n])
        used += n
    slots = [t[L // S] * S + L % S for t, L in zip(tables, lengths)]
    tokens = [3, 14, 159, 265]
    graphs = DecodeGraphs(model, pool, M, buckets=(4,))
    host = pack_decode_metadata(tokens, lengths, slots, tables, 4, M)
    ids, meta = metadata_views(host.to(DEV), 4, M)
    with torch.inference_mode():
        eager = model.decode_batch(ids, meta, pool)[:, -1, :].clone()
        eager_tok = torch.argmax(eager, dim=-1).tolist()
        idle_ids, idle_meta = metadata_views(pack_decode_metadata([], [], [], [], 4, M).to(DEV), 4, M)
        for i in range(4):
            print(f"  replay {i} {dtype}", flush=True)
            logits, toks = graphs.run(tokens, lengths, slots, tables)
            torch.cuda.synchronize()
            assert torch.equal(logits.view(torch.int16 if dtype == torch.bfloat16 else torch.int32),
                               eager.view(torch.int16 if dtype == torch.bfloat16 else torch.int32))
            assert toks == eager_tok
            model.decode_batch(idle_ids, idle_meta, pool)      # eager work between replays
            torch.cuda.synchronize()


@pytest.mark.parametrize("case", _e2e.GOLDEN_C1["cases"],
                         ids=lambda c: f"B{c['batch']}_P{c['prompt_len']}")
def test_small_model_golden_tokens_with_graphs(case, monkeypatch):
    torch.backends.cuda.matmul.allow_tf32 = False
    from minivllm import model_runner

    real_init = model_runner.ModelRunner.__init__

    def init_with_graphs(self, model, kv_pool, block_manager):
        real_init(self, model, kv_pool, block_manager)
        self.enable_decode_graphs()

    monkeypatch.setattr(model_runner.ModelRunner, "__init__", init_with_graphs)
    tokens, rt = _e2e.run_c1(case, "cuda", "hip")
    assert getattr(rt.runner, "_decode_graphs", None) is not None
    assert tokens == case["outputs"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_preemption_runtime_graphs_match_eager(dtype):
    """Graph replays pad the batch to a bucket, so GEMM shapes differ from the
    eager step: fp32 tokens must be identical; bf16 tokens may differ only
    where the eager step's top-2 logit margin is a near tie (< 0.1)."""
    spec = _e2e.RuntimeSpec(n_requests=12, prompt_mean=96, prompt_cap=320, output_len=12, n_embd=512,
                            n_head=4, n_layer=2, vocab=2048, max_running=12, token_budget=256, seed=3)
    prompts = _e2e.make_prompts(spec)
    model = _e2e.make_model(spec, DEV, dtype)
    model.set_decode_attention_backend("hip")
    out, margins = {}, {}
    for graphs in (False, True):
        rt, seqs = _e2e.make_runtime(spec, model, prompts, DEV, dtype)
        if graphs:
            rt.runner.enable_decode_graphs()
        else:
            margins = _e2e.record_margins(rt)
        stats = _e2e.run_to_completion(rt, seqs)
        out[graphs] = ({s.seq_id: (len(s.prompt_tokens), s.generated_tokens) for s in seqs}, stats)
    assert out[False][1]["preemptions"] > 0
    for key in ("steps", "preemptions", "repeated_kv_tokens", "output_tokens"):
        assert out[False][1][key] == out[True][1][key], key
    diverged = _e2e.first_divergences(out[False][0], out[True][0], margins)
    assert all(k > 0 for _, k, _ in diverged)
    print(f"  graphs vs eager, {dtype}: diverged {diverged}", flush=True)
    if dtype == torch.float32:
        assert not diverged
    else:
        assert all(m < 0.1 for _, _, m in diverged), diverged
