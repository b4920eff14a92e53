"""End to end: greedy token streams of the Mini-GPT configuration
(dim 256, 8 heads, 4 layers, vocab 256, fp32, seed 0; paged KV block 16;
prompts 128/256 x batch 1/4; chunked prefill, token budget 64; 8 greedy
tokens) must equal the reference runtime's, recorded in
golden/c1_greedy_tokens.json by golden/make_c1_greedy_tokens.py.

CPU: the PyTorch "reference" decode backend. GPU: the HIP backend
(kv_append + paged decode kernels) on cuda:0.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import pytest
import torch

from minivllm.block_manager import BlockManager
from minivllm.kv_block_pool import KVBlockPool
from minivllm.mini_runtime import MiniRuntime
from minivllm.model import MiniGPT
from minivllm.model_runner import ModelRunner
from minivllm.scheduler import Scheduler
from minivllm.sequence import SequenceState, Status

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "c1_greedy_tokens.json").read_text())
CFG = GOLDEN["config"]


def run_c1(case: dict, device: str, backend: str) -> tuple[list[list[int]], MiniRuntime]:
    torch.manual_seed(CFG["seed"])
    model = MiniGPT(n_embd=CFG["n_embd"], n_head=CFG["n_head"], vocab_size=CFG["vocab_size"],
                    block_size=CFG["block_size"], dropout=0.0, n_layer=CFG["n_layer"]).eval().to(device)
    model.set_prefill_fastpath_mode(CFG["prefill_mode"])
    model.set_decode_attention_backend(backend)
    B, P, S = case["batch"], case["prompt_len"], CFG["block_size_kv"]
    blocks = B * math.ceil((P + CFG["output_len"] - 1) / S)
    assert blocks == case["num_blocks"]
    manager = BlockManager(num_blocks=blocks, block_size=S)
    rt = MiniRuntime.__new__(MiniRuntime)
    rt.block_manager = manager
    rt.scheduler = Scheduler(manager, max_running=B, max_num_batched_tokens=CFG["token_budget"],
                             preemption_policy="conservative")
    pool = KVBlockPool(n_layer=CFG["n_layer"], num_blocks=blocks, block_size=S, n_head=CFG["n_head"],
                       head_dim=CFG["n_embd"] // CFG["n_head"], device=device)
    pool.k.fill_(float("nan"))
    pool.v.fill_(float("nan"))
    rt.runner = ModelRunner(model, pool, manager)
    rt.iteration, rt.records = 0, []
    seqs = [SequenceState(seq_id=f"req_{i:02d}", prompt_tokens=case["prompts"][i],
                          max_tokens=P + CFG["output_len"]) for i in range(B)]
    for s in seqs:
        rt.add_request(s)
    with torch.inference_mode():
        for _ in range(1000):
            if all(s.status == Status.FINISHED for s in seqs):
                break
            rt.step()
            manager.check_invariants([s for s in seqs if s.status != Status.FINISHED])
    assert all(s.status == Status.FINISHED for s in seqs)
    return [s.generated_tokens for s in seqs], rt


def _ids(case):
    return f"B{case['batch']}_P{case['prompt_len']}"


@pytest.mark.parametrize("case", GOLDEN["cases"], ids=_ids)
def test_reference_backend_matches_golden_tokens_cpu(case):
    torch.set_num_threads(1)
    tokens, rt = run_c1(case, "cpu", "reference")
    assert tokens == case["outputs"]
    summary = rt.metrics_summary()
    assert (rt.iteration, summary["prefill_tokens"], summary["decode_tokens"]) == \
        (case["iterations"], case["prefill_tokens"], case["decode_tokens"])


@pytest.mark.gpu
@pytest.mark.parametrize("case", GOLDEN["cases"], ids=_ids)
def test_hip_backend_matches_golden_tokens_gpu(case):
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    print(f"  C1 hip backend {_ids(case)}", flush=True)
    tokens, rt = run_c1(case, "cuda", "hip")
    assert tokens == case["outputs"]
    assert rt.iteration == case["iterations"]
