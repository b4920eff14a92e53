"""End-to-end runtime workloads built on the minivllm API.

Mini-GPT configuration with golden greedy tokens (``run_c1``): dim 256,
8 heads, 4 layers, vocab 256, fp32, seed 0; paged KV block 16; prompts of
128/256 tokens, batch 1/4; chunked prefill with token budget 64; 8 greedy
tokens. Inputs and the reference runtime's outputs are in
golden/c1_greedy_tokens.json (written by golden/make_c1_greedy_tokens.py).

Full runtime under recompute preemption (the large end-to-end configuration):
  model     MiniGPT(n_embd=2048, n_head=16, vocab_size=32000,
            block_size=max_prompt + output, n_layer=12), random init after
            torch.manual_seed(seed), cast to the run dtype (bf16)
  requests  256, prompt length = min(4096, max(1, round(lognormal(mu, 1.0))))
            with mu = ln 512 - 1/2 (mean 512), uniform token ids, output 128
  KV pool   block_size 16, floor(0.6 * sum_r ceil((P_r + out - 1) / 16))
            blocks (at least the largest single request), so BlockManager
            runs out and the scheduler preempts and recomputes
  schedule  max_running 256, token budget 2048, "recompute" policy,
            prefill mode "sdpa_v2"
Reduced variants (fewer requests / layers / tokens) keep the same recipe.
"""
from __future__ import annotations

import json
import math
import time
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from minivllm.block_manager import BlockManager
from minivllm.kv_block_pool import KVBlockPool
from minivllm.mini_runtime import MiniRuntime
from minivllm.model import MiniGPT
from minivllm.model_runner import ModelRunner
from minivllm.scheduler import Scheduler
from minivllm.sequence import SequenceState, Status


@dataclass
class RuntimeSpec:
    n_requests: int = 256
    prompt_mean: int = 512
    prompt_sigma: float = 1.0
    prompt_cap: int = 4096
    output_len: int = 128
    n_embd: int = 2048
    n_head: int = 16
    n_layer: int = 12
    vocab: int = 32000
    block_size: int = 16
    pool_fraction: float = 0.6
    max_running: int = 256
    token_budget: int = 2048
    policy: str = "recompute"
    prefill_mode: str = "sdpa_v2"
    seed: int = 0


def make_prompts(spec: RuntimeSpec) -> list[list[int]]:
    rng = np.random.default_rng(spec.seed)
    mu = math.log(spec.prompt_mean) - spec.prompt_sigma ** 2 / 2
    lengths = np.clip(np.rint(rng.lognormal(mu, spec.prompt_sigma, spec.n_requests)), 1, spec.prompt_cap)
    return [rng.integers(0, spec.vocab, int(n)).tolist() for n in lengths]


def pool_blocks(spec: RuntimeSpec, prompts: list[list[int]]) -> int:
    S = spec.block_size
    per_req = [math.ceil((len(p) + spec.output_len - 1) / S) for p in prompts]
    return max(max(per_req), int(spec.pool_fraction * sum(per_req)))


def make_model(spec: RuntimeSpec, device, dtype) -> MiniGPT:
    torch.manual_seed(spec.seed)
    model = MiniGPT(n_embd=spec.n_embd, n_head=spec.n_head, vocab_size=spec.vocab,
                    block_size=spec.prompt_cap + spec.output_len, dropout=0.0, n_layer=spec.n_layer)
    model = model.eval().to(device=device, dtype=dtype)
    model.set_prefill_fastpath_mode(spec.prefill_mode)
    return model


def make_runtime(spec: RuntimeSpec, model: MiniGPT, prompts, device, dtype):
    blocks = pool_blocks(spec, prompts)
    manager = BlockManager(num_blocks=blocks, block_size=spec.block_size)
    rt = MiniRuntime.__new__(MiniRuntime)
    rt.block_manager = manager
    rt.scheduler = Scheduler(manager, max_running=spec.max_running,
                             max_num_batched_tokens=spec.token_budget, preemption_policy=spec.policy)
    pool = KVBlockPool(n_layer=spec.n_layer, num_blocks=blocks, block_size=spec.block_size,
                       n_head=spec.n_head, head_dim=spec.n_embd // spec.n_head, device=device, dtype=dtype)
    rt.runner = ModelRunner(model, pool, manager)
    rt.iteration, rt.records, rt.sync_cuda_timing, rt.verbose = 0, [], False, False
    rt._kv_high_watermark = {}
    seqs = [SequenceState(seq_id=f"req_{i:03d}", prompt_tokens=p, max_tokens=len(p) + spec.output_len)
            for i, p in enumerate(prompts)]
    for s in seqs:
        rt.add_request(s)
    return rt, seqs


def record_margins(rt: MiniRuntime) -> dict:
    """Wraps the runner so every greedy choice records its top-2 logit
    margin, keyed by (seq_id, position of the last input token): decode steps
    at the sequence length before the step, prefill chunks at their last row.
    Returns the (filling) dict."""
    margins: dict = {}
    inner_dec, inner_pre = rt.runner.decode_batch, rt.runner.prefill_chunk

    def decode_batch(sequences):
        pos = [s.length for s in sequences]
        logits, toks = inner_dec(sequences)
        top = torch.topk(logits.float(), 2, dim=-1).values.tolist()
        for s, p, t in zip(sequences, pos, top):
            margins[(s.seq_id, p)] = t[0] - t[1]
        return logits, toks

    def prefill_chunk(seq, start_pos, num_tokens):
        logits = inner_pre(seq=seq, start_pos=start_pos, num_tokens=num_tokens)
        t = torch.topk(logits[0, -1].float(), 2).values.tolist()
        margins[(seq.seq_id, start_pos + num_tokens - 1)] = t[0] - t[1]
        return logits

    rt.runner.decode_batch, rt.runner.prefill_chunk = decode_batch, prefill_chunk
    return margins


def first_divergences(base: dict, other: dict, margins: dict) -> list:
    """base/other: seq_id -> (prompt_len, generated tokens). For each stream
    that differs: (seq_id, index of the first different token, the base run's
    top-2 margin at that choice)."""
    out = []
    for sid, (plen, a) in base.items():
        b = other[sid][1]
        if a != b:
            k = next(i for i, (x, y) in enumerate(zip(a, b)) if x != y)
            out.append((sid, k, margins.get((sid, plen + k - 1))))
    return out


def run_to_completion(rt: MiniRuntime, seqs, max_steps: int = 100000, on_step=None) -> dict:
    """Steps the runtime until every request finished; returns throughput figures."""
    sync = torch.cuda.synchronize if torch.cuda.is_available() else (lambda: None)
    sync()
    t0 = time.perf_counter()
    with torch.inference_mode():
        for _ in range(max_steps):
            if all(s.status == Status.FINISHED for s in seqs):
                break
            rt.step()
            if on_step is not None:
                on_step(rt)
    sync()
    wall = time.perf_counter() - t0
    if not all(s.status == Status.FINISHED for s in seqs):
        raise RuntimeError("runtime did not finish")
    summ = rt.metrics_summary()
    decode_ms = sum(r.decode_ms for r in rt.records)
    return {"steps": rt.iteration, "wall_s": round(wall, 3), "output_tokens": summ["output_tokens"],
            "decode_tokens": summ["decode_tokens"], "prefill_tokens": summ["prefill_tokens"],
            "preemptions": summ["preemptions"], "repeated_kv_tokens": summ["repeated_kv_tokens"],
            "output_tok_s": round(summ["output_tokens"] / wall, 1),
            "decode_tok_s_in_decode_phase": round(summ["decode_tokens"] / (decode_ms / 1e3), 1) if decode_ms else None,
            "decode_ms_total": round(decode_ms, 1)}


# ------------------------------------------------- golden-token configuration

GOLDEN_C1 = json.loads((Path(__file__).resolve().parent / "golden" / "c1_greedy_tokens.json").read_text())


def run_c1(case: dict, device, backend: str, prefill_mode: str | None = None):
    """Runs one golden case; returns (generated tokens per request, runtime).

    prefill_mode overrides the recorded configuration's prefill mode (the
    golden tokens were produced with it)."""
    cfg = GOLDEN_C1["config"]
    torch.manual_seed(cfg["seed"])
    model = MiniGPT(n_embd=cfg["n_embd"], n_head=cfg["n_head"], vocab_size=cfg["vocab_size"],
                    block_size=cfg["block_size"], dropout=0.0, n_layer=cfg["n_layer"]).eval().to(device)
    model.set_prefill_fastpath_mode(prefill_mode or cfg["prefill_mode"])
    model.set_decode_attention_backend(backend)
    B, P, S = case["batch"], case["prompt_len"], cfg["block_size_kv"]
    blocks = B * math.ceil((P + cfg["output_len"] - 1) / S)
    assert blocks == case["num_blocks"]
    manager = BlockManager(num_blocks=blocks, block_size=S)
    rt = MiniRuntime.__new__(MiniRuntime)
    rt.block_manager = manager
    rt.scheduler = Scheduler(manager, max_running=B, max_num_batched_tokens=cfg["token_budget"],
                             preemption_policy="conservative")
    pool = KVBlockPool(n_layer=cfg["n_layer"], num_blocks=blocks, block_size=S, n_head=cfg["n_head"],
                       head_dim=cfg["n_embd"] // cfg["n_head"], device=device)
    pool.k.fill_(float("nan"))
    pool.v.fill_(float("nan"))
    rt.runner = ModelRunner(model, pool, manager)
    rt.iteration, rt.records = 0, []
    seqs = [SequenceState(seq_id=f"req_{i:02d}", prompt_tokens=case["prompts"][i],
                          max_tokens=P + cfg["output_len"]) for i in range(B)]
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
