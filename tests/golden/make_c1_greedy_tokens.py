"""Writes c1_greedy_tokens.json: greedy token streams of the reference runtime.

Runs the reference implementation (imported from /root/reference, which only
exists in the build container) on the Mini-GPT end-to-end configuration and
records inputs and outputs as a small fixture:
  model   MiniGPT(n_embd=256, n_head=8, vocab_size=256, block_size=296,
          n_layer=4), fp32, random init after torch.manual_seed(0)
  prefill 'sdpa_v2' mode, chunked with token budget 64
  KV      paged, block_size 16, B * ceil((P + 8 - 1) / 16) blocks
  sched   max_running = B, 'conservative' policy
  work    prompts of P in {128, 256} uniform-random ids in [0, 256), batch
          B in {1, 4}, 8 output tokens each (greedy)
Prompts come from torch.Generator seeded 10_000 + 100 * B + P.

Usage (build container only):  python tests/golden/make_c1_greedy_tokens.py
The reference modules are compiled from their .py sources into a temporary
bytecode cache (sys.pycache_prefix); the .pyc files shipped in the reference
tree are never read.
"""
from __future__ import annotations

import json
import math
import sys
import tempfile
from pathlib import Path

REFERENCE = "/root/reference"
OUT = Path(__file__).resolve().parent / "c1_greedy_tokens.json"
CONFIG = dict(n_embd=256, n_head=8, vocab_size=256, block_size=296, n_layer=4, block_size_kv=16,
              token_budget=64, output_len=8, prefill_mode="sdpa_v2", seed=0)


def prompts_for(torch, B: int, P: int) -> list[list[int]]:
    g = torch.Generator().manual_seed(10_000 + 100 * B + P)
    return torch.randint(0, CONFIG["vocab_size"], (B, P), generator=g).tolist()


def run_case(B: int, P: int) -> dict:
    import torch
    from minivllm.block_manager import BlockManager
    from minivllm.kv_block_pool import KVBlockPool
    from minivllm.mini_runtime import MiniRuntime
    from minivllm.model import MiniGPT
    from minivllm.model_runner import ModelRunner
    from minivllm.scheduler import Scheduler
    from minivllm.sequence import SequenceState, Status

    torch.manual_seed(CONFIG["seed"])
    model = MiniGPT(n_embd=CONFIG["n_embd"], n_head=CONFIG["n_head"], vocab_size=CONFIG["vocab_size"],
                    block_size=CONFIG["block_size"], dropout=0.0, n_layer=CONFIG["n_layer"]).eval()
    model.set_prefill_fastpath_mode(CONFIG["prefill_mode"])
    prompts = prompts_for(torch, B, P)
    S, out_len = CONFIG["block_size_kv"], CONFIG["output_len"]
    blocks = B * math.ceil((P + out_len - 1) / S)
    manager = BlockManager(num_blocks=blocks, block_size=S)
    rt = MiniRuntime.__new__(MiniRuntime)
    rt.block_manager = manager
    rt.scheduler = Scheduler(manager, max_running=B, max_num_batched_tokens=CONFIG["token_budget"],
                             preemption_policy="conservative")
    pool = KVBlockPool(n_layer=CONFIG["n_layer"], num_blocks=blocks, block_size=S,
                       n_head=CONFIG["n_head"], head_dim=CONFIG["n_embd"] // CONFIG["n_head"])
    rt.runner = ModelRunner(model, pool, manager)
    rt.iteration, rt.records, rt.sync_cuda_timing, rt.verbose = 0, [], False, False
    rt._kv_high_watermark = {}
    seqs = [SequenceState(seq_id=f"req_{i:02d}", prompt_tokens=prompts[i], max_tokens=P + out_len)
            for i in range(B)]
    for s in seqs:
        rt.add_request(s)
    with torch.inference_mode():
        for _ in range(1000):
            if all(s.status == Status.FINISHED for s in seqs):
                break
            rt.step()
    assert all(s.status == Status.FINISHED for s in seqs)
    summary = rt.metrics_summary()
    return {"batch": B, "prompt_len": P, "num_blocks": blocks, "prompts": prompts,
            "outputs": [s.generated_tokens for s in seqs], "iterations": rt.iteration,
            "prefill_tokens": summary["prefill_tokens"], "decode_tokens": summary["decode_tokens"]}


def main() -> None:
    # Compile the reference's .py sources into a fresh bytecode cache, so no
    # .pyc shipped next to them is ever loaded.
    sys.pycache_prefix = tempfile.mkdtemp(prefix="ref_pycache_")
    sys.dont_write_bytecode = False
    sys.path.insert(0, REFERENCE)
    import torch

    torch.set_num_threads(1)
    cases = [run_case(B, P) for P in (128, 256) for B in (1, 4)]
    OUT.write_text(json.dumps({"config": CONFIG, "source": "reference MiniRuntime on CPU, fp32",
                               "torch": torch.__version__, "cases": cases}, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
