"""End to end: greedy token streams of the Mini-GPT configuration
(dim 256, 8 heads, 4 layers, vocab 256, fp32, seed 0; paged KV block 16;
prompts 128/256 x batch 1/4; chunked prefill, token budget 64; 8 greedy
tokens) must equal the reference runtime's, recorded in
golden/c1_greedy_tokens.json by golden/make_c1_greedy_tokens.py.

CPU: the PyTorch "reference" decode backend. GPU: the HIP backend
(kv_append + paged decode kernels) on cuda:0.

Forced recompute preemption: the batch-4 cases on a pool of half the blocks
the whole run needs ("recompute" policy, capacity factor 0.5 as
experiments/gpu_e2e_runtime.py:96-103 sizes it) preempt one request once and
replay 16 KV tokens, the lifecycle of the reference's published
forced-preemption row (README.md:221-223: 1 preemption, 16 replayed KV
tokens, identical tokens and lifecycle counts in both backends). The token
streams equal the golden ones of the run without preemption.
"""
from __future__ import annotations

import pytest
import torch

from _e2e import GOLDEN_C1 as GOLDEN
from _e2e import run_c1


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


FORCED = [c for c in GOLDEN["cases"] if c["batch"] == 4]


def _lifecycle(rt):
    m = rt.metrics_summary()
    return (rt.iteration, m["output_tokens"], m["preemptions"], m["repeated_kv_tokens"], m["prefill_tokens"],
            m["decode_tokens"])


@pytest.mark.parametrize("case", FORCED, ids=_ids)
def test_forced_recompute_preemption_reference_cpu(case):
    torch.set_num_threads(1)
    tokens, rt = run_c1(case, "cpu", "reference", policy="recompute", kv_factor=0.5)
    summary = rt.metrics_summary()
    assert (summary["preemptions"], summary["repeated_kv_tokens"]) == (1, 16)
    assert tokens == case["outputs"]


@pytest.mark.gpu
@pytest.mark.parametrize("case", FORCED, ids=_ids)
def test_forced_recompute_preemption_both_backends_gpu(case):
    """Reference and HIP decode backends on the GPU: one preemption, 16
    replayed KV tokens, identical tokens and lifecycle counts."""
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    out = {}
    for backend in ("reference", "hip"):
        print(f"  C1 forced preemption {backend} {_ids(case)}", flush=True)
        tokens, rt = run_c1(case, "cuda", backend, policy="recompute", kv_factor=0.5)
        out[backend] = (tokens, _lifecycle(rt))
    assert out["hip"] == out["reference"]
    assert out["hip"][1][2:4] == (1, 16)
    assert out["hip"][0] == case["outputs"]
