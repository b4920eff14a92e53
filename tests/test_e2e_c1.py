"""End to end: greedy token streams of the Mini-GPT configuration
(dim 256, 8 heads, 4 layers, vocab 256, fp32, seed 0; paged KV block 16;
prompts 128/256 x batch 1/4; chunked prefill, token budget 64; 8 greedy
tokens) must equal the reference runtime's, recorded in
golden/c1_greedy_tokens.json by golden/make_c1_greedy_tokens.py.

CPU: the PyTorch "reference" decode backend. GPU: the HIP backend
(kv_append + paged decode kernels) on cuda:0.
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
