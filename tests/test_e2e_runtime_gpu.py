"""The full runtime under recompute preemption on the GPU: the HIP decode
backend against the PyTorch reference backend, same weights, same requests
(reduced version of the large end-to-end configuration so the PyTorch
backend, which launches ~20 ops per block-table column per layer, finishes
in seconds).

Comparison (as in experiments/gpu_day6_runtime_decode_ab.py:59-130):
  * scheduling is token-independent, so iterations, preemptions, repeated KV
    tokens and prefill/decode token counts must be identical;
  * fp32: decode logits within 2e-4 and greedy tokens identical;
  * bf16 and f16: the reference backend accumulates in the 16-bit type and
    the HIP kernels in fp32, so tokens may only differ where the reference's
    top-2 logit margin is a near tie (< 0.1); the first token (from prefill,
    shared by both backends) must always agree.
"""
from __future__ import annotations

import pytest
import torch

import _e2e

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SPEC = _e2e.RuntimeSpec(n_requests=12, prompt_mean=96, prompt_cap=320, output_len=12, n_embd=512, n_head=4,
                        n_layer=2, vocab=2048, max_running=12, token_budget=256, seed=3)
NEAR_TIE = 0.1


def run_capture(model, backend, prompts, dtype):
    print(f"  runtime backend={backend} dtype={dtype}", flush=True)
    model.set_decode_attention_backend(backend)
    rt, seqs = _e2e.make_runtime(SPEC, model, prompts, DEV, dtype)
    captured = {}
    inner = rt.runner.decode_batch

    def decode_batch(sequences):
        positions = [s.length for s in sequences]
        logits, tokens = inner(sequences)
        top = torch.topk(logits.float(), 2, dim=-1)
        for s, pos, vals, row in zip(sequences, positions, top.values.tolist(), logits.float()):
            captured[(s.seq_id, pos)] = (vals[0] - vals[1], row.cpu())
        return logits, tokens

    rt.runner.decode_batch = decode_batch
    stats = _e2e.run_to_completion(rt, seqs)
    rt.block_manager.check_invariants([])
    assert not rt.block_manager.block_owner
    return {s.seq_id: (len(s.prompt_tokens), list(s.generated_tokens)) for s in seqs}, captured, stats


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_runtime_with_preemption_hip_matches_reference(dtype):
    torch.backends.cuda.matmul.allow_tf32 = False
    prompts = _e2e.make_prompts(SPEC)
    model = _e2e.make_model(SPEC, DEV, dtype)
    ref, ref_logits, ref_stats = run_capture(model, "reference", prompts, dtype)
    hip, hip_logits, hip_stats = run_capture(model, "hip", prompts, dtype)
    assert ref_stats["preemptions"] > 0, "workload must exercise recompute preemption"
    for key in ("steps", "preemptions", "repeated_kv_tokens", "prefill_tokens", "decode_tokens",
                "output_tokens"):
        assert ref_stats[key] == hip_stats[key], key
    diverged = []
    for sid, (plen, a) in ref.items():
        b = hip[sid][1]
        if a == b:
            continue
        k = next(i for i, (x, y) in enumerate(zip(a, b)) if x != y)
        assert k > 0, f"{sid}: first (prefill) token differs"
        margin = ref_logits[(sid, plen + k - 1)][0]
        diverged.append((sid, k, margin))
    print(f"  identical sequences: {len(ref) - len(diverged)}/{len(ref)}; diverged at "
          f"(seq, token, ref top-2 margin) {diverged}", flush=True)
    if dtype == torch.float32:
        assert not diverged
        for key, (_, row) in ref_logits.items():
            torch.testing.assert_close(hip_logits[key][1], row, rtol=2e-4, atol=2e-4)
    else:
        assert all(m < NEAR_TIE for _, _, m in diverged), diverged
