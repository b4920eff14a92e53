"""Lock-step comparison of the HIP decode backend with the PyTorch reference
decode backend inside the runtime under recompute preemption, as
experiments/gpu_day6_runtime_decode_ab.py:59-130 compares its two backends:
two runtimes over one model, one request set and two KV pools of the same
size, stepped alternately; after every step the schedules, sequence states,
block tables, lifecycle counts, decode logits, greedy tokens and the
logical KV of every active sequence are compared (see _e2e.Lockstep).

* Full configuration, bf16 (dim 2048 x 16 heads x 12 layers, vocab 32000,
  256 requests with lognormal prompts of mean 512 capped at 4096, 128 output
  tokens, pool at 60% of peak demand, max_running 256, token budget 2048,
  prefill "sdpa_v2" in both runtimes), run to completion (283 iterations, 62
  preemptions, 32 512 decode rows), twice:
    - against the reference backend as it runs in bf16: online_v1 keeps its
      running softmax state in bf16 (rounded at every block) while the HIP
      kernel accumulates in fp32, so the two differ by bf16 rounding that
      grows with the context; bound 2^-6 + 2^-6 * max|ref row| on logits and
      decode-written KV (_e2e.C5_BF16_LOCKSTEP);
    - against online_v1 on float32 copies of q and K/V with its output
      rounded to bf16 (_e2e.online_v1_fp32), the HIP kernel's own arithmetic
      in another order; bound 0.75 * 2^-6 * (1 + max|ref row|)
      (_e2e.C5_FP32_REF_LOCKSTEP).
  Layer-0 and prefill-written KV must be bit-identical. A greedy token may
  differ only where the reference's top-2 margin is below twice its row's
  logit bound; the reference's token is then written into the HIP runtime,
  so the two keep decoding the same tokens and every decode row and every
  live sequence's KV is compared at every step.
* Reduced configuration in fp32 (12 requests, dim 512, 2 layers), run to
  completion with the reference harness's own tolerances (atol 2e-5, rtol
  2e-4, elementwise) on logits and on KVBlockPool.gather_sequence, and
  identical tokens with no forcing.
"""
from __future__ import annotations

import collections
import time

import pytest
import torch

import _e2e

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

C5 = _e2e.RuntimeSpec()
C5_MAX_STEPS = 400
C5_DECODE_ROWS = 256 * (128 - 1)   # every request decodes all but its first output token

REDUCED = _e2e.RuntimeSpec(n_requests=12, prompt_mean=96, prompt_cap=320, output_len=12, n_embd=512, n_head=4,
                           n_layer=2, vocab=2048, max_running=12, token_budget=256, seed=3)


def _report(ls: _e2e.Lockstep, t0: float) -> str:
    s = ls.stats
    return (f"step {s['steps']} decode_rows {s['decode_rows_checked']}/{s['decode_rows']} "
            f"preemptions {s['preemptions']} recomputed {len(s['recomputed_seqs'])} "
            f"forced {len(ls.forced)} in {len(ls.forced_streams)} streams "
            f"max|dlogit| {s['max_logit_abs']:.4g} ({s['max_logit_ratio']:.2f} of bound) "
            f"max|dKV| {s['max_kv_abs']:.4g} ({s['max_kv_ratio']:.2f} of bound) "
            f"kv_tokens {s['kv_tokens_checked']} ({time.perf_counter() - t0:.1f} s)")


def _run_full(progress, criterion: dict, ref_attention=None) -> _e2e.Lockstep:
    torch.backends.cuda.matmul.allow_tf32 = False
    progress("  building the full configuration (dim 2048 x 12 layers, 256 requests, bf16)")
    prompts = _e2e.make_prompts(C5)
    model = _e2e.make_model(C5, DEV, torch.bfloat16)
    ls = _e2e.Lockstep(C5, model, prompts, DEV, torch.bfloat16, ref_attention=ref_attention, **criterion)
    t0 = time.perf_counter()
    with torch.inference_mode():
        while not ls.finished:
            ls.step()
            if ls.stats["steps"] % 10 == 0:
                progress("  " + _report(ls, t0))
            assert ls.stats["steps"] < C5_MAX_STEPS
    progress("  " + _report(ls, t0))
    margins = collections.Counter(round(m, 6) for *_, m in ls.forced)
    progress(f"  streams never forced: {len(ls.ref.seqs) - len(ls.forced_streams)}/{len(ls.ref.seqs)}; "
             f"forced-tie margins: {dict(sorted(margins.items()))}; seconds in steps: reference "
             f"{ls.wall['reference']:.1f}, hip {ls.wall['hip']:.1f}")
    ls.finish_checks()
    assert ls.stats["preemptions"] > 0, "the run must reach recompute preemption"
    assert ls.stats["recomputed_seqs"], "the run must reach a recompute prefill"
    assert ls.stats["decode_rows"] == C5_DECODE_ROWS
    assert ls.stats["decode_rows_checked"] == C5_DECODE_ROWS
    for x in ls.ref.seqs:
        assert x.generated_tokens == ls.hip.by_id[x.seq_id].generated_tokens
    return ls


@pytest.mark.timeout(900)
def test_lockstep_full_runtime_bf16_to_completion(progress):
    _run_full(progress, _e2e.C5_BF16_LOCKSTEP)


@pytest.mark.timeout(900)
def test_lockstep_full_runtime_vs_fp32_accumulating_reference(progress):
    _run_full(progress, _e2e.C5_FP32_REF_LOCKSTEP, ref_attention=_e2e.online_v1_fp32)


@pytest.mark.timeout(600)
def test_lockstep_reduced_runtime_fp32_to_completion(progress):
    torch.backends.cuda.matmul.allow_tf32 = False
    prompts = _e2e.make_prompts(REDUCED)
    model = _e2e.make_model(REDUCED, DEV, torch.float32)
    ls = _e2e.Lockstep(REDUCED, model, prompts, DEV, torch.float32, logit_tol=(2e-5, 2e-4), tie_margin=0.0,
                       kv_tol=None)
    t0 = time.perf_counter()
    with torch.inference_mode():
        while not ls.finished:
            ls.step()
            assert ls.stats["steps"] < 10000
    progress("  " + _report(ls, t0))
    ls.finish_checks()
    assert not ls.forced
    assert ls.stats["decode_rows_checked"] == ls.stats["decode_rows"] > 0
    assert ls.stats["preemptions"] > 0, "the workload must exercise recompute preemption"
    assert ls.stats["recomputed_seqs"]
