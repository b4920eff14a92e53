"""Paged decode attention on one MI355X: achieved HBM GB/s (and % of the
8 TB/s peak) plus sequences/s, on the decode microbench workload:
B=64 sequences, 32 heads, head_dim 128, block_size 16, contexts ~ U[512, 4096],
block tables drawn as a random permutation of a 20000-block pool, seeded
N(0,1) values. One step = one paged_attention_batch_hip call (one layer of
one decode step) over the batch, inputs resident in HBM.

Prints ONE JSON line. `value` = algorithmic bytes / time per step, where the
algorithmic bytes are
  sum_b ctx_b*H*D*e*2 + B*H*D*(e_q + e_out) + sum_b ceil(ctx_b/S)*e_idx + B*e_idx
(valid tokens only; partial-block padding, split partials and the merge pass
are overhead). Time per step is the median of K per-call HIP event pairs on
torch's current stream (the stream the kernels launch on), after about
50 ms of untimed calls (the GPU's clocks settle under sustained load) and W
untimed calls, the region bracketed by device synchronisations. `cpu_baseline`
times the C restatement of the reference's online-softmax decode
(oracle/paged_decode_oracle.c, fp32 accumulation) on this host's cores over
the same workload, with rows for the package's PyTorch online_v1 on the CPU
(bf16 as-is and fp32-upcast), the KV append plus decode step, the long
contexts, the small end-to-end model and a window of the full runtime.

Extras (skipped with --no-extras) time other decode shapes, the KV append,
the KV append plus decode attention of one high-batch step on one pool, the
paged prefill kernel, attention-only speedups against the PyTorch online_v1
and the small-model end-to-end A/B against the PyTorch reference backend
(the reference's method: 2 warm-ups and 7 alternating repeats, with and
without forced recompute preemption). The end-to-end block (skipped with
--no-e2e) runs the full runtime under recompute preemption and puts its
decode tokens/s (generated tokens / wall seconds) in `end_to_end`, then runs
it to completion in lock step against the PyTorch reference decode backend
(skipped with --no-lockstep; --lockstep-fp32 adds a second run against
online_v1 on float32 copies), checking every decode row.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--dtype bf16|fp32]
                       [--split-tokens P] [--no-extras] [--no-cpu-baseline]
                       [--no-e2e] [--e2e-requests R] [--no-lockstep]
                       [--lockstep-fp32] [--prefill]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "mini-gpt-inference_amd"), str(ROOT), str(ROOT / "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "paged decode attn HBM GB/s (% of peak) + decode tokens/s, 1 MI355X"
PEAK_GBPS = 8000.0
# Main-line decode shapes: name -> (B, pool blocks, ctx low, ctx high, description); 32 heads,
# head_dim 128, block_size 16, seed 0.
WORKLOADS = {
    "microbench": (64, 20000, 512, 4096, "paged decode attention microbench (one layer, one decode step)"),
    "longctx": (8, 65536, 32768, 131072, "paged decode attention, long contexts (one layer, one decode step)"),
    "b256": (256, 32768, 128, 2048, "paged decode attention, high batch (one layer, one decode step)"),
}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # Untimed calls after the ~50 ms clock-settle phase every decode line runs;
    # with that phase the median no longer depends on this count (the median
    # read 82.68-82.70 % after 10 calls and no settle phase, 82.85-82.89 % after 200).
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--dtype", choices=("bf16", "fp32"), default="bf16")
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--workload", choices=tuple(WORKLOADS), default="microbench",
                    help="decode shape of the main line (default: the microbench; the others are the "
                         "long-context and high-batch shapes of the extras, for profiling)")
    ap.add_argument("--no-extras", action="store_true", help="skip the other workload shapes")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the full runtime under recompute preemption (dim 2048, 12 layers, "
                         "vocab 32000, bf16, 256 requests, 128 output tokens) that reports decode "
                         "tokens/s")
    ap.add_argument("--e2e-requests", type=int, default=256)
    ap.add_argument("--no-lockstep", action="store_true",
                    help="skip the full runtime run in lock step against the PyTorch reference decode "
                         "backend (about 3 minutes)")
    ap.add_argument("--lockstep-fp32", action="store_true",
                    help="also run the lock step against online_v1 on float32 copies of q and K/V "
                         "(about 3 more minutes)")
    ap.add_argument("--prefill", action="store_true",
                    help="also time the paged prefill kernel (implied unless --no-extras)")
    ap.add_argument("--e2e-trace", action="store_true",
                    help="run only the full runtime once (HIP prefill and decode, eager) and print "
                         "its statistics with the decode attention's algorithmic KV bytes, for a "
                         "kernel trace")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="also run a device-to-device copy of this many MiB (3 times) so rocprof "
                         "counters can be scaled by a kernel of known traffic")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_steps(fn, steps: int, warmup: int) -> float:
    """Milliseconds per call of fn over `steps` back-to-back calls (one HIP
    event pair around all of them, on the current stream): the throughput
    rate, host overhead included when the host is slower than the GPU."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def warm_up(fn, ms: float = 50.0, cap: int = 2000) -> None:
    """Untimed back-to-back calls of fn for about `ms` of GPU time (at most
    `cap` calls): under sustained matrix-core load the GPU's clocks take tens
    of milliseconds to settle, and a few warm-up calls leave the first timed
    ones 10-20 % slow."""
    import torch

    fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    fn()
    end.record()
    torch.cuda.synchronize()
    one = max(start.elapsed_time(end), 1e-3)
    for _ in range(min(cap, int(ms / one))):
        fn()
    torch.cuda.synchronize()


def time_calls(fn, steps: int, warmup: int) -> dict:
    """Per-call HIP event pairs on the current stream (the stream the kernels
    launch on), `steps` calls after `warmup` untimed ones, bracketed by device
    synchronisations: median, mean and min milliseconds per call, plus the
    host wall time of the bracketed region per call."""
    import torch

    for _ in range(warmup):
        fn()
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s, e in pairs:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps * 1e3
    ms = [s.elapsed_time(e) for s, e in pairs]
    return {"median_ms": statistics.median(ms), "mean_ms": statistics.fmean(ms), "min_ms": min(ms),
            "wall_ms": wall, "calls": steps}


def decode_line(w, steps, warmup, split):
    """One decode-attention call per step; the rate is algorithmic bytes over
    the median of the per-call event timings. About 50 ms of untimed calls
    run first so the GPU's clocks settle (as for the prefill lines), then
    `warmup` untimed calls, then the `steps` timed ones."""
    from minivllm import hip_paged_decode as hpd

    fn = lambda: hpd.paged_attention_batch_hip(w.q, w.pool, w.tables, w.ctx, w.layer,  # noqa: E731
                                               split_tokens=split)
    warm_up(fn)
    t = time_calls(fn, steps, warmup)
    ms = t["median_ms"]
    nbytes = w.algorithmic_bytes()
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"ms": round(ms, 5), "mean_ms": round(t["mean_ms"], 5), "min_ms": round(t["min_ms"], 5),
            "wall_ms_per_call": round(t["wall_ms"], 5), "calls": t["calls"],
            "gbps": round(gbps, 1), "pct_of_peak": round(100 * gbps / PEAK_GBPS, 2),
            "alg_bytes": nbytes, "sum_ctx": int(w.ctx.sum()),
            "seq_per_s_per_layer": round(w.q.shape[0] / (ms * 1e-3), 1)}


def append_line(steps, warmup, dev):
    """KV append at B=256, H=32, D=128, bf16 into a fragmented 32768-block pool."""
    import torch

    from minivllm import hip_paged_decode as hpd
    from minivllm.kv_block_pool import KVBlockPool

    B, H, D, S, N = 256, 32, 128, 16, 32768
    g = torch.Generator().manual_seed(0)
    slots = torch.randperm(N * S, generator=g)[:B]
    slots[torch.randperm(B, generator=g)[: B // 10]] = -1
    pool = KVBlockPool(1, N, S, H, D, device=dev, dtype=torch.bfloat16)
    k = torch.randn(B, H, D, device=dev).to(torch.bfloat16)
    v = torch.randn(B, H, D, device=dev).to(torch.bfloat16)
    sl = slots.to(dev)
    fn = lambda: hpd.kv_append(pool, 0, k, v, sl)  # noqa: E731
    t = time_calls(fn, steps, warmup)
    back_to_back = time_steps(fn, steps, warmup)
    n_valid = int((slots >= 0).sum())
    nbytes = n_valid * H * D * 2 * 2 * 2 + B * 8
    ms = t["median_ms"]
    return {"us": round(ms * 1e3, 2), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "back_to_back_us_per_call": round(back_to_back * 1e3, 2), "valid_rows": n_valid,
            "alg_bytes": nbytes,
            "note": "us: median per-call event pair, from before the Python wrapper to the end of the "
                    "kernel (launch-latency bound; the working set is cache resident); back_to_back: "
                    "calls issued in a loop, the host rate"}


def c3_step_line(steps, warmup, dev):
    """One high-batch decode step of one layer as the KV-append-plus-decode
    configuration states it: B=256, H=32, D=128, bf16, ctx ~ U[128, 2048],
    a 32768-block pool allocated from a seeded permutation. Each row's new
    token is appended at slot table[ctx // 16] * 16 + ctx % 16 (a fresh block
    when ctx % 16 == 0), 10 % of the rows are padding (slot -1), then decode
    attention runs over ctx + 1 tokens for appended rows and ctx for padded
    ones. The append and the attention are timed together, on one pool: as
    the two calls (kv_append, then paged decode) and as the one fused call
    (paged_attention_batch_append_hip, the runtime's default), whose outputs
    are checked bit-identical to the two calls'."""
    import torch

    import _fixtures as fx
    from minivllm import hip_paged_decode as hpd
    from minivllm.kv_block_pool import KVBlockPool

    B, H, D, S, N = 256, 32, 128, 16, 32768
    g = torch.Generator().manual_seed(0)
    ctx = torch.randint(128, 2049, (B,), generator=g, dtype=torch.int64)
    pad = torch.zeros(B, dtype=torch.bool)
    pad[torch.randperm(B, generator=g)[: B // 10]] = True
    lens = torch.where(pad, ctx, ctx + 1)
    nblk = (lens + S - 1) // S
    M = int(nblk.max())
    perm = torch.randperm(N, generator=g)
    tables = torch.full((B, M), -1, dtype=torch.int64)
    starts = torch.cumsum(nblk, 0) - nblk
    for b in range(B):
        tables[b, : nblk[b]] = perm[starts[b]: starts[b] + nblk[b]]
    col = torch.clamp(ctx // S, max=M - 1)
    slots = torch.where(pad, torch.full_like(ctx, -1), tables[torch.arange(B), col] * S + ctx % S)
    assert bool((slots[~pad] >= 0).all())
    pool = KVBlockPool(1, N, S, H, D, device=dev, dtype=torch.bfloat16)
    gd = torch.Generator(device=dev).manual_seed(1)
    for t in (pool.k, pool.v):
        t.normal_(generator=gd)
    q = torch.randn((B, H, D), generator=gd, device=dev).to(torch.bfloat16)
    k_new = torch.randn((B, H, D), generator=gd, device=dev).to(torch.bfloat16)
    v_new = torch.randn((B, H, D), generator=gd, device=dev).to(torch.bfloat16)
    tables_d, lens_d, slots_d = tables.to(dev), lens.to(dev), slots.to(dev)

    def step():
        hpd.kv_append(pool, 0, k_new, v_new, slots_d)
        return hpd.paged_attention_batch_hip(q, pool, tables_d, lens_d, 0)

    def fused():
        return hpd.paged_attention_batch_append_hip(q, pool, tables_d, lens_d, 0, k_new, v_new, slots_d)

    same = bool(torch.equal(step(), fused()))
    ms = time_calls(step, steps, warmup)["median_ms"]
    ms_fused = time_calls(fused, steps, warmup)["median_ms"]
    n_valid = int((~pad).sum())
    append_bytes = n_valid * H * D * 2 * 2 * 2 + B * 8
    attn_bytes = fx.DecodeWorkload(q, pool, tables_d, lens_d, 0, {}).algorithmic_bytes()
    gbps = (append_bytes + attn_bytes) / (ms * 1e-3) / 1e9
    gbps_fused = (append_bytes + attn_bytes) / (ms_fused * 1e-3) / 1e9
    return {"us": round(ms * 1e3, 2), "gbps": round(gbps, 1), "pct_of_peak": round(100 * gbps / PEAK_GBPS, 2),
            "fused_us": round(ms_fused * 1e3, 2), "fused_pct_of_peak": round(100 * gbps_fused / PEAK_GBPS, 2),
            "fused_bit_identical": same,
            "append_bytes": append_bytes, "attention_bytes": attn_bytes, "valid_rows": n_valid,
            "sum_ctx": int(lens.sum()), "rows_per_s_per_layer": round(B / (ms_fused * 1e-3), 1)}


def copy_line(mib: int, dev, reps: int = 3):
    """Device-to-device copy of `mib` MiB: read + write bandwidth, the sanity ceiling."""
    import torch

    src = torch.empty(mib * (1 << 20), dtype=torch.uint8, device=dev)
    src.fill_(1)
    dst = torch.empty_like(src)
    ms = time_steps(lambda: dst.copy_(src), reps, 1)
    return {"mib": mib, "ms": round(ms, 4), "gbps_read_plus_write": round(2 * src.numel() / (ms * 1e-3) / 1e9, 1)}


_E2E_MODEL = {}


def e2e_model(dev):
    """The end-to-end model (random init, seed 0, bf16, HIP decode), built once."""
    import torch

    import _e2e

    if "m" not in _E2E_MODEL:
        spec = _e2e.RuntimeSpec()
        model = _e2e.make_model(spec, dev, torch.bfloat16)
        model.set_decode_attention_backend("hip")
        _E2E_MODEL["m"] = model
    return _E2E_MODEL["m"]


def e2e_trace_line(n_requests: int, dev):
    """One run of the full runtime (HIP prefill and decode, eager) that also
    sums the decode attention's algorithmic KV bytes: every decode row reads
    its context, H*D*2*2 bytes per token and layer. The accounting adds host
    work, so this run is for kernel traces, not for tokens/s."""
    import torch

    import _e2e

    spec = _e2e.RuntimeSpec(n_requests=n_requests, prefill_mode="hip")
    model = e2e_model(dev)
    model.set_prefill_fastpath_mode("hip")
    rt, seqs = _e2e.make_runtime(spec, model, _e2e.make_prompts(spec), dev, torch.bfloat16)
    acc = {"sum_ctx": 0, "calls": 0}
    inner = rt.runner.decode_batch

    def decode_batch(sequences):
        acc["sum_ctx"] += sum(s.length + 1 for s in sequences)
        acc["calls"] += 1
        return inner(sequences)

    rt.runner.decode_batch = decode_batch
    stats = _e2e.run_to_completion(rt, seqs)
    torch.cuda.synchronize()
    head_dim = spec.n_embd // spec.n_head
    stats.update({"decode_steps": acc["calls"], "decode_sum_ctx": acc["sum_ctx"],
                  "decode_attention_calls": acc["calls"] * spec.n_layer,
                  "decode_attention_kv_bytes": acc["sum_ctx"] * spec.n_head * head_dim * 2 * 2 * spec.n_layer})
    return stats


def e2e_line(n_requests: int, dev, graphs: bool, prefill_mode: str = "sdpa_v2",
             record_margins: bool = False):
    """The full runtime under recompute preemption with the HIP decode backend
    and the given prefill mode; with `graphs`, decode steps replay HIP graphs
    captured (before timing) for every batch bucket up to max_running."""
    import torch

    import _e2e

    spec = _e2e.RuntimeSpec(n_requests=n_requests, prefill_mode=prefill_mode)
    prompts = _e2e.make_prompts(spec)
    model = e2e_model(dev)
    model.set_prefill_fastpath_mode(prefill_mode)
    # warm-up: a few requests through prefill + decode
    warm = _e2e.RuntimeSpec(n_requests=4, output_len=4, seed=99)
    rt, seqs = _e2e.make_runtime(warm, model, _e2e.make_prompts(warm), dev, torch.bfloat16)
    _e2e.run_to_completion(rt, seqs)
    del rt, seqs
    rt, seqs = _e2e.make_runtime(spec, model, prompts, dev, torch.bfloat16)
    margins = _e2e.record_margins(rt) if record_margins else None
    if graphs:
        rt.runner.enable_decode_graphs()
        rt.runner.capture_decode_graphs([b for b in (1, 2, 4, 8, 16, 32, 64, 128, 256) if b <= spec.max_running])

    def progress(r):
        if r.iteration % 25 == 0:
            s = r.metrics_summary()
            log(f"e2e step {r.iteration}: output {s['output_tokens']} prefill {s['prefill_tokens']} "
                f"preemptions {s['preemptions']}")

    stats = _e2e.run_to_completion(rt, seqs, on_step=progress)
    stats.update({"requests": n_requests, "pool_blocks": _e2e.pool_blocks(spec, prompts),
                  "sum_prompt_tokens": sum(len(p) for p in prompts),
                  "model": "MiniGPT dim 2048, 16 heads, 12 layers, vocab 32000, bf16, random init (seed 0)",
                  "schedule": "max_running 256, token budget 2048, recompute preemption",
                  "prefill_mode": prefill_mode,
                  "decode_backend": "hip", "decode_graphs": graphs,
                  "tokens": [s.generated_tokens for s in seqs]})
    if margins is not None:
        stats.update({"margins": margins, "prompt_lens": [len(s.prompt_tokens) for s in seqs],
                      "seq_ids": [s.seq_id for s in seqs]})
    return stats


def e2e_lockstep_line(dev, fp32_reference: bool = False):
    """The full runtime (256 requests, dim 2048 x 12 layers, bf16, recompute
    preemption, sdpa_v2 prefill) run to completion twice in lock step, once
    with the PyTorch reference decode backend (or, with ``fp32_reference``,
    online_v1 on float32 copies of q and K/V) and once with the HIP backend,
    checking every iteration as tests/test_e2e_lockstep_gpu.py does
    (schedules, states, block tables, every decode row's logits, every live
    sequence's KV; a token may differ only at a near tie, where the
    reference's token is forced into the HIP runtime). Reports whether every
    check held, the rows checked and the forced ties with their margins."""
    import collections

    import torch

    import _e2e

    spec = _e2e.RuntimeSpec()
    model = e2e_model(dev)
    model.set_prefill_fastpath_mode("sdpa_v2")
    criterion = _e2e.C5_FP32_REF_LOCKSTEP if fp32_reference else _e2e.C5_BF16_LOCKSTEP
    ls = _e2e.Lockstep(spec, model, _e2e.make_prompts(spec), dev, torch.bfloat16,
                       ref_attention=_e2e.online_v1_fp32 if fp32_reference else None, **criterion)
    t0 = time.perf_counter()
    err = None
    try:
        with torch.inference_mode():
            while not ls.finished:
                ls.step()
                if ls.stats["steps"] % 25 == 0:
                    log(f"lock step {ls.stats['steps']}: forced ties {len(ls.forced)} "
                        f"preemptions {ls.stats['preemptions']} ({time.perf_counter() - t0:.0f} s)")
                if ls.stats["steps"] >= 2000:
                    raise AssertionError("the run did not finish in 2000 iterations")
        ls.finish_checks()
    except AssertionError as exc:
        err = str(exc)
    model.set_decode_attention_backend("hip")
    st = ls.stats
    margins = collections.Counter(round(m, 6) for *_, m in ls.forced)
    atol, rtol = criterion["logit_tol"]
    out = {"checks_passed": err is None, "error": err, "iterations": st["steps"],
           "reference": ("online_v1 on float32 copies of q, K, V (output rounded to bf16)" if fp32_reference
                         else "reference decode backend (online_v1 in bf16)"),
           "decode_rows": st["decode_rows"], "decode_rows_checked": st["decode_rows_checked"],
           "kv_token_rows_checked": st["kv_tokens_checked"],
           "forced_ties": len(ls.forced), "streams_with_forced_ties": len(ls.forced_streams),
           "streams_never_forced": f"{len(ls.ref.seqs) - len(ls.forced_streams)}/{len(ls.ref.seqs)}",
           "forced_tie_margins": {str(k): v for k, v in sorted(margins.items())},
           "max_logit_abs": st["max_logit_abs"], "max_logit_fraction_of_bound": round(st["max_logit_ratio"], 3),
           "max_kv_abs": st["max_kv_abs"], "max_kv_fraction_of_bound": round(st["max_kv_ratio"], 3),
           "preemptions": st["preemptions"], "recomputed_sequences": len(st["recomputed_seqs"]),
           "reference_runtime_s": round(ls.wall["reference"], 2), "hip_runtime_s": round(ls.wall["hip"], 2),
           "same_gpu_speedup": round(ls.wall["reference"] / ls.wall["hip"], 2) if ls.wall["hip"] else None,
           "runtime_time_note": "seconds inside each runtime's steps over the same schedule (sdpa_v2 prefill "
                                "in both; device-synchronised per step, checks excluded)",
           "wall_s": round(time.perf_counter() - t0, 1),
           "criterion": f"logits and decode-written KV within {atol:g} + {rtol:g}*max|ref row|; layer-0 and "
                        "prefill-written KV bit-identical; a token may differ only at a reference top-2 "
                        "margin below twice its row's bound, and the reference's token is then forced "
                        "into the HIP runtime so every row stays checked"}
    del ls
    torch.cuda.empty_cache()
    return out


PEAK_BF16_TFLOPS = 2500.0


def prefill_line(dev, start: int, T: int, H: int = 16, D: int = 128, steps: int = 20):
    """Paged prefill attention of one bf16 chunk (T queries after a cached
    prefix of `start` tokens, block size 16, scattered table): the HIP kernel
    against the fp32 gather + SDPA of prefill mode sdpa_v2 on the same GPU.
    The HIP calls are timed after about 50 ms of untimed ones (warm_up).
    FLOPs are the causal algorithmic count 4*H*D*sum_i (start + i + 1)."""
    import types

    import torch

    from minivllm import hip_paged_decode as hpd
    from minivllm.attention import KVCacheCausalSelfAttention
    from minivllm.kv_block_pool import KVBlockPool

    S = 16
    n_blocks = -(-(start + T) // S)
    N = n_blocks + 64
    g = torch.Generator().manual_seed(1)
    table = torch.randperm(N, generator=g)[:n_blocks]
    pool = KVBlockPool(1, N, S, H, D, device=dev, dtype=torch.bfloat16)
    pool.k.normal_()
    pool.v.normal_()
    qkv = torch.randn(1, T, 3, H, D, device=dev).to(torch.bfloat16)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    tdev = table.to(dev)
    warm_up(lambda: hpd.paged_prefill_hip(q[0], pool, tdev, start, 0))
    hip_ms = time_steps(lambda: hpd.paged_prefill_hip(q[0], pool, tdev, start, 0), steps, 3)
    attn = KVCacheCausalSelfAttention(H * D, H, start + T).to(dev)
    seq = types.SimpleNamespace(block_table=table.tolist())
    sdpa_ms = time_steps(lambda: attn._dense_prefill(q, k, v, start, pool, seq, 0), max(3, steps // 4), 1)
    flops = 4 * H * D * (T * start + T * (T + 1) // 2)
    tflops = flops / (hip_ms * 1e-3) / 1e12
    split = hpd._native.lib().mgi_paged_prefill_workspace_bytes(start, T, H, D, hpd._native.DTYPE_CODES[q.dtype]) > 0
    return {"start": start, "T": T, "H": H, "D": D, "key_split": bool(split), "us": round(hip_ms * 1e3, 2),
            "tflops": round(tflops, 1), "pct_of_bf16_mfma_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
            "sdpa_v2_fp32_us": round(sdpa_ms * 1e3, 1), "speedup_vs_sdpa_v2": round(sdpa_ms / hip_ms, 1)}


def decode_step_latency(dev, batches=(1, 4, 16, 64, 256), ctx: int = 512, steps: int = 20):
    """Wall time of one greedy decode step of the end-to-end model (dim 2048,
    16 heads, 12 layers, vocab 32000, bf16, HIP decode) at batch B and context
    `ctx`, through the runtime's own step preparation (staging against the
    device-resident block tables, one host-to-device copy) and including the
    token read-back: eager launches against the replay of the step captured
    for B's bucket at the table width of these contexts."""
    import torch

    import _e2e
    from minivllm.decode_graphs import DecodeGraphs, pack_decode_step, step_metadata
    from minivllm.device_block_tables import DeviceBlockTables
    from minivllm.kv_block_pool import KVBlockPool

    spec = _e2e.RuntimeSpec()
    model = e2e_model(dev)
    S = spec.block_size
    per_seq = -(-(ctx + 1) // S)
    pool = KVBlockPool(spec.n_layer, max(batches) * per_seq, S, spec.n_head, spec.n_embd // spec.n_head,
                       device=dev, dtype=torch.bfloat16)
    pool.k.normal_()
    pool.v.normal_()
    M_graph = -(-model.block_size // S)
    graphs = DecodeGraphs(model, pool, M_graph, buckets=tuple(batches))
    out = {}
    for B in batches:
        tables = [list(range(b * per_seq, (b + 1) * per_seq)) for b in range(B)]
        seq_ids = [f"s{b}" for b in range(B)]
        tokens = [(7 * b + 3) % spec.vocab for b in range(B)]
        positions = [ctx] * B
        slots = [t[ctx // S] * S + ctx % S for t in tables]
        dtab = DeviceBlockTables(dev, cols=M_graph)

        def stage(B_pad):
            rows, upd = dtab.stage(seq_ids, tables)
            step = pack_decode_step(tokens, positions, slots, rows, upd, B_pad).to(dev)
            dtab.apply(step[5 * B_pad:])
            return step

        def eager():
            ids, meta = step_metadata(stage(B), B, dtab, per_seq)
            logits = model.decode_batch(ids, meta, pool)[:, -1, :]
            return torch.argmax(logits, dim=-1).tolist()

        key = graphs.target(B, per_seq)

        def replay():
            return graphs.replay_staged(key, stage(key[0]), B, dtab)[1]

        graphs.capture(*key)
        res = {}
        for name, fn in (("eager", eager), ("graph", replay)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            res[name] = (time.perf_counter() - t0) / steps * 1e3
        out[f"B{B}"] = {"eager_ms": round(res["eager"], 3), "graph_ms": round(res["graph"], 3),
                        "speedup": round(res["eager"] / res["graph"], 2)}
        log(f"decode step latency B={B} ctx={ctx}: {out[f'B{B}']}")
    return {"ctx": ctx, "by_batch": out}


def metadata_prep_line(dev, steps: int = 50):
    """Host-to-device preparation of one decode step's metadata, synchronised:
    every -1 padded table built on the host and copied in the step's one copy
    (pack_decode_metadata) against device-resident tables that receive only
    changed entries (DeviceBlockTables). A sixteenth of the rows gains a block
    every step, as in steady decoding with block size 16."""
    import torch

    from minivllm.decode_graphs import metadata_views, pack_decode_metadata, pack_decode_step, step_metadata
    from minivllm.device_block_tables import DeviceBlockTables

    out = {}
    for B, ctx in ((64, 512), (256, 512), (256, 2048)):
        nb = ctx // 16 + 1
        g = torch.Generator().manual_seed(B + ctx)
        perm = torch.randperm(B * (nb + steps), generator=g).tolist()
        tables = [perm[b * nb:(b + 1) * nb] for b in range(B)]
        spare = iter(perm[B * nb:])
        seq_ids = [f"s{b}" for b in range(B)]
        tokens, positions, slots = list(range(B)), [ctx] * B, [t[-1] * 16 for t in tables]
        dtab = DeviceBlockTables(dev, cols=2 * nb)

        def host_built():
            M = max(len(t) for t in tables)
            return metadata_views(pack_decode_metadata(tokens, positions, slots, tables, B, M).to(dev), B, M)

        def device_resident():
            rows, upd = dtab.stage(seq_ids, tables)
            step = pack_decode_step(tokens, positions, slots, rows, upd, B).to(dev)
            dtab.apply(step[5 * B:])
            return step_metadata(step, B, dtab, max(len(t) for t in tables))

        res = {}
        for name, fn in (("host_built_ms", host_built), ("device_resident_ms", device_resident)):
            fn()  # the first device-resident step uploads every table
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(steps):
                for t in tables[(i % 16) * B // 16:(i % 16 + 1) * B // 16]:
                    t.append(next(spare))
                meta = fn()[1]
                torch.cuda.synchronize()
            res[name] = round((time.perf_counter() - t0) / steps * 1e3, 3)
            M = max(len(t) for t in tables)
            assert meta.block_tables.tolist() == [t + [-1] * (M - len(t)) for t in tables]
        out[f"B{B}_ctx{ctx}"] = res
        log(f"metadata prep B={B} ctx={ctx}: {res}")
    return out


def attention_speedup_grid(dev):
    """HIP decode vs the PyTorch online_v1 backend on the same GPU, over the
    default grid of the reference's fused-decode A/B script
    (experiments/gpu_day6_fused_decode_ab.py:231-242): batches 1,2,4;
    contexts 32,128,256; 8 heads; head_dim 32; block 16; fp32. The reference
    publishes 12.18x-81.68x for its Triton kernel (RTX 5090)."""
    import torch

    import _fixtures as fx
    from minivllm import hip_paged_decode as hpd
    from minivllm.paged_attention_batch import paged_attention_batch_online_v1

    rows = []
    for B in (1, 2, 4):
        for ctx in (32, 128, 256):
            q, pool, tables, lens, layer = fx.build_case(B, ctx, 8, 32, 16, "mixed")
            dpool = fx.pool_to_device(pool, dev)
            qd, td, ld = q.to(dev), tables.to(dev), lens.to(dev)
            ref_ms = time_steps(lambda: paged_attention_batch_online_v1(qd, dpool, td, ld, layer), 20, 3)
            hip_ms = time_steps(lambda: hpd.paged_attention_batch_hip(qd, dpool, td, ld, layer), 50, 5)
            rows.append({"batch": B, "ctx": ctx, "online_v1_ms": round(ref_ms, 4), "hip_ms": round(hip_ms, 4),
                         "speedup": round(ref_ms / hip_ms, 1)})
    sp = [r["speedup"] for r in rows]
    return {"min_speedup": min(sp), "max_speedup": max(sp), "grid": rows}


def e2e_c1_ab(dev, warmups: int = 2, repeats: int = 7):
    """Mini-GPT end to end (dim 256, 8 heads, 4 layers, vocab 256, fp32,
    seed 0; block 16; token budget 64; sdpa_v2 prefill; 8 greedy tokens),
    HIP decode backend against the PyTorch reference backend on the same GPU,
    timed as experiments/gpu_day6_runtime_decode_ab.py:146-185 times its two
    backends: one model built before any timing; per case `warmups` + `repeats`
    rounds, the backend order alternating round by round; each run's runtime
    (pool, block manager, scheduler, requests) is built before its clock
    starts and the clock covers the whole step loop, with device
    synchronisations at both ends. Every run's tokens and lifecycle counts
    must equal the first run's. Per backend: median wall ms and median
    output tokens/s (generated tokens / wall seconds, output_tok_s of
    experiments/gpu_e2e_runtime.py:198) over the timed repeats; the speedup
    is the ratio of the median walls. Cases: the four golden cases (batch
    1/4 x prompt 128/256, "conservative", the whole run's blocks) and the two
    batch-4 cases forced into recompute preemption (pool factor 0.5: one
    preemption, 16 replayed KV tokens). The reference publishes 3.80x-6.34x
    (no preemption) and 4.31x-5.44x (forced preemption) for its Triton
    backend on an RTX 5090."""
    import statistics

    import torch

    import _e2e

    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    model = _e2e.make_c1_model(dev)
    runs = [(c, "conservative", 1.0) for c in _e2e.GOLDEN_C1["cases"]]
    runs += [(c, "recompute", 0.5) for c in _e2e.GOLDEN_C1["cases"] if c["batch"] == 4]
    rows = []
    for case, policy, factor in runs:
        first = None
        wall = {"reference": [], "hip": []}
        for rep in range(warmups + repeats):
            for backend in (("reference", "hip") if rep % 2 == 0 else ("hip", "reference")):
                model.set_decode_attention_backend(backend)
                rt, seqs = _e2e.make_c1_runtime(model, case, dev, policy, factor)
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                _e2e.step_c1(rt, seqs, check=False)
                torch.cuda.synchronize()
                dt = time.perf_counter() - t0
                m = rt.metrics_summary()
                got = ([s.generated_tokens for s in seqs],
                       (rt.iteration, m["output_tokens"], m["preemptions"], m["repeated_kv_tokens"],
                        m["prefill_tokens"], m["decode_tokens"]))
                if first is None:
                    first = got
                if got != first:
                    raise AssertionError(f"C1 B={case['batch']} P={case['prompt_len']} {policy}: {backend} "
                                         "tokens or lifecycle counts differ between runs")
                if rep >= warmups:
                    wall[backend].append(dt)
        out_tokens = first[1][1]
        row = {"batch": case["batch"], "prompt_len": case["prompt_len"], "policy": policy, "kv_factor": factor,
               "iterations": first[1][0], "preemptions": first[1][2], "repeated_kv_tokens": first[1][3],
               "tokens_match_golden": first[0] == case["outputs"]}
        for backend, ts in wall.items():
            med = statistics.median(ts)
            row[backend] = {"wall_ms_median": round(med * 1e3, 3),
                            "output_tok_s_median": round(statistics.median(out_tokens / t for t in ts), 1)}
        row["e2e_speedup"] = round(row["reference"]["wall_ms_median"] / row["hip"]["wall_ms_median"], 2)
        rows.append(row)
        log(f"C1 A/B B={case['batch']} P={case['prompt_len']} {policy}: {row}")
    plain = [r["e2e_speedup"] for r in rows if r["policy"] == "conservative"]
    forced = [r["e2e_speedup"] for r in rows if r["policy"] == "recompute"]
    return {"method": f"{warmups} warm-ups + {repeats} alternating repeats per backend, model built once, "
                      "runtime built outside each run's clock",
            "speedup_no_preemption": [min(plain), max(plain)], "speedup_forced_preemption": [min(forced), max(forced)],
            "cases": rows}


def cpu_threads() -> tuple[int, int]:
    """Threads of the CPU baseline: every core of this process's affinity set,
    capped by OMP_NUM_THREADS when the environment sets it (the host's share
    of cores for its one GPU on a shared machine). Returns (threads used,
    affinity cores)."""
    aff = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS") or 0)
    return (min(aff, share) if share > 0 else aff), aff


def _seconds(fn, warmup: int, repeats: int) -> float:
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(w, dev) -> dict:
    """The decode path on this host's cores, beside the GPU figures. The main
    figure is the C restatement of paged_attention_batch_online_v1
    (oracle/paged_decode_oracle.c, fp32 accumulation) on the decode workload;
    `rows` add the package's PyTorch online_v1 (the "reference" decode
    backend, the reference's own CPU path) on the same input as-is in bf16
    and upcast to fp32, the KV append plus decode step at B=256, the long
    contexts (one repeat), the small end-to-end model and a window of the
    full runtime. Every row names its sample, threads and repeats."""
    import torch

    import _e2e
    import _fixtures as fx
    from minivllm.paged_attention_batch import paged_attention_batch_online_v1
    from oracle import c_oracle

    threads, aff = cpu_threads()
    torch.set_num_threads(threads)
    host = {"cores": threads, "affinity_cores": aff, "cpu": _cpu_model()}
    rows = {}

    def port_row(wl, repeats, name, desc):
        args = wl.compact_host()
        sec = _seconds(lambda: c_oracle.paged_decode(*args, acc_double=False, threads=threads),
                       1 if repeats > 1 else 0, repeats)
        rows[name] = {"value": round(wl.algorithmic_bytes() / sec / 1e9, 3), "unit": "GB/s",
                      "ms": round(sec * 1e3, 2), "kind": "port", **host,
                      "sample": f"{desc} through oracle/paged_decode_oracle.c (fp32 accumulation); "
                                f"median of {repeats}" + (" after 1 warmup" if repeats > 1 else "")}
        log(f"cpu {name}: {rows[name]}")

    port_row(w, 3, "decode_port", f"the decode workload (B={w.q.shape[0]}, sum ctx={int(w.ctx.sum())}, "
                                   f"{w.meta['dtype']})")

    cw = w.compact_cpu()
    with torch.inference_mode():
        for name, dt in (("decode_online_v1_torch", None), ("decode_online_v1_torch_fp32_upcast", torch.float32)):
            q, pool = cw.q, cw.pool
            if dt is not None:
                q = q.to(dt)
                from minivllm.kv_block_pool import KVBlockPool
                pool = KVBlockPool(1, cw.pool.num_blocks, cw.pool.block_size, cw.pool.n_head, cw.pool.head_dim,
                                   dtype=dt)
                pool.k.copy_(cw.pool.k)
                pool.v.copy_(cw.pool.v)
            sec = _seconds(lambda: paged_attention_batch_online_v1(q, pool, cw.tables, cw.ctx, 0), 1, 3)
            nbytes = fx.DecodeWorkload(q, pool, cw.tables, cw.ctx, 0, {}).algorithmic_bytes()
            rows[name] = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "ms": round(sec * 1e3, 1),
                          "kind": "port", **host,
                          "sample": "the same decode workload through minivllm.paged_attention_batch."
                                    "paged_attention_batch_online_v1 on CPU tensors (the reference's per-"
                                    "block gather/mask/online loop, torch ops in "
                                    f"{str(q.dtype).replace('torch.', '')}); median of 3 after 1 warmup"}
            log(f"cpu {name}: {rows[name]}")
            del q, pool
    del cw

    # KV append + decode at B=256, ctx U[128, 2048]: torch index_put_ of the
    # 10%-padded rows, then the C restatement over the appended contexts.
    w3 = fx.make_decode_workload(256, 32, 128, 16, 32768, 128, 2048, torch.bfloat16, dev, seed=0, poison=False)
    c3 = w3.compact_cpu()
    g = torch.Generator().manual_seed(0)
    pad = torch.zeros(256, dtype=torch.bool)
    pad[torch.randperm(256, generator=g)[:25]] = True
    last = c3.ctx - 1
    slots = c3.tables[torch.arange(256), last // 16] * 16 + last % 16
    slots = torch.where(pad, torch.full_like(slots, -1), slots)
    k_new = torch.randn(256, 32, 128, generator=g).to(torch.bfloat16)
    v_new = torch.randn(256, 32, 128, generator=g).to(torch.bfloat16)
    args = c3.compact_host()

    def c3_step():
        keep = slots >= 0
        s = slots[keep]
        c3.pool.k[0, s // 16, s % 16] = k_new[keep]
        c3.pool.v[0, s // 16, s % 16] = v_new[keep]
        c_oracle.paged_decode(*args, acc_double=False, threads=threads)

    sec = _seconds(c3_step, 1, 3)
    nbytes = w3.algorithmic_bytes() + int((~pad).sum()) * 32 * 128 * 2 * 2 * 2
    rows["append_plus_decode_B256"] = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s",
                                       "ms": round(sec * 1e3, 2), "kind": "port", **host,
                                       "sample": "KV append (torch index_put_ of 231 rows, 25 padding rows "
                                                 "skipped) then decode over B=256 ctx U[128,2048] bf16 through "
                                                 "oracle/paged_decode_oracle.c; median of 3 after 1 warmup"}
    log(f"cpu append_plus_decode_B256: {rows['append_plus_decode_B256']}")
    del w3, c3, args
    torch.cuda.empty_cache()

    w4 = fx.make_decode_workload(8, 32, 128, 16, 65536, 32768, 131072, torch.bfloat16, dev, seed=0, poison=False)
    port_row(w4, 1, "longctx_port", "the long-context workload (B=8, ctx U[32768,131072], bf16), one repeat,")
    del w4
    torch.cuda.empty_cache()

    # The small end-to-end model on the CPU with the reference decode backend.
    t_all, toks = 0.0, 0
    for case in _e2e.GOLDEN_C1["cases"]:
        t0 = time.perf_counter()
        tokens, _ = _e2e.run_c1(case, "cpu", "reference")
        t_all += time.perf_counter() - t0
        toks += sum(len(t) for t in tokens)
    rows["e2e_small_model"] = {"value": round(toks / t_all, 1), "unit": "generated tokens/s",
                               "s": round(t_all, 3), "kind": "port", **host,
                               "sample": "the Mini-GPT end-to-end runs (dim 256, 4 layers, fp32; prompts "
                                         "128/256 x batch 1/4; budget 64; 8 greedy tokens), all four cases "
                                         "once, reference decode backend, sdpa_v2 prefill, on the CPU"}
    log(f"cpu e2e_small_model: {rows['e2e_small_model']}")

    # A labelled window of the full runtime: its first iterations (prefill
    # dominated), as the runtime runs them, on the CPU.
    spec = _e2e.RuntimeSpec()
    model = _e2e.make_model(spec, "cpu", torch.bfloat16)
    model.set_decode_attention_backend("reference")
    rt, seqs = _e2e.make_runtime(spec, model, _e2e.make_prompts(spec), "cpu", torch.bfloat16)
    n_iter = 3
    t0 = time.perf_counter()
    with torch.inference_mode():
        for _ in range(n_iter):
            rt.step()
    sec = time.perf_counter() - t0
    summ = rt.metrics_summary()
    rows["full_runtime_window"] = {"value": round(summ["scheduled_tokens"] / sec, 1),
                                   "unit": "scheduled tokens/s", "s": round(sec, 2), "kind": "port", **host,
                                   "iterations": n_iter, "prefill_tokens": summ["prefill_tokens"],
                                   "decode_tokens": summ["decode_tokens"],
                                   "sample": f"iterations 1-{n_iter} of the full runtime (dim 2048 x 12 layers, "
                                             "vocab 32000, bf16, 256 requests; prefill dominated) on the CPU, "
                                             "reference decode backend, sdpa_v2 prefill; a window, not the "
                                             "whole run"}
    log(f"cpu full_runtime_window: {rows['full_runtime_window']}")
    del rt, seqs, model

    main = rows["decode_port"]
    return {"value": main["value"], "unit": "GB/s", "cores": threads, "kind": "port", "sample": main["sample"],
            "ms": main["ms"], "affinity_cores": aff, "cpu": host["cpu"], "rows": rows}


def cpu_prefill_baseline(start: int = 0, T: int = 512, H: int = 16, D: int = 128, S: int = 16):
    """The prefill oracle (numpy, float32 arithmetic, host BLAS threads) on one
    chunk of the prefill workload: the CPU restatement of the reference's
    per-token prefill loop, timed beside the kernel's TFLOP/s."""
    import numpy as np

    from oracle import paged_decode as ora

    rng = np.random.default_rng(1)
    nb = -(-(start + T) // S)
    k = rng.standard_normal((1, nb, S, H, D), dtype=np.float32)
    v = rng.standard_normal((1, nb, S, H, D), dtype=np.float32)
    q = rng.standard_normal((T, H, D), dtype=np.float32)
    table = rng.permutation(nb)
    times = []
    for i in range(3):  # 1 warmup + 2 timed
        t0 = time.perf_counter()
        ora.paged_prefill(q, k, v, table, start, 0, acc=np.float32)
        if i:
            times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    flops = 4 * H * D * (T * start + T * (T + 1) // 2)
    threads, _ = cpu_threads()
    return {"value": round(flops / sec / 1e12, 4), "unit": "TFLOP/s", "ms": round(sec * 1e3, 2),
            "cores": threads, "kind": "port", "cpu": _cpu_model(),
            "sample": f"one prefill chunk (start {start}, T {T}, H {H}, D {D}) through "
                      "oracle.paged_decode.paged_prefill in float32; median of 2 after 1 warmup"}


def profiled_traffic(workload: str, split: dict):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    counter summary (FETCH_SIZE and WRITE_SIZE, each scaled by a copy kernel of
    known size), when profiles/ holds one for this workload and split."""
    for md in sorted((ROOT / "profiles").glob("*.md")):
        for block in re.findall(r"```json\n(.*?)```", md.read_text(), flags=re.S):
            try:
                d = json.loads(block)
            except json.JSONDecodeError:
                continue
            if d.get("workload") == workload and d.get("split") == split:
                kib = d["fetch_kib_per_dispatch"] * d["fetch_scale"] + d["write_kib_per_dispatch"] * d["write_scale"]
                return int(kib * 1024), md.name
    return None, None


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> None:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the paged decode path runs "
              "on a single MI355X. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    import _fixtures as fx

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.e2e_trace:
        with torch.inference_mode():
            print(json.dumps(e2e_trace_line(args.e2e_requests, dev)), flush=True)
        return
    dtype = torch.bfloat16 if args.dtype == "bf16" else torch.float32
    B, N, ctx_lo, ctx_hi, wl_desc = WORKLOADS[args.workload]
    H, D, S = 32, 128, 16

    with torch.inference_mode():
        log(f"building decode workload B={B} H={H} D={D} S={S} N={N} ctx U[{ctx_lo},{ctx_hi}] {args.dtype}")
        w = fx.make_decode_workload(B, H, D, S, N, ctx_lo, ctx_hi, dtype, dev, seed=0, poison=False)
        from minivllm import _native

        M = w.tables.shape[1]
        bal = int(_native.lib().mgi_paged_decode_balanced_waves(B, H, D, S, M, args.split_tokens))
        if bal:
            split = {"mode": "balanced", "waves": bal * -(-H // 4)}  # 4 heads per wavefront at D=128
        else:
            split = {"mode": "partition",
                     "split_tokens": int(_native.lib().mgi_paged_decode_split_tokens(B, H, D, S, M,
                                                                                     args.split_tokens))}
        log("timing decode")
        main_line = decode_line(w, args.steps, args.warmup, args.split_tokens)
        log(f"decode: {main_line}")

        extras = {}
        if not args.no_extras:
            other = torch.float32 if dtype == torch.bfloat16 else torch.bfloat16
            tag = "fp32" if other == torch.float32 else "bf16"
            w2 = fx.make_decode_workload(64, H, D, S, 20000, 512, 4096, other, dev, seed=0, poison=False)
            extras[f"decode_{tag}"] = decode_line(w2, max(5, args.steps // 2), 3, args.split_tokens)
            del w2
            log(f"extra decode_{tag}: {extras[f'decode_{tag}']}")
            w3 = fx.make_decode_workload(64, H, D, S, 20000, 4096, 4096, dtype, dev, seed=0,
                                         fixed_ctx=4096, poison=False)
            extras[f"decode_{args.dtype}_ctx4096"] = decode_line(w3, max(5, args.steps // 2), 3,
                                                                  args.split_tokens)
            del w3
            log(f"extra ctx4096: {extras[f'decode_{args.dtype}_ctx4096']}")
            w4 = fx.make_decode_workload(8, H, D, S, 65536, 32768, 131072, torch.bfloat16, dev, seed=0,
                                         poison=False)
            extras["longctx_bf16_B8_ctx32k-128k"] = decode_line(w4, max(5, args.steps // 5), 2, 0)
            del w4
            log(f"extra longctx: {extras['longctx_bf16_B8_ctx32k-128k']}")
            w5 = fx.make_decode_workload(256, H, D, S, 32768, 128, 2048, torch.bfloat16, dev, seed=0,
                                         poison=False)
            extras["decode_bf16_B256_ctx128-2048"] = decode_line(w5, max(5, args.steps // 2), 3, 0)
            del w5
            log(f"extra B256: {extras['decode_bf16_B256_ctx128-2048']}")
            # One GPU's share of an 8-way head split (tensor parallel): the same
            # batches and contexts with 32 / 8 = 4 heads.
            w6 = fx.make_decode_workload(64, 4, D, S, 20000, 512, 4096, torch.bfloat16, dev, seed=0, poison=False)
            extras["tp8_shard_decode_bf16_H4_ctx512-4096"] = decode_line(w6, max(10, args.steps), 5, 0)
            del w6
            log(f"extra tp8 shard: {extras['tp8_shard_decode_bf16_H4_ctx512-4096']}")
            w7 = fx.make_decode_workload(8, 4, D, S, 65536, 32768, 131072, torch.bfloat16, dev, seed=0,
                                         poison=False)
            extras["tp8_shard_longctx_bf16_B8_H4_ctx32k-128k"] = decode_line(w7, max(10, args.steps // 2), 3, 0)
            del w7
            log(f"extra tp8 shard long: {extras['tp8_shard_longctx_bf16_B8_H4_ctx32k-128k']}")
            extras["kv_append_bf16_B256"] = append_line(max(20, args.steps), 5, dev)
            log(f"extra append: {extras['kv_append_bf16_B256']}")
            extras["append_plus_decode_bf16_B256_ctx128-2048"] = c3_step_line(max(10, args.steps // 2), 3, dev)
            log(f"extra append+decode: {extras['append_plus_decode_bf16_B256_ctx128-2048']}")
            extras["d2d_copy_4GiB"] = copy_line(4096, dev, reps=5)
            log(f"extra copy: {extras['d2d_copy_4GiB']}")
            torch.cuda.empty_cache()
            extras["attention_speedup_vs_online_v1"] = attention_speedup_grid(dev)
            log(f"extra attention speedup: {extras['attention_speedup_vs_online_v1']['min_speedup']}x-"
                f"{extras['attention_speedup_vs_online_v1']['max_speedup']}x")
            extras["e2e_small_model_ab"] = e2e_c1_ab(dev)
            log(f"extra small-model A/B: no preemption {extras['e2e_small_model_ab']['speedup_no_preemption']}, "
                f"forced preemption {extras['e2e_small_model_ab']['speedup_forced_preemption']}")
            torch.cuda.empty_cache()

        if not args.no_extras or not args.no_e2e or args.prefill:
            for start, T in ((0, 512), (2048, 2048), (4096, 256)):
                key = f"prefill_bf16_start{start}_T{T}_H16_D128"
                extras[key] = prefill_line(dev, start, T)
                log(f"extra {key}: {extras[key]}")
            if not args.no_extras:
                # The same 2048 rows after a long prefix: every query tile's
                # chain is nearly as long, so this shows the kernel's steady
                # state without the causal imbalance of the chunk above.
                key = "prefill_bf16_start16384_T2048_H16_D128"
                extras[key] = prefill_line(dev, 16384, 2048)
                log(f"extra {key}: {extras[key]}")
            torch.cuda.empty_cache()

        e2e_summary = None
        if not args.no_e2e:
            runs = (("e2e_runtime_bf16_preemption", False, "sdpa_v2"),
                    ("e2e_runtime_bf16_preemption_hip_prefill", False, "hip"),
                    ("e2e_runtime_bf16_preemption_hip_prefill_graphs", True, "hip"))
            for key, graphs, mode in runs:
                log(f"end-to-end runtime, {args.e2e_requests} requests, prefill {mode}, decode graphs {graphs}")
                extras[key] = e2e_line(args.e2e_requests, dev, graphs, mode)
                torch.cuda.empty_cache()
            log("e2e: untimed replay of the first configuration recording top-2 logit margins")
            margins_run = e2e_line(args.e2e_requests, dev, False, "sdpa_v2", record_margins=True)
            base = extras[runs[0][0]]["tokens"]
            extras[runs[0][0]]["deterministic_rerun"] = margins_run["tokens"] == base
            for key, _, _ in runs[1:]:
                other = extras[key]["tokens"]
                same = sum(a == b for a, b in zip(base, other))
                margin_at = []
                for a, b, plen, sid in zip(base, other, margins_run["prompt_lens"], margins_run["seq_ids"]):
                    if a != b:
                        k = next(i for i, (x, y) in enumerate(zip(a, b)) if x != y)
                        margin_at.append(margins_run["margins"].get((sid, plen + k - 1)))
                known = [m for m in margin_at if m is not None]
                extras[key]["identical_token_streams_vs_first"] = f"{same}/{args.e2e_requests}"
                extras[key]["first_divergence_margin_max"] = round(max(known), 4) if known else None
                extras[key]["first_divergences_at_exact_bf16_tie"] = sum(m == 0.0 for m in known)
            for key, _, _ in runs:
                extras[key].pop("tokens")
                log(f"e2e {key}: {extras[key]}")
            extras["decode_step_latency_eager_vs_graph"] = decode_step_latency(dev)
            extras["decode_metadata_prep"] = metadata_prep_line(dev)
            if not args.no_lockstep and args.e2e_requests == 256:
                log("e2e: full runtime in lock step, reference decode backend vs HIP (about 3 minutes)")
                extras["e2e_lockstep_vs_reference_backend"] = e2e_lockstep_line(dev)
                log(f"e2e lock step: {extras['e2e_lockstep_vs_reference_backend']}")
                if args.lockstep_fp32:
                    log("e2e: lock step against the fp32-accumulating reference (about 3 minutes)")
                    extras["e2e_lockstep_vs_fp32_accumulating_reference"] = e2e_lockstep_line(dev, True)
                    log(f"e2e lock step fp32: {extras['e2e_lockstep_vs_fp32_accumulating_reference']}")
            hip = extras["e2e_runtime_bf16_preemption_hip_prefill"]
            hip_g = extras["e2e_runtime_bf16_preemption_hip_prefill_graphs"]
            e2e_summary = {"decode_tokens_per_s": hip["output_tok_s"],
                           "decode_tokens_per_s_with_graphs": hip_g["output_tok_s"],
                           "decode_tokens_per_s_definition":
                               "generated tokens / wall seconds of the whole run, prefill included "
                               "(output_tok_s of experiments/gpu_e2e_runtime.py:198)",
                           "decode_phase_tokens_per_s": hip["decode_tok_s_in_decode_phase"],
                           "decode_phase_tokens_per_s_with_graphs": hip_g["decode_tok_s_in_decode_phase"],
                           "decode_phase_tokens_per_s_definition":
                               "decode tokens / seconds spent inside decode steps only",
                           "workload": "full runtime, 256 requests, MiniGPT dim 2048 x 12 layers, bf16, "
                                       "HIP decode + HIP prefill, recompute preemption (eager; "
                                       "'with_graphs': decode steps of <= 128 rows replay HIP graphs)"}
            _E2E_MODEL.clear()
            torch.cuda.empty_cache()

        if args.calibrate_copy_mib:
            extras["copy_calibration"] = copy_line(args.calibrate_copy_mib, dev, reps=3)
            log(f"copy calibration: {extras['copy_calibration']}")

        cpu = None
        if not args.no_cpu_baseline:
            log("timing CPU baseline")
            cpu = cpu_baseline(w, dev)
            cpu["rows"]["prefill_chunk"] = cpu_prefill_baseline()
            log(f"cpu: {cpu}")

    workload_tag = f"decode_{args.workload}_{args.dtype}_B{B}_H{H}_D{D}_ctx{ctx_lo}-{ctx_hi}"
    traffic, traffic_src = profiled_traffic(workload_tag, split)
    result = {
        "metric": METRIC,
        "value": main_line["gbps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_line["ms"],
        "ms_per_step_mean": main_line["mean_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic: seeded N(0,1) q/K/V, contexts and a random block permutation (seed 0)",
        "config": {"workload": wl_desc,
                   "batch": B, "heads": H, "head_dim": D, "block_size": S, "pool_blocks": N,
                   "ctx": f"U[{ctx_lo},{ctx_hi}]", "sum_ctx": main_line["sum_ctx"], "split": split},
        "pct_of_peak": main_line["pct_of_peak"],
        "decode_seq_per_s_per_layer": main_line["seq_per_s_per_layer"],
        "end_to_end": e2e_summary,
        "roofline": {"bound": "hbm", "achieved": main_line["gbps"], "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": round(main_line["gbps"] / PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_src,
                     "alg_bytes_per_launch": main_line["alg_bytes"],
                     "kernel": ("paged_decode_fast_bal" if split["mode"] == "balanced" else "paged_decode_fast")
                               + " + paged_decode_merge (one mgi_paged_decode call)"},
        "cpu_baseline": cpu,
        "extra": extras,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
