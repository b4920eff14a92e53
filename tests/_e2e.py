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


def make_c1_model(device, prefill_mode: str | None = None) -> MiniGPT:
    """The golden configuration's Mini-GPT (seed 0, fp32); prefill_mode
    overrides the recorded configuration's prefill mode."""
    cfg = GOLDEN_C1["config"]
    torch.manual_seed(cfg["seed"])
    model = MiniGPT(n_embd=cfg["n_embd"], n_head=cfg["n_head"], vocab_size=cfg["vocab_size"],
                    block_size=cfg["block_size"], dropout=0.0, n_layer=cfg["n_layer"]).eval().to(device)
    model.set_prefill_fastpath_mode(prefill_mode or cfg["prefill_mode"])
    return model


def c1_pool_blocks(case: dict, kv_factor: float = 1.0) -> int:
    """Pool size of a golden case: every request's whole run
    (B * ceil((P + out - 1) / S) blocks) times kv_factor, at least one
    request's, as experiments/gpu_e2e_runtime.py:96-103 sizes it."""
    cfg = GOLDEN_C1["config"]
    per = math.ceil((case["prompt_len"] + cfg["output_len"] - 1) / cfg["block_size_kv"])
    return max(per, math.ceil(case["batch"] * per * kv_factor))


def make_c1_runtime(model: MiniGPT, case: dict, device, policy: str = "conservative", kv_factor: float = 1.0):
    """A runtime over one golden case's requests on a NaN-filled pool of
    c1_pool_blocks(case, kv_factor) blocks; returns (runtime, sequences)."""
    cfg = GOLDEN_C1["config"]
    B, P, S = case["batch"], case["prompt_len"], cfg["block_size_kv"]
    blocks = c1_pool_blocks(case, kv_factor)
    manager = BlockManager(num_blocks=blocks, block_size=S)
    rt = MiniRuntime.__new__(MiniRuntime)
    rt.block_manager = manager
    rt.scheduler = Scheduler(manager, max_running=B, max_num_batched_tokens=cfg["token_budget"],
                             preemption_policy=policy)
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
    return rt, seqs


def step_c1(rt: MiniRuntime, seqs, check: bool = True) -> None:
    """Steps a golden-case runtime to completion (block-manager invariants
    after every step unless ``check`` is off)."""
    with torch.inference_mode():
        for _ in range(1000):
            if all(s.status == Status.FINISHED for s in seqs):
                break
            rt.step()
            if check:
                rt.block_manager.check_invariants([s for s in seqs if s.status != Status.FINISHED])
    assert all(s.status == Status.FINISHED for s in seqs)


def run_c1(case: dict, device, backend: str, prefill_mode: str | None = None, policy: str = "conservative",
           kv_factor: float = 1.0):
    """Runs one golden case; returns (generated tokens per request, runtime).

    prefill_mode overrides the recorded configuration's prefill mode (the
    golden tokens were produced with it); policy and kv_factor size the pool
    and choose the preemption policy (the golden run: "conservative", 1.0)."""
    model = make_c1_model(device, prefill_mode)
    model.set_decode_attention_backend(backend)
    if kv_factor == 1.0:
        assert c1_pool_blocks(case) == case["num_blocks"]
    rt, seqs = make_c1_runtime(model, case, device, policy, kv_factor)
    step_c1(rt, seqs)
    return [s.generated_tokens for s in seqs], rt


# ------------------------------------------------------ lock-step comparison

class _Probe:
    """Wraps one runtime so each step records its schedule, its decode logits
    and, per sequence, the end of the KV its current prefill wrote."""

    def __init__(self, rt: MiniRuntime, seqs):
        self.rt, self.seqs = rt, seqs
        self.by_id = {s.seq_id: s for s in seqs}
        self.plan = None
        self.logits = None
        self.decoded: list[str] = []
        self.prefill_end: dict[str, int] = {}
        schedule, decode, prefill = rt.scheduler.schedule, rt.runner.decode_batch, rt.runner.prefill_chunk

        def schedule_probe():
            out = schedule()
            self.plan = ([(i.seq.seq_id, i.start_pos, i.num_tokens) for i in out.prefill],
                         [s.seq_id for s in out.decode])
            return out

        def decode_probe(sequences):
            logits, tokens = decode(sequences)
            self.logits = logits.float()
            self.decoded = [s.seq_id for s in sequences]
            return logits, tokens

        def prefill_probe(seq, start_pos, num_tokens):
            out = prefill(seq=seq, start_pos=start_pos, num_tokens=num_tokens)
            # Chunks of one incarnation are contiguous from position 0.
            self.prefill_end[seq.seq_id] = start_pos + num_tokens
            return out

        rt.scheduler.schedule = schedule_probe
        rt.runner.decode_batch = decode_probe
        rt.runner.prefill_chunk = prefill_probe

    def step(self) -> None:
        self.plan, self.logits, self.decoded = None, None, []
        self.rt.step()


def _token_slots(seq: SequenceState, S: int) -> list[int]:
    t = seq.block_table
    return [t[p // S] * S + p % S for p in range(seq.length)]


# Lock-step criteria of the full configuration in bf16 (see Lockstep and
# test_e2e_lockstep_gpu.py), scaled by each row's largest magnitude:
# |hip - ref| <= atol + rtol * max|ref row| on logits and on decode-written KV;
# a token may differ only where the reference's top-2 margin is below twice
# its row's logit bound, and the reference's token is then forced into the
# HIP runtime.
#   * against the reference backend as it runs in bf16 (online_v1 keeps its
#     running max, sum and output in bf16, rounded at every block): 2^-6 +
#     2^-6 * max|row|, four bf16 ulps of the row's largest entry plus 2^-6;
#   * against online_v1 run on float32 copies of q, K and V, its output
#     rounded to bf16 (the HIP kernel's own arithmetic: fp32 accumulation of
#     bf16 data): the two differ by the order of fp32 sums and by the
#     exponential's last bits, which flip the bf16 rounding of an attention
#     output now and then; every later bf16 rounding (GEMM outputs, residual
#     stream, logits) then moves by whole ulps, so a logit differs by at
#     least one ulp of its own size once anything upstream differs. The
#     bound is three quarters of the bf16 one: 0.75 * 2^-6 (1 + max|row|).
C5_BF16_LOCKSTEP = dict(logit_tol=(2.0 ** -6, 2.0 ** -6), tie_margin=None, kv_tol=(2.0 ** -6, 2.0 ** -6),
                        row_scaled=True)
_FP32_REF_TOL = 0.75 * 2.0 ** -6
C5_FP32_REF_LOCKSTEP = dict(logit_tol=(_FP32_REF_TOL, _FP32_REF_TOL), tie_margin=None,
                            kv_tol=(_FP32_REF_TOL, _FP32_REF_TOL), row_scaled=True)


class _Upcast:
    """Indexing returns a float32 copy of the indexed part of a pool tensor."""

    def __init__(self, t: torch.Tensor):
        self.t = t

    def __getitem__(self, idx):
        return self.t[idx].float()


class _Float32Pool:
    """The k / v / block_size view of a KVBlockPool that paged_attention_batch_online_v1
    reads, with every gathered block converted to float32."""

    def __init__(self, pool: KVBlockPool):
        self.k, self.v, self.block_size = _Upcast(pool.k), _Upcast(pool.v), pool.block_size


def online_v1_fp32(q, pool, block_tables, context_lengths, layer_idx):
    """The package's online_v1 on float32 copies of q and of each gathered
    K/V block (fp32 accumulation of the stored bf16 values); the output is
    rounded back to q's dtype."""
    from minivllm.paged_attention_batch import paged_attention_batch_online_v1

    out = paged_attention_batch_online_v1(q=q.float(), pool=_Float32Pool(pool), block_tables=block_tables,
                                          context_lengths=context_lengths, layer_idx=layer_idx)
    return out.to(q.dtype)


class Lockstep:
    """The reference runtime and the HIP runtime stepped alternately over one
    model, one request set and two KV pools of the same size, as
    experiments/gpu_day6_runtime_decode_ab.py:59-130 steps its two backends.
    Prefill uses the model's prefill mode in both, so the only difference
    between the runs is the decode attention backend ("reference" = the
    PyTorch online-softmax path, or ``ref_attention`` in its place when
    given; "hip" = kv_append + the HIP decode kernel).

    ``step()`` advances both runtimes by one iteration and checks:
      * identical schedules (prefill chunks, decode batch order), sequence
        states (status, length, prompt position, block table) and lifecycle
        counts;
      * decode logits of every row within ``logit_tol`` = (atol, rtol):
        |hip - ref| <= atol + rtol * |ref| elementwise, or, with
        ``row_scaled``, atol + rtol * max|ref row| (rounding of the hidden
        state moves every logit of a row in proportion to the row's scale,
        not to the logit's own size);
      * greedy tokens identical, except where the reference's top-2 logit
        margin is below ``tie_margin`` (None: twice that row's logit bound,
        the largest gap two logits each moved by the bound can close). There
        the reference's token is written into the HIP runtime's sequence
        (its last generated token and its next decode input) and the event is
        recorded in ``forced``, so both runtimes keep decoding the same
        tokens and every later row stays in the logit and KV checks;
      * logical KV of every active sequence read through its block table:
        bit-identical in layer 0 (its input is the token and position
        embedding alone) and at every position the current prefill wrote
        (prefill is shared and deterministic), within ``kv_tol`` at
        positions decode wrote in later layers (the decode attention outputs
        differ in rounding; ``row_scaled`` scales by each token's [H, D] row
        in that layer). ``kv_tol=None`` checks through
        KVBlockPool.gather_sequence on the host instead, with ``kv_tol``
        replaced by ``logit_tol`` elementwise, as the reference harness does.

    Statistics of every check accumulate in ``stats``.
    """

    def __init__(self, spec: RuntimeSpec, model: MiniGPT, prompts, device, dtype, *,
                 logit_tol: tuple[float, float], tie_margin: float | None, kv_tol: tuple[float, float] | None,
                 row_scaled: bool = False, ref_attention=None):
        self.model = model
        self.logit_tol, self.tie_margin, self.kv_tol = logit_tol, tie_margin, kv_tol
        self.row_scaled = row_scaled
        self.ref_attention = ref_attention
        self.ref = _Probe(*make_runtime(spec, model, prompts, device, dtype))
        self.hip = _Probe(*make_runtime(spec, model, prompts, device, dtype))
        self.forced: list[tuple[int, str, int, float]] = []   # (step, seq_id, token index, ref margin)
        # Seconds inside each runtime's steps (device-synchronised at both
        # ends of every step; the checks between steps are not counted).
        self.wall = {"reference": 0.0, "hip": 0.0}
        # max_*_ratio: the largest deviation as a fraction of its bound (<= 1 passes).
        self.stats = {"steps": 0, "decode_rows": 0, "decode_rows_checked": 0, "max_logit_abs": 0.0,
                      "max_logit_ratio": 0.0, "kv_tokens_checked": 0, "kv_exact_tokens": 0, "max_kv_abs": 0.0,
                      "max_kv_ratio": 0.0, "preemptions": 0, "recomputed_seqs": set()}

    @property
    def finished(self) -> bool:
        return all(s.status == Status.FINISHED for s in self.ref.seqs)

    @property
    def forced_streams(self) -> set[str]:
        return {sid for _, sid, _, _ in self.forced}

    def _step_reference(self) -> None:
        if self.ref_attention is None:
            self.ref.step()
            return
        import minivllm.attention as attention_mod

        inner = attention_mod.paged_attention_batch_online_v1
        attention_mod.paged_attention_batch_online_v1 = self.ref_attention
        try:
            self.ref.step()
        finally:
            attention_mod.paged_attention_batch_online_v1 = inner

    def step(self) -> None:
        step = self.stats["steps"] + 1
        sync = torch.cuda.synchronize if self.model.language_model_head.weight.is_cuda else (lambda: None)
        sync()
        t0 = time.perf_counter()
        self.model.set_decode_attention_backend("reference")
        self._step_reference()
        sync()
        t1 = time.perf_counter()
        self.model.set_decode_attention_backend("hip")
        self.hip.step()
        sync()
        self.wall["reference"] += t1 - t0
        self.wall["hip"] += time.perf_counter() - t1
        self.stats["steps"] = step
        a, b = self.ref, self.hip
        if a.plan != b.plan:
            raise AssertionError(f"step {step}: schedules differ: {a.plan} vs {b.plan}")
        if a.decoded != b.decoded:
            raise AssertionError(f"step {step}: decode batches differ")
        sa, sb = a.rt.metrics_summary(), b.rt.metrics_summary()
        for key in ("iterations", "scheduled_tokens", "prefill_tokens", "decode_tokens", "output_tokens",
                    "preemptions", "repeated_kv_tokens"):
            if sa[key] != sb[key]:
                raise AssertionError(f"step {step}: {key} {sa[key]} vs {sb[key]}")
        self.stats["preemptions"] = sa["preemptions"]
        self.stats["decode_rows"] = sa["decode_tokens"]
        for sid, _, _ in a.plan[0]:
            if a.by_id[sid].num_preemptions:
                self.stats["recomputed_seqs"].add(sid)
        self._check_states(step)
        self._check_decode(step)
        self._check_kv(step)

    def _check_states(self, step: int) -> None:
        for x in self.ref.seqs:
            y = self.hip.by_id[x.seq_id]
            if (x.status, x.length, x.prompt_pos, x.block_table, x.num_preemptions) != \
                    (y.status, y.length, y.prompt_pos, y.block_table, y.num_preemptions):
                raise AssertionError(f"step {step}: state of {x.seq_id} differs")
            if len(x.generated_tokens) != len(y.generated_tokens):
                raise AssertionError(f"step {step}: {x.seq_id} generated counts differ")

    def _check_decode(self, step: int) -> None:
        a, b = self.ref, self.hip
        if (a.logits is None) != (b.logits is None):
            raise AssertionError(f"step {step}: decode ran in one runtime only")
        atol, rtol = self.logit_tol
        if a.logits is not None:
            diff = (a.logits - b.logits).abs()
            scale = a.logits.abs().amax(dim=1, keepdim=True) if self.row_scaled else a.logits.abs()
            ratio = (diff / (atol + rtol * scale)).max().item()
            self.stats["max_logit_abs"] = max(self.stats["max_logit_abs"], diff.max().item())
            self.stats["max_logit_ratio"] = max(self.stats["max_logit_ratio"], ratio)
            self.stats["decode_rows_checked"] += a.logits.shape[0]
            if ratio > 1:
                raise AssertionError(f"step {step}: decode logits differ by {diff.max().item():.4g} "
                                     f"(tolerance atol {atol} + rtol {rtol} * |ref|)")
        # Tokens: every stream agrees up to this step (earlier differences were
        # forced away); a token drawn in this step may differ only at a near
        # tie of the reference's logits, and is then replaced by the reference's.
        for x in a.seqs:
            y = b.by_id[x.seq_id]
            if x.generated_tokens == y.generated_tokens:
                continue
            k = next(i for i, (p, q) in enumerate(zip(x.generated_tokens, y.generated_tokens)) if p != q)
            if k != len(x.generated_tokens) - 1 or a.logits is None or x.seq_id not in a.decoded:
                raise AssertionError(f"step {step}: {x.seq_id} token {k} differs outside a decode step")
            row = a.logits[a.decoded.index(x.seq_id)]
            top = torch.topk(row, 2).values.tolist()
            margin = top[0] - top[1]
            allowed = self.tie_margin
            if allowed is None:
                allowed = 2 * (atol + rtol * row.abs().max().item())
            if margin >= allowed:
                raise AssertionError(f"step {step}: {x.seq_id} token {k} differs at reference top-2 "
                                     f"margin {margin:.4g} (allowed only below {allowed:.4g})")
            if y.last_token != y.generated_tokens[-1] or x.last_token != x.generated_tokens[-1]:
                raise AssertionError(f"step {step}: {x.seq_id} pending token is not its last generated one")
            y.generated_tokens[-1] = x.generated_tokens[-1]
            y.last_token = x.last_token
            self.forced.append((step, x.seq_id, k, margin))

    def _check_kv(self, step: int) -> None:
        live = [x for x in self.ref.seqs if x.status != Status.FINISHED and x.length > 0]
        if not live:
            return
        if self.kv_tol is None:
            atol, rtol = self.logit_tol
            for x in live:
                y = self.hip.by_id[x.seq_id]
                ka, va = self.ref.rt.runner.kv_pool.gather_sequence(x)
                kb, vb = self.hip.rt.runner.kv_pool.gather_sequence(y)
                for u, w in ((ka, kb), (va, vb)):
                    torch.testing.assert_close(w, u, atol=atol, rtol=rtol,
                                               msg=lambda m: f"step {step}: logical KV of {x.seq_id}: {m}")
                    self.stats["max_kv_abs"] = max(self.stats["max_kv_abs"], (u - w).abs().max().item())
                self.stats["kv_tokens_checked"] += x.length
            return
        pa, pb = self.ref.rt.runner.kv_pool, self.hip.rt.runner.kv_pool
        S, dev = pa.block_size, pa.k.device
        slots, exact = [], []
        for x in live:
            slots += _token_slots(x, S)
            end = self.ref.prefill_end.get(x.seq_id, 0)
            exact += [p < end for p in range(x.length)]
        idx = torch.tensor(slots, dtype=torch.long, device=dev)
        ex = torch.tensor(exact, dtype=torch.bool, device=dev)
        atol, rtol = self.kv_tol
        L, N, _, H, D = pa.k.shape
        for layer in range(L):
            for ta, tb in ((pa.k, pb.k), (pa.v, pb.v)):
                u = ta[layer].reshape(N * S, H, D).index_select(0, idx)
                w = tb[layer].reshape(N * S, H, D).index_select(0, idx)
                same = (u.view(torch.int16) == w.view(torch.int16)).all(dim=(1, 2)) \
                    if u.element_size() == 2 else (u.view(torch.int32) == w.view(torch.int32)).all(dim=(1, 2))
                must = ex if layer > 0 else torch.ones_like(ex)
                bad = must & ~same
                if bool(bad.any()):
                    raise AssertionError(f"step {step}: layer {layer} KV not bit-identical at "
                                         f"{int(bad.sum())} prefill-written or layer-0 positions")
                uf, wf = u.float(), w.float()
                diff = (uf - wf).abs()
                scale = uf.abs().amax(dim=(1, 2), keepdim=True) if self.row_scaled else uf.abs()
                worst = (diff / (atol + rtol * scale)).max().item()
                self.stats["max_kv_abs"] = max(self.stats["max_kv_abs"], diff.max().item())
                self.stats["max_kv_ratio"] = max(self.stats["max_kv_ratio"], worst)
                if worst > 1:
                    raise AssertionError(f"step {step}: layer {layer} logical KV differs by "
                                         f"{diff.max().item():.4g} (tolerance atol {atol} + rtol {rtol} * |ref|)")
        self.stats["kv_tokens_checked"] += len(slots)
        self.stats["kv_exact_tokens"] += int(ex.sum())

    def finish_checks(self) -> None:
        """End-of-run checks of a completed workload (no KV leak, invariants)."""
        for probe in (self.ref, self.hip):
            bm = probe.rt.block_manager
            if bm.block_owner or len(bm.free_blocks) != bm.num_blocks:
                raise AssertionError("KV capacity leak after the completed workload")
            bm.check_invariants(probe.seqs)
