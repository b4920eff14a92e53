"""The serving loop: one scheduler plan per iteration, executed by the model
runner, with a telemetry record per iteration.

Public surface of minivllm/mini_runtime.py (MiniRuntime, IterationRecord,
metrics_summary, export_records_json). Runtimes are also assembled without
__init__ (``MiniRuntime.__new__`` plus block_manager, scheduler, runner,
iteration and records set by hand), so every other attribute has a default.

An iteration:
  1. plan (Scheduler.schedule);
  2. decode: one batched step for the planned RUNNING sequences; each gets
     its greedy token;
  3. prefill: the planned chunks in plan order. A sequence whose prefill
     input is complete becomes RUNNING. After an ordinary prefill its first
     token is the greedy choice of the chunk's last row; after a rebuild
     (recompute preemption) no token is drawn, since the pending one was
     drawn before the eviction;
  4. retire finished sequences and append an IterationRecord.

``repeated_kv_tokens`` counts logical KV positions executed a second time:
each sequence keeps the highest position it has ever executed, which
survives eviction.
"""
from __future__ import annotations

import json
import time
from dataclasses import asdict, dataclass
from pathlib import Path

import torch

from .block_manager import BlockManager
from .kv_block_pool import KVBlockPool
from .model import MiniGPT
from .model_runner import ModelRunner
from .scheduler import ScheduleOutput, Scheduler
from .sequence import SequenceState, Status


@dataclass
class IterationRecord:
    iteration: int
    prefill_requests: int
    decode_requests: int
    prefill_tokens: int
    decode_tokens: int
    scheduled_tokens: int
    waiting: int
    prefilling: int
    running: int
    used_blocks: int
    free_blocks: int
    kv_utilization: float
    prefill_ms: float
    decode_ms: float
    iteration_ms: float
    # Host wall-clock milliseconds, or device-synchronised ones with
    # sync_cuda_timing.
    schedule_ms: float = 0.0
    preemptions: int = 0
    repeated_kv_tokens: int = 0
    output_tokens: int = 0
    finished_requests: int = 0


class MiniRuntime:
    verbose = False
    sync_cuda_timing = False

    def __init__(self, num_blocks, block_size, max_running, max_num_batched_tokens,
                 preemption_policy="conservative", sync_cuda_timing=False, verbose=False):
        self.block_manager = BlockManager(num_blocks, block_size)
        self.scheduler = Scheduler(self.block_manager, max_running, max_num_batched_tokens,
                                   preemption_policy=preemption_policy)
        model = MiniGPT(n_embd=512, n_head=8, vocab_size=1024, block_size=1024, dropout=0.0, n_layer=8)
        pool = KVBlockPool(n_layer=8, num_blocks=num_blocks, block_size=block_size, n_head=8, head_dim=64)
        self.runner = ModelRunner(model=model, kv_pool=pool, block_manager=self.block_manager)
        self.iteration = 0
        self.records: list[IterationRecord] = []
        self.sync_cuda_timing = sync_cuda_timing
        self.verbose = verbose
        self._kv_high_watermark: dict[str, int] = {}

    def add_request(self, seq: SequenceState) -> None:
        self.scheduler.add_request(seq)

    # ----------------------------------------------------------- telemetry

    def _clock(self) -> float:
        """perf_counter, after draining the device when timing is synchronised."""
        if self.sync_cuda_timing and torch.cuda.is_available():
            torch.cuda.synchronize()
        return time.perf_counter()

    def _repeated(self, seq: SequenceState, start: int, count: int) -> int:
        """Positions of [start, start + count) this sequence executed before;
        raises its high-water mark to start + count."""
        marks = self.__dict__.setdefault("_kv_high_watermark", {})
        before = marks.get(seq.seq_id, 0)
        marks[seq.seq_id] = max(before, start + count)
        return max(0, min(before, start + count) - start)

    def metrics_summary(self) -> dict:
        """Totals over the recorded iterations (scheduler accounting; the
        times are whatever the records hold)."""
        recs = self.records
        n = len(recs)

        def total(name):
            return sum(getattr(r, name) for r in recs)

        return {
            "iterations": n,
            "scheduled_tokens": total("scheduled_tokens"),
            "prefill_tokens": total("prefill_tokens"),
            "decode_tokens": total("decode_tokens"),
            "output_tokens": total("output_tokens"),
            "preemptions": total("preemptions"),
            "repeated_kv_tokens": total("repeated_kv_tokens"),
            "peak_used_blocks_at_step_end": max((r.used_blocks for r in recs), default=0),
            "average_kv_utilization_at_step_end": total("kv_utilization") / n if n else 0.0,
            "total_iteration_ms": total("iteration_ms"),
        }

    def export_records_json(self, path, metadata: dict | None = None) -> None:
        synced = self.sync_cuda_timing and torch.cuda.is_available()
        doc = {"timing_mode": "cuda_synchronized" if synced else "host_wall",
               "summary": self.metrics_summary(),
               "records": [asdict(r) for r in self.records]}
        if metadata is not None:
            doc["metadata"] = metadata
        out = Path(path)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(doc, indent=2), encoding="utf-8")

    # -------------------------------------------------------------- phases

    def _validate(self, plan: ScheduleOutput) -> None:
        sched = self.scheduler
        if len(sched.running) + len(plan.prefill) > sched.max_running:
            raise AssertionError(f"plan exceeds max_running={sched.max_running}: "
                                 f"{len(sched.running)} running + {len(plan.prefill)} prefills")
        tokens = sum(w.num_tokens for w in plan.prefill) + len(plan.decode)
        if tokens != plan.num_scheduled_tokens or tokens > sched.max_num_batched_tokens:
            raise AssertionError(f"plan token count {tokens} vs {plan.num_scheduled_tokens} "
                                 f"(budget {sched.max_num_batched_tokens})")
        if {w.seq.seq_id for w in plan.prefill} & {s.seq_id for s in plan.decode}:
            raise AssertionError("a sequence is planned for prefill and decode in one iteration")

    def _decode(self, batch: list[SequenceState]) -> tuple[int, int]:
        """Runs the decode batch; returns (output tokens, repeated positions)."""
        if not batch:
            return 0, 0
        positions = [s.length for s in batch]
        _, tokens = self.runner.decode_batch(batch)
        repeated = sum(self._repeated(s, p, 1) for s, p in zip(batch, positions))
        for seq, tok in zip(batch, tokens):
            seq.generated_tokens.append(tok)
            seq.last_token = tok
        return len(tokens), repeated

    def _start_decoding(self, seq: SequenceState, logits: torch.Tensor) -> int:
        """A sequence whose prefill input is complete joins the decode queue;
        returns the output tokens drawn (1 after an ordinary prefill, 0 after
        a rebuild)."""
        drawn = 0
        if seq.recompute_tokens is None:
            tok = int(torch.argmax(logits[:, -1], dim=-1).item())
            seq.generated_tokens.append(tok)
            seq.last_token = tok
            seq.first_token_iter = self.iteration
            drawn = 1
        else:
            # The rebuilt KV stops before the pending token, which stays the
            # next decode input.
            if not (seq.generated_tokens and seq.last_token == seq.generated_tokens[-1]
                    and seq.length == len(seq.recompute_tokens)):
                raise AssertionError(f"{seq.seq_id}: rebuilt KV does not end before the pending token")
            seq.recompute_tokens = None
            seq.prompt_pos = seq.prompt_length
        seq.status = Status.RUNNING
        self.scheduler.prefilling.remove(seq)
        self.scheduler.running.append(seq)
        return drawn

    def _prefill(self, plan: ScheduleOutput) -> tuple[int, int]:
        """Runs the planned chunks; returns (output tokens, repeated positions)."""
        drawn = repeated = 0
        for work in plan.prefill:
            seq = work.seq
            if seq.first_schedule_iter is None:
                seq.first_schedule_iter = self.iteration
            logits = self.runner.prefill_chunk(seq=seq, start_pos=work.start_pos, num_tokens=work.num_tokens)
            repeated += self._repeated(seq, work.start_pos, work.num_tokens)
            seq.prompt_pos += work.num_tokens
            if seq.prompt_pos != seq.length:
                raise AssertionError(f"{seq.seq_id}: prefill position {seq.prompt_pos} != length {seq.length}")
            if seq.prompt_finished:
                drawn += self._start_decoding(seq, logits)
        return drawn, repeated

    def _retire(self) -> int:
        done = [s for s in self.scheduler.running if s.is_finished()]
        for seq in done:
            seq.finish_iter = self.iteration
        self.scheduler.retire_finished()
        return len(done)

    # ---------------------------------------------------------------- step

    def step(self) -> None:
        self.iteration += 1
        sched = self.scheduler
        t_begin = self._clock()
        evictions_before = sched.num_preemptions
        plan = sched.schedule()
        t_planned = time.perf_counter()
        self._validate(plan)
        if self.verbose:
            print(f"[iteration {self.iteration}] prefill {[w.seq.seq_id for w in plan.prefill]} "
                  f"decode {[s.seq_id for s in plan.decode]} tokens {plan.num_scheduled_tokens}")

        t0 = time.perf_counter()
        dec_out, dec_rep = self._decode(plan.decode)
        t1 = self._clock()
        pre_out, pre_rep = self._prefill(plan)
        t2 = self._clock()
        finished = self._retire()
        t_end = self._clock()

        free = len(self.block_manager.free_blocks)
        used = self.block_manager.num_blocks - free
        self.records.append(IterationRecord(
            iteration=self.iteration,
            prefill_requests=len(plan.prefill),
            decode_requests=len(plan.decode),
            prefill_tokens=sum(w.num_tokens for w in plan.prefill),
            decode_tokens=len(plan.decode),
            scheduled_tokens=plan.num_scheduled_tokens,
            waiting=len(sched.waiting),
            prefilling=len(sched.prefilling),
            running=len(sched.running),
            used_blocks=used,
            free_blocks=free,
            kv_utilization=used / self.block_manager.num_blocks,
            prefill_ms=(t2 - t1) * 1e3,
            decode_ms=(t1 - t0) * 1e3,
            iteration_ms=(t_end - t_begin) * 1e3,
            schedule_ms=(t_planned - t_begin) * 1e3,
            preemptions=sched.num_preemptions - evictions_before,
            repeated_kv_tokens=dec_rep + pre_rep,
            output_tokens=dec_out + pre_out,
            finished_requests=finished,
        ))
        if self.verbose:
            print(f"[iteration {self.iteration}] free blocks {free}")
