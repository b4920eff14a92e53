"""Runtime loop and per-iteration telemetry (minivllm/mini_runtime.py:14-315).

``step()`` asks the scheduler for a plan, runs the decode batch first (one
token per RUNNING sequence through ``ModelRunner.decode_batch``), then the
prefill chunks; a sequence whose prompt completes gets its first token by
greedy argmax unless it was rebuilding KV after recompute preemption (its
pending token was already generated). Finished sequences are retired and an
``IterationRecord`` is appended.
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
from .scheduler import Scheduler
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
    # Host wall-clock durations unless sync_cuda_timing is set.
    schedule_ms: float = 0.0
    preemptions: int = 0
    repeated_kv_tokens: int = 0
    output_tokens: int = 0
    finished_requests: int = 0


class MiniRuntime:
    # Class-level default keeps runtimes assembled via __new__ quiet.
    verbose = False

    def __init__(self, num_blocks, block_size, max_running, max_num_batched_tokens,
                 preemption_policy="conservative", sync_cuda_timing=False, verbose=False):
        self.block_manager = BlockManager(num_blocks, block_size)
        self.scheduler = Scheduler(self.block_manager, max_running, max_num_batched_tokens,
                                   preemption_policy=preemption_policy)
        self.runner = ModelRunner(
            model=MiniGPT(n_embd=512, n_head=8, vocab_size=1024, block_size=1024, dropout=0.0, n_layer=8),
            kv_pool=KVBlockPool(n_layer=8, num_blocks=num_blocks, block_size=block_size, n_head=8,
                                head_dim=64),
            block_manager=self.block_manager,
        )
        self.iteration = 0
        self.records: list[IterationRecord] = []
        self.sync_cuda_timing = sync_cuda_timing
        self.verbose = verbose
        self._kv_high_watermark: dict[str, int] = {}

    # -------------------------------------------------------------- helpers

    def _timing_sync(self) -> None:
        if getattr(self, "sync_cuda_timing", False) and torch.cuda.is_available():
            torch.cuda.synchronize()

    def _track_executed_kv(self, seq: SequenceState, start: int, count: int) -> int:
        """Logical KV positions in [start, start+count) executed before (recompute work)."""
        if not hasattr(self, "_kv_high_watermark"):
            self._kv_high_watermark = {}
        previous = self._kv_high_watermark.get(seq.seq_id, 0)
        end = start + count
        self._kv_high_watermark[seq.seq_id] = max(previous, end)
        return max(0, min(end, previous) - start)

    def metrics_summary(self) -> dict:
        """Aggregated per-iteration accounting, not a serving benchmark."""
        r = self.records
        return {
            "iterations": len(r),
            "scheduled_tokens": sum(x.scheduled_tokens for x in r),
            "prefill_tokens": sum(x.prefill_tokens for x in r),
            "decode_tokens": sum(x.decode_tokens for x in r),
            "output_tokens": sum(x.output_tokens for x in r),
            "preemptions": sum(x.preemptions for x in r),
            "repeated_kv_tokens": sum(x.repeated_kv_tokens for x in r),
            "peak_used_blocks_at_step_end": max((x.used_blocks for x in r), default=0),
            "average_kv_utilization_at_step_end": (sum(x.kv_utilization for x in r) / len(r)) if r else 0.0,
            "total_iteration_ms": sum(x.iteration_ms for x in r),
        }

    def export_records_json(self, path, metadata: dict | None = None) -> None:
        dest = Path(path)
        dest.parent.mkdir(parents=True, exist_ok=True)
        synced = getattr(self, "sync_cuda_timing", False) and torch.cuda.is_available()
        payload = {
            "timing_mode": "cuda_synchronized" if synced else "host_wall",
            "summary": self.metrics_summary(),
            "records": [asdict(rec) for rec in self.records],
        }
        if metadata is not None:
            payload["metadata"] = metadata
        dest.write_text(json.dumps(payload, indent=2), encoding="utf-8")

    def add_request(self, seq: SequenceState) -> None:
        self.scheduler.add_request(seq)

    # ----------------------------------------------------------------- step

    def step(self) -> None:
        self.iteration += 1
        self._timing_sync()
        t_iter = time.perf_counter()
        preemptions_before = self.scheduler.num_preemptions
        plan = self.scheduler.schedule()
        schedule_ms = (time.perf_counter() - t_iter) * 1000
        repeated = 0
        outputs = 0
        assert len(self.scheduler.running) + len(plan.prefill) <= self.scheduler.max_running
        if self.verbose:
            print(f"\nIteration {self.iteration}")
            print("prefill:", [x.seq.seq_id for x in plan.prefill])
            print("decode:", [x.seq_id for x in plan.decode])
            print("scheduled tokens:", plan.num_scheduled_tokens)

        t_decode = time.perf_counter()
        if plan.decode:
            starts = [(seq, seq.length) for seq in plan.decode]
            _, next_tokens = self.runner.decode_batch(plan.decode)
            for seq, start in starts:
                repeated += self._track_executed_kv(seq, start, 1)
            outputs += len(next_tokens)
            for seq, token in zip(plan.decode, next_tokens):
                seq.generated_tokens.append(token)
                seq.last_token = token
        self._timing_sync()
        decode_ms = (time.perf_counter() - t_decode) * 1000

        t_prefill = time.perf_counter()
        for item in plan.prefill:
            seq = item.seq
            if seq.first_schedule_iter is None:
                seq.first_schedule_iter = self.iteration
            logits = self.runner.prefill_chunk(seq=seq, start_pos=item.start_pos, num_tokens=item.num_tokens)
            repeated += self._track_executed_kv(seq, item.start_pos, item.num_tokens)
            seq.prompt_pos += item.num_tokens
            assert seq.prompt_pos == seq.length
            if not seq.prompt_finished:
                continue
            if seq.recompute_tokens is not None:
                # Rebuilt KV excludes the pending last token: never re-sample it.
                assert seq.generated_tokens
                assert seq.last_token == seq.generated_tokens[-1]
                assert seq.length == len(seq.recompute_tokens)
                seq.recompute_tokens = None
                seq.prompt_pos = seq.prompt_length
            else:
                first = int(torch.argmax(logits[:, -1], dim=-1).item())
                seq.generated_tokens.append(first)
                seq.last_token = first
                seq.first_token_iter = self.iteration
                outputs += 1
            seq.status = Status.RUNNING
            self.scheduler.prefilling.remove(seq)
            self.scheduler.running.append(seq)
        self._timing_sync()
        prefill_ms = (time.perf_counter() - t_prefill) * 1000

        prefill_tokens = sum(item.num_tokens for item in plan.prefill)
        decode_tokens = len(plan.decode)
        assert prefill_tokens + decode_tokens == plan.num_scheduled_tokens
        assert plan.num_scheduled_tokens <= self.scheduler.max_num_batched_tokens
        assert {x.seq.seq_id for x in plan.prefill}.isdisjoint({x.seq_id for x in plan.decode})

        finished = 0
        for seq in self.scheduler.running:
            if seq.is_finished():
                seq.finish_iter = self.iteration
                finished += 1
        self.scheduler.retire_finished()

        self._timing_sync()
        iteration_ms = (time.perf_counter() - t_iter) * 1000
        free = len(self.block_manager.free_blocks)
        used = self.block_manager.num_blocks - free
        self.records.append(IterationRecord(
            iteration=self.iteration,
            prefill_requests=len(plan.prefill),
            decode_requests=len(plan.decode),
            prefill_tokens=prefill_tokens,
            decode_tokens=decode_tokens,
            scheduled_tokens=plan.num_scheduled_tokens,
            waiting=len(self.scheduler.waiting),
            prefilling=len(self.scheduler.prefilling),
            running=len(self.scheduler.running),
            used_blocks=used,
            free_blocks=free,
            kv_utilization=used / self.block_manager.num_blocks,
            prefill_ms=prefill_ms,
            decode_ms=decode_ms,
            iteration_ms=iteration_ms,
            schedule_ms=schedule_ms,
            preemptions=self.scheduler.num_preemptions - preemptions_before,
            repeated_kv_tokens=repeated,
            output_tokens=outputs,
            finished_requests=finished,
        ))
        if self.verbose:
            print("the number of free blocks: ", free)
