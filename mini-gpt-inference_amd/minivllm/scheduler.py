"""Iteration scheduler (minivllm/scheduler.py:24-242).

Each step plans, in order: one decode token for every RUNNING sequence,
then prefill chunks for sequences already PREFILLING, then new admissions
from the waiting queue -- bounded by ``max_num_batched_tokens``, the free
KV blocks and ``max_running``. With ``preemption_policy="recompute"`` a
shortage of blocks evicts unprotected active sequences (newest partial
prefill first, then newest decode); an evicted sequence keeps its token
history and is re-prefilled later. After any eviction in a step no new
request is admitted in that step.
"""
from __future__ import annotations

from dataclasses import dataclass

from .block_manager import BlockManager
from .sequence import SequenceState, Status


@dataclass
class PrefillWorkItem:
    seq: SequenceState
    start_pos: int
    num_tokens: int

    @property
    def end_pos(self) -> int:
        return self.start_pos + self.num_tokens


@dataclass
class ScheduleOutput:
    prefill: list[PrefillWorkItem]
    decode: list[SequenceState]
    num_scheduled_tokens: int


class Scheduler:
    def __init__(self, block_manager: BlockManager, max_running: int, max_num_batched_tokens: int,
                 preemption_policy: str = "conservative"):
        if preemption_policy not in ("conservative", "recompute"):
            raise ValueError("preemption_policy must be 'conservative' or 'recompute'")
        self.waiting: list[SequenceState] = []
        self.prefilling: list[SequenceState] = []
        self.running: list[SequenceState] = []
        self.block_manager = block_manager
        self.max_running = max_running
        self.max_num_batched_tokens = max_num_batched_tokens
        self.preemption_policy = preemption_policy
        self.num_preemptions = 0

    # ---------------------------------------------------------- capacity

    def _max_kv_blocks(self, seq: SequenceState) -> int:
        # The final sampled token never enters the KV pool.
        S = self.block_manager.block_size
        return (seq.max_tokens - 1 + S - 1) // S

    def _can_admit_without_preemption(self, seq: SequenceState) -> bool:
        committed = sum(self._max_kv_blocks(s) for s in self.running + self.prefilling)
        return committed + self._max_kv_blocks(seq) <= self.block_manager.num_blocks

    def add_request(self, seq: SequenceState) -> None:
        if not seq.prompt_tokens or seq.max_tokens <= seq.prompt_length:
            raise ValueError("prompt must be nonempty and output token must be positive")
        if self._max_kv_blocks(seq) > self.block_manager.num_blocks:
            raise ValueError("request's maximum KV demand exceeds total block capacity")
        self.waiting.append(seq)

    # ----------------------------------------------------------- eviction

    def preempt(self, seq: SequenceState) -> None:
        """Evicts an active sequence's KV and requeues it first. Between steps only."""
        if seq in self.running:
            assert seq.generated_tokens, "RUNNING request has no output token"
            assert seq.last_token == seq.generated_tokens[-1]
            seq.recompute_tokens = seq.prompt_tokens + seq.generated_tokens[:-1]
            assert len(seq.recompute_tokens) == seq.length
            self.running.remove(seq)
        elif seq in self.prefilling:
            # Partial prefill KV is discarded; an interrupted recompute keeps
            # its recompute_tokens, an ordinary prefill keeps None.
            self.prefilling.remove(seq)
        else:
            raise ValueError("Only active requests may be preempted")
        self.num_preemptions += 1
        seq.num_preemptions += 1
        self.block_manager.free(seq)
        seq.prompt_pos = 0
        seq.status = Status.WAITING
        self.waiting.insert(0, seq)

    def retire_finished(self) -> None:
        alive = []
        for seq in self.running:
            if seq.is_finished():
                seq.status = Status.FINISHED
                self.block_manager.free(seq)
            else:
                alive.append(seq)
        self.running = alive

    def _choose_victim(self, target: SequenceState, protected_ids: set[int]) -> SequenceState | None:
        for seq in [*reversed(self.prefilling), *reversed(self.running)]:
            if seq is target or id(seq) in protected_ids:
                continue
            if seq.block_table:
                return seq
        return None

    def _free_for(self, target: SequenceState, needed: int, available: int,
                  protected_ids: set[int]) -> tuple[int, bool]:
        """Evicts victims until `needed` blocks are available (recompute policy)."""
        evicted = False
        if self.preemption_policy != "recompute":
            return available, evicted
        while available < needed:
            victim = self._choose_victim(target, protected_ids)
            if victim is None:
                break
            released = len(victim.block_table)
            self.preempt(victim)
            available += released
            evicted = True
        return available, evicted

    def _prefill_chunk_size(self, seq: SequenceState, remaining_budget: int, available_blocks: int) -> int:
        desired = min(seq.remaining_prompt_tokens, remaining_budget)
        if self.preemption_policy != "recompute":
            return desired
        # Only what already-held plus uncommitted blocks can store.
        fit = (len(seq.block_table) + available_blocks) * self.block_manager.block_size - seq.length
        return min(desired, max(0, fit))

    # ----------------------------------------------------------- planning

    def schedule(self) -> ScheduleOutput:
        prefill: list[PrefillWorkItem] = []
        decode: list[SequenceState] = []
        budget = self.max_num_batched_tokens
        free_blocks = len(self.block_manager.free_blocks)
        protected: set[int] = set()      # planned this step: never evicted
        evicted_this_step = False

        for seq in list(self.running):
            if budget < 1:
                break
            if seq.status != Status.RUNNING:
                continue                 # evicted earlier in this step
            needed = self.block_manager.num_new_blocks_needed(seq, 1)
            if needed > free_blocks:
                free_blocks, did = self._free_for(seq, needed, free_blocks, protected)
                evicted_this_step |= did
            if needed > free_blocks:
                continue
            decode.append(seq)
            protected.add(id(seq))
            budget -= 1
            free_blocks -= needed

        for seq in list(self.prefilling):
            if budget <= 0:
                break
            if seq.status != Status.PREFILLING:
                continue
            if seq.remaining_prompt_tokens <= 0:
                continue
            chunk = self._prefill_chunk_size(seq, budget, free_blocks)
            if chunk == 0 and self.preemption_policy == "recompute":
                free_blocks, did = self._free_for(seq, 1, free_blocks, protected)
                evicted_this_step |= did
                chunk = self._prefill_chunk_size(seq, budget, free_blocks)
            if chunk <= 0:
                continue
            needed = self.block_manager.num_new_blocks_needed(seq, chunk)
            if needed > free_blocks:
                continue
            prefill.append(PrefillWorkItem(seq, seq.prompt_pos, chunk))
            protected.add(id(seq))
            budget -= chunk
            free_blocks -= needed

        # After an eviction, admit nobody this step (avoids evict/re-admit ping-pong).
        while self.waiting and budget > 0 and not evicted_this_step:
            if len(self.running) + len(self.prefilling) >= self.max_running:
                break
            seq = self.waiting[0]
            if self.preemption_policy == "conservative" and not self._can_admit_without_preemption(seq):
                break
            chunk = self._prefill_chunk_size(seq, budget, free_blocks)
            if chunk <= 0:
                break
            needed = self.block_manager.num_new_blocks_needed(seq, chunk)
            if needed > free_blocks:
                break
            self.waiting.pop(0)
            seq.status = Status.PREFILLING
            self.prefilling.append(seq)
            prefill.append(PrefillWorkItem(seq, seq.prompt_pos, chunk))
            protected.add(id(seq))
            budget -= chunk
            free_blocks -= needed

        return ScheduleOutput(prefill=prefill, decode=decode,
                              num_scheduled_tokens=self.max_num_batched_tokens - budget)
