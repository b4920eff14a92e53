"""Per-iteration scheduling of decode tokens and prefill chunks.

Public surface of minivllm/scheduler.py (Scheduler, PrefillWorkItem,
ScheduleOutput, the waiting / prefilling / running queues, preempt,
retire_finished, num_preemptions). The decision order is what fixes the
reference's block tables and known counts, so it is kept exactly:

An iteration spends two budgets, batched tokens and free KV blocks, in three
passes, each over a snapshot of its queue taken when the pass starts:

1. decode: each RUNNING sequence, in queue order, asks for one token and
   the blocks that token needs; the pass ends when fewer than one token is
   left;
2. continuing prefills: each PREFILLING sequence with prompt left asks for
   a chunk; the pass ends when no token is left;
3. admissions from the head of the waiting queue (FIFO), only if nothing was
   evicted earlier in this iteration; it stops at the first request that
   does not fit (max_running, the conservative reservation, the chunk or
   its blocks).

A chunk is min(prompt left, tokens left); under "recompute" it is further
capped by what the sequence's blocks plus the free blocks can still hold.
When a decode token, or (under "recompute") a prefill that could not get a
single token, lacks blocks, victims are evicted until the blocks suffice or
no candidate is left: newest PREFILLING first, then newest RUNNING, never
the sequence asking, never one already planned this iteration, never one
without blocks. A sequence that still does not fit is skipped for this
iteration. Evicted sequences go back to the head of the waiting queue with
their history (running ones keep prompt + generated[:-1] to rebuild).
"""
from __future__ import annotations

from collections.abc import Iterator
from dataclasses import dataclass, field

from .block_manager import BlockManager
from .sequence import SequenceState, Status

POLICIES = ("conservative", "recompute")


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


@dataclass
class _Budget:
    """What is left to spend in one iteration, and what it has committed."""
    tokens: int
    blocks: int
    planned: set[int] = field(default_factory=set)   # id() of sequences planned this iteration
    evicted: bool = False

    def commit(self, seq: SequenceState, tokens: int, blocks: int) -> None:
        self.tokens -= tokens
        self.blocks -= blocks
        self.planned.add(id(seq))


class Scheduler:
    def __init__(self, block_manager: BlockManager, max_running: int, max_num_batched_tokens: int,
                 preemption_policy: str = "conservative"):
        if preemption_policy not in POLICIES:
            raise ValueError("preemption_policy must be 'conservative' or 'recompute'")
        self.block_manager = block_manager
        self.max_running = max_running
        self.max_num_batched_tokens = max_num_batched_tokens
        self.preemption_policy = preemption_policy
        self.waiting: list[SequenceState] = []
        self.prefilling: list[SequenceState] = []
        self.running: list[SequenceState] = []
        self.num_preemptions = 0

    # ------------------------------------------------------------ accounting

    @property
    def _recompute(self) -> bool:
        return self.preemption_policy == "recompute"

    def _lifetime_blocks(self, seq: SequenceState) -> int:
        """Blocks a request holds at its longest: every token but the last
        sampled one enters the pool."""
        S = self.block_manager.block_size
        return -(-(seq.max_tokens - 1) // S)

    def _reservation_fits(self, seq: SequenceState) -> bool:
        """Conservative admission: the lifetime blocks of every active request
        plus this one fit the pool."""
        held = sum(self._lifetime_blocks(s) for s in (*self.running, *self.prefilling))
        return held + self._lifetime_blocks(seq) <= self.block_manager.num_blocks

    def _chunk(self, seq: SequenceState, budget: _Budget) -> int:
        """Prefill tokens to plan for `seq` now (0: none fit)."""
        n = min(seq.remaining_prompt_tokens, budget.tokens)
        if self._recompute:
            S = self.block_manager.block_size
            room = (len(seq.block_table) + budget.blocks) * S - seq.length
            n = min(n, max(room, 0))
        return n

    # -------------------------------------------------------------- requests

    def add_request(self, seq: SequenceState) -> None:
        if not seq.prompt_tokens or seq.max_tokens <= seq.prompt_length:
            raise ValueError("a request needs a nonempty prompt and at least one output token")
        if self._lifetime_blocks(seq) > self.block_manager.num_blocks:
            raise ValueError("the request's largest KV footprint exceeds the block pool")
        self.waiting.append(seq)

    def preempt(self, seq: SequenceState) -> None:
        """Releases an active request's KV and puts it first in the waiting
        queue. Only between iterations."""
        if seq in self.running:
            if not seq.generated_tokens or seq.last_token != seq.generated_tokens[-1]:
                raise RuntimeError(f"{seq.seq_id}: running request without a pending output token")
            # Rebuild everything whose KV was committed; the pending token
            # stays the next decode input.
            rebuild = seq.prompt_tokens + seq.generated_tokens[:-1]
            if len(rebuild) != seq.length:
                raise RuntimeError(f"{seq.seq_id}: committed KV does not match its token history")
            seq.recompute_tokens = rebuild
            self.running.remove(seq)
        elif seq in self.prefilling:
            # The partial KV is dropped; recompute_tokens (if any) stay.
            self.prefilling.remove(seq)
        else:
            raise ValueError(f"{seq.seq_id} is not active and cannot be preempted")
        self.block_manager.free(seq)     # also clears the table and length
        seq.prompt_pos = 0
        seq.status = Status.WAITING
        seq.num_preemptions += 1
        self.num_preemptions += 1
        self.waiting.insert(0, seq)

    def retire_finished(self) -> None:
        still = []
        for seq in self.running:
            if not seq.is_finished():
                still.append(seq)
                continue
            seq.status = Status.FINISHED
            self.block_manager.free(seq)
        self.running = still

    # -------------------------------------------------------------- eviction

    def _victims(self, asking: SequenceState, budget: _Budget) -> Iterator[SequenceState]:
        """Eviction candidates in order: newest prefill first, then newest decode."""
        for seq in (*reversed(self.prefilling), *reversed(self.running)):
            if seq is not asking and id(seq) not in budget.planned and seq.block_table:
                yield seq

    def _make_room(self, asking: SequenceState, blocks: int, budget: _Budget) -> bool:
        """Evicts (recompute policy only) until `blocks` free blocks are
        available to `asking`; True when they are."""
        if budget.blocks >= blocks:
            return True
        if not self._recompute:
            return False
        for victim in self._victims(asking, budget):
            budget.blocks += len(victim.block_table)
            self.preempt(victim)
            budget.evicted = True
            if budget.blocks >= blocks:
                return True
        return False

    # ---------------------------------------------------------------- passes

    def _plan_decodes(self, budget: _Budget) -> list[SequenceState]:
        out = []
        for seq in list(self.running):
            if budget.tokens < 1:
                break
            if seq.status is not Status.RUNNING:       # evicted earlier in this pass
                continue
            need = self.block_manager.num_new_blocks_needed(seq, 1)
            if not self._make_room(seq, need, budget):
                continue
            budget.commit(seq, 1, need)
            out.append(seq)
        return out

    def _plan_prefills(self, budget: _Budget) -> list[PrefillWorkItem]:
        out = []
        for seq in list(self.prefilling):
            if budget.tokens <= 0:
                break
            if seq.status is not Status.PREFILLING or seq.remaining_prompt_tokens <= 0:
                continue
            n = self._chunk(seq, budget)
            if n == 0 and self._recompute:
                self._make_room(seq, 1, budget)
                n = self._chunk(seq, budget)
            if n <= 0:
                continue
            need = self.block_manager.num_new_blocks_needed(seq, n)
            if need > budget.blocks:
                continue
            budget.commit(seq, n, need)
            out.append(PrefillWorkItem(seq, seq.prompt_pos, n))
        return out

    def _plan_admissions(self, budget: _Budget) -> list[PrefillWorkItem]:
        out = []
        while self.waiting and budget.tokens > 0:
            if len(self.running) + len(self.prefilling) >= self.max_running:
                break
            seq = self.waiting[0]
            if not self._recompute and not self._reservation_fits(seq):
                break
            n = self._chunk(seq, budget)
            if n <= 0:
                break
            need = self.block_manager.num_new_blocks_needed(seq, n)
            if need > budget.blocks:
                break
            self.waiting.pop(0)
            seq.status = Status.PREFILLING
            self.prefilling.append(seq)
            budget.commit(seq, n, need)
            out.append(PrefillWorkItem(seq, seq.prompt_pos, n))
        return out

    def schedule(self) -> ScheduleOutput:
        budget = _Budget(tokens=self.max_num_batched_tokens, blocks=len(self.block_manager.free_blocks))
        decode = self._plan_decodes(budget)
        prefill = self._plan_prefills(budget)
        # An eviction closes admissions for this iteration: the evicted
        # request would otherwise take its blocks straight back.
        if not budget.evicted:
            prefill += self._plan_admissions(budget)
        return ScheduleOutput(prefill=prefill, decode=decode,
                              num_scheduled_tokens=self.max_num_batched_tokens - budget.tokens)
