"""Physical block allocation and block tables (minivllm/block_manager.py:4-176).

The free list is a LIFO stack that initially pops 0, 1, 2, ...; released
blocks are pushed back in block-table order and reused first. These exact
allocation orders make block tables identical across backends, which the
lock-step comparisons rely on. ``slot = block * block_size + offset``.
"""
from __future__ import annotations

from .sequence import SequenceState


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.free_blocks: list[int] = list(reversed(range(num_blocks)))
        self.block_owner: dict[int, str] = {}

    def _allocate_block(self, seq: SequenceState) -> int:
        if not self.free_blocks:
            raise RuntimeError("KV block pool exhausted")
        block = self.free_blocks.pop()
        assert block not in self.block_owner
        self.block_owner[block] = seq.seq_id
        seq.block_table.append(block)
        return block

    def num_new_blocks_needed(self, seq: SequenceState, num_tokens: int) -> int:
        S = self.block_size
        target_blocks = (seq.length + num_tokens + S - 1) // S
        return max(0, target_blocks - len(seq.block_table))

    def can_reserve(self, seq: SequenceState, num_tokens: int) -> bool:
        return self.num_new_blocks_needed(seq, num_tokens) <= len(self.free_blocks)

    def _slot_for(self, seq: SequenceState, logical_pos: int) -> tuple[int, int, int]:
        logical_block, offset = divmod(logical_pos, self.block_size)
        if logical_block == len(seq.block_table):
            self._allocate_block(seq)
        assert logical_block < len(seq.block_table)
        block = seq.block_table[logical_block]
        return block, offset, block * self.block_size + offset

    def reserve_append_slot(self, seq: SequenceState) -> tuple[int, int, int]:
        """(physical_block, block_offset, physical_slot) for position seq.length."""
        return self._slot_for(seq, seq.length)

    def reserve_slots(self, seq: SequenceState, num_tokens: int) -> list[int]:
        """Physical slots for positions seq.length .. seq.length + num_tokens - 1."""
        return [self._slot_for(seq, seq.length + i)[2] for i in range(num_tokens)]

    def logical_to_slot(self, seq: SequenceState, logical_pos: int) -> int:
        if not 0 <= logical_pos < seq.length:
            raise IndexError(f"logical_pos={logical_pos}, length={seq.length}")
        logical_block, offset = divmod(logical_pos, self.block_size)
        return seq.block_table[logical_block] * self.block_size + offset

    def free(self, seq: SequenceState) -> list[int]:
        released = list(seq.block_table)
        for block in released:
            owner = self.block_owner.pop(block)
            assert owner == seq.seq_id
            self.free_blocks.append(block)
        seq.block_table.clear()
        seq.length = 0
        return released

    def check_invariants(self, sequences: list[SequenceState]) -> None:
        free = set(self.free_blocks)
        allocated = set(self.block_owner)
        assert len(free) == len(self.free_blocks)
        assert free.isdisjoint(allocated)
        assert free | allocated == set(range(self.num_blocks))
        S = self.block_size
        for seq in sequences:
            assert len(seq.block_table) == len(set(seq.block_table))
            for block in seq.block_table:
                assert self.block_owner[block] == seq.seq_id
            assert len(seq.block_table) == (seq.length + S - 1) // S
