"""Per-call execution contexts (minivllm/kv_runtime.py:7-55)."""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .block_manager import BlockManager
from .kv_block_pool import KVBlockPool
from .sequence import SequenceState


@dataclass
class KVRuntimeContext:
    """One-token serial decode of one layer."""
    seq_state: SequenceState
    block_manager: BlockManager
    kv_pool: KVBlockPool
    layer_idx: int
    logical_pos: int
    context_length: int
    physical_block: int
    block_offset: int
    physical_slot: int


@dataclass
class PrefillRuntimeContext:
    """Whole-prompt prefill of one layer.

    block_table optionally carries the sequence's first
    ceil(context_length / S) physical blocks as an integer tensor on the
    pool's device (the HIP prefill kernel reads it; built once per call).
    """
    seq_state: SequenceState
    kv_pool: KVBlockPool
    layer_idx: int
    start_pos: int
    context_length: int
    slot_mapping: list[int] | torch.Tensor
    block_table: torch.Tensor | None = None


@dataclass
class PrefillChunkContext:
    """One prefill chunk [start_pos, start_pos + num_tokens) of one layer.

    slot_mapping is a list of physical slots, or the same slots as an int64
    tensor on the pool's device (the runner moves them once per chunk).
    block_table optionally carries the sequence's first
    ceil((start_pos + num_tokens) / S) physical blocks as a device tensor.
    """
    seq_state: SequenceState
    kv_pool: KVBlockPool
    layer_idx: int
    start_pos: int
    num_tokens: int
    slot_mapping: list[int] | torch.Tensor
    block_table: torch.Tensor | None = None
