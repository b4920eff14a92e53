"""Per-step batched decode metadata (minivllm/decode_batch_metadata.py:6-14).

All four tensors live on the model device, int64 in the runtime:
  positions       [B]     logical position of the token being decoded
  context_lengths [B]     positions + 1 (includes the token written this step)
  block_tables    [B, M]  logical -> physical block ids, -1 past each row's blocks
  slot_mapping    [B]     physical slot (block * S + offset) receiving the new
                          K/V; a negative slot marks a padding row that the
                          KV append skips
"""
from __future__ import annotations

from dataclasses import dataclass

from torch import Tensor


@dataclass
class DecodeBatchMetadata:
    positions: Tensor
    context_lengths: Tensor
    block_tables: Tensor
    slot_mapping: Tensor
