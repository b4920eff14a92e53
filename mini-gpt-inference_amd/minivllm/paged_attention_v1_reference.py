"""Single-sequence paged online attention (minivllm/paged_attention_v1_reference.py:10-83).

Attends one query [H, D] over the first ``context_length`` logical tokens of
``seq`` (through its block table), in ``q.dtype``.
"""
from __future__ import annotations

import math

import torch

from .kv_block_pool import KVBlockPool
from .paged_attention_batch import _online_step
from .sequence import SequenceState


def paged_attention_online(q: torch.Tensor, pool: KVBlockPool, seq: SequenceState, layer_idx: int,
                           context_length: int) -> torch.Tensor:
    H, D = q.shape
    S = pool.block_size
    scale = 1.0 / math.sqrt(D)
    m = torch.full((H,), float("-inf"), device=q.device, dtype=q.dtype)
    l = torch.zeros(H, device=q.device, dtype=q.dtype)
    O = torch.zeros_like(q)
    for logical, physical in enumerate(seq.block_table):
        n = min(S, context_length - logical * S)
        if n <= 0:
            break
        keys = pool.k[layer_idx, physical, :n].transpose(0, 1).contiguous()
        values = pool.v[layer_idx, physical, :n].transpose(0, 1).contiguous()
        scores = (keys @ q[..., None]).squeeze(-1) * scale
        m, l, O = _online_step(m, l, O, scores, values)
    return O
