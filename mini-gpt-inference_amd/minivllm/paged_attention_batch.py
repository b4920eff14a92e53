"""PyTorch paged decode attention -- the ``"reference"`` decode backend.

Same contract and recurrence as minivllm/paged_attention_batch.py:
  * paged_attention_batch_reference (:7-118): per sequence, per logical block,
    host reads of lengths and table entries;
  * paged_attention_batch_online_v1 (:121-278): batched over sequences, one
    iteration per block-table column with masking of slots past each
    context (NaN-safe: values are masked before any arithmetic).
Both compute in ``q.dtype`` and return a fresh [B, H, D] tensor. This is a
user-selectable backend (the reference's default), not a fallback of the HIP
backend.
"""
from __future__ import annotations

import math

import torch

from .kv_block_pool import KVBlockPool


def _online_step(m, l, O, scores, values):
    """One online-softmax fold of a block of scores [.., T] and values [.., T, D].

    Keeps O normalised: O' = (alpha * l * O + sum_t p_t v_t) / l'.
    """
    m_new = torch.maximum(m, scores.max(dim=-1).values)
    alpha = torch.exp(m - m_new)
    p = torch.exp(scores - m_new[..., None])
    l_new = alpha * l + p.sum(dim=-1)
    O_new = (alpha[..., None] * l[..., None] * O + (p[..., None, :] @ values).squeeze(-2)) / l_new[..., None]
    return m_new, l_new, O_new


def paged_attention_batch_reference(q: torch.Tensor, pool: KVBlockPool, block_tables: torch.Tensor,
                                    context_lengths: torch.Tensor, layer_idx: int) -> torch.Tensor:
    B, H, D = q.shape
    S = pool.block_size
    scale = 1.0 / math.sqrt(D)
    rows = []
    for b in range(B):
        ctx = int(context_lengths[b].item())
        assert ctx > 0
        m = torch.full((H,), float("-inf"), device=q.device, dtype=q.dtype)
        l = torch.zeros(H, device=q.device, dtype=q.dtype)
        O = torch.zeros(H, D, device=q.device, dtype=q.dtype)
        for logical in range((ctx + S - 1) // S):
            physical = int(block_tables[b, logical].item())
            assert physical >= 0
            n = min(S, ctx - logical * S)
            keys = pool.k[layer_idx, physical, :n].transpose(0, 1).contiguous()    # [H, n, D]
            values = pool.v[layer_idx, physical, :n].transpose(0, 1).contiguous()  # [H, n, D]
            scores = (keys @ q[b][..., None]).squeeze(-1) * scale     # [H, n]
            m, l, O = _online_step(m, l, O, scores, values)
        rows.append(O)
    return torch.stack(rows, dim=0)


def paged_attention_batch_online_v1(q: torch.Tensor, pool: KVBlockPool, block_tables: torch.Tensor,
                                    context_lengths: torch.Tensor, layer_idx: int) -> torch.Tensor:
    B, H, D = q.shape
    S = pool.block_size
    scale = 1.0 / math.sqrt(D)
    M = block_tables.shape[1]
    m = torch.full((B, H), float("-inf"), device=q.device, dtype=q.dtype)
    l = torch.zeros(B, H, device=q.device, dtype=q.dtype)
    O = torch.zeros(B, H, D, device=q.device, dtype=q.dtype)
    slot_ids = torch.arange(S, device=q.device)
    for logical in range(M):
        blocks = block_tables[:, logical].clamp(min=0)
        keys = pool.k[layer_idx, blocks].permute(0, 2, 1, 3)    # [B, H, S, D]
        values = pool.v[layer_idx, blocks].permute(0, 2, 1, 3)  # [B, H, S, D]
        n_valid = (context_lengths - logical * S).clamp(min=0, max=S)
        valid = slot_ids[None, :] < n_valid[:, None]            # [B, S]
        # Unwritten slots may hold NaN: zero them before any product.
        keys = torch.where(valid[:, None, :, None], keys, torch.zeros_like(keys)).contiguous()
        values = torch.where(valid[:, None, :, None], values, torch.zeros_like(values)).contiguous()
        scores = (keys @ q[..., None]).squeeze(-1)              # [B, H, S]
        scores = scores.masked_fill(~valid[:, None, :], float("-inf")) * scale
        m_blk = scores.max(dim=-1).values
        m_new = torch.maximum(m, m_blk)
        alpha = torch.exp(m - m_new)
        p = torch.exp(scores - m_new[..., None])
        p = torch.where(valid[:, None, :], p, torch.zeros_like(p))
        l_new = alpha * l + p.sum(dim=-1)
        O_new = (alpha[..., None] * l[..., None] * O + (p[..., None, :] @ values).squeeze(-2)) / l_new[..., None]
        active = n_valid > 0
        m = torch.where(active[:, None], m_new, m)
        l = torch.where(active[:, None], l_new, l)
        O = torch.where(active[:, None, None], O_new, O)
    return O
