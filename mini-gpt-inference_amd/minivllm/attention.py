"""KV-cache causal self-attention of MiniGPT (minivllm/attention.py).

The decode hot path is ``forward_decode_batch`` (minivllm/attention.py:349-424):
QKV projection -> KV append of the new token into the paged pool -> paged
decode attention -> output projection. The KV append completes before the
attention reads the pool (same stream). The decode backend is chosen by name:

  "reference"          PyTorch: index_put_ KV write + paged_attention_batch_online_v1
  "hip" / "triton_v0"  HIP kernels through libminivllm_hip.so: the KV append
                       and paged_attention_batch_hip as one call
                       (paged_attention_batch_append_hip, which writes the
                       new K/V inside the attention launch where it can), or
                       as kv_append then paged_attention_batch_hip when
                       ``fused_decode_append`` is False ("triton_v0" is
                       accepted so callers that select the reference's Triton
                       backend by name run the HIP kernels)

With a HIP backend, prefill KV writes go through the same kv_append kernel
(one launch per chunk instead of a per-token copy loop). Both HIP entry
points are imported at call time from minivllm.hip_paged_decode, so tests can
patch them there. A HIP backend never falls back: CPU tensors or a missing
library raise.

Prefill attention (``set_prefill_fastpath_mode``): "reference" attends each
query token through the pool with paged_attention_online; "sdpa_v1" /
"sdpa_v2" use scaled_dot_product_attention over the chunk (and, for v2, the
gathered cached prefix) with an absolute-position causal mask. The SDPA
paths run in float32 for every model dtype. "hip" runs every chunk (first or
later) through the paged prefill kernel of libminivllm_hip.so, which reads
the cached prefix and the chunk straight from the pool after the chunk's
KV append (minivllm.hip_paged_decode.paged_prefill_hip, imported at call
time); it needs the model and pool on a GPU and raises otherwise.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from .decode_batch_metadata import DecodeBatchMetadata
from .kv_block_pool import KVBlockPool
from .kv_runtime import KVRuntimeContext, PrefillChunkContext, PrefillRuntimeContext
from .paged_attention_batch import paged_attention_batch_online_v1
from .paged_attention_v1_reference import paged_attention_online

DECODE_BACKENDS = ("reference", "hip", "triton_v0")
HIP_BACKENDS = ("hip", "triton_v0")
PREFILL_MODES = ("reference", "sdpa_v1", "sdpa_v2", "hip")


@dataclass
class KVCache:
    k: Tensor
    v: Tensor
    length: int


def create_kv_cache(batch_size, n_head, block_size, head_size, device, dtype) -> KVCache:
    shape = (batch_size, n_head, block_size, head_size)
    return KVCache(k=torch.empty(shape, device=device, dtype=dtype),
                   v=torch.empty(shape, device=device, dtype=dtype), length=0)


def write_kv_rows(pool: KVBlockPool, layer_idx: int, k: Tensor, v: Tensor, slots: Tensor,
                  use_hip: bool) -> None:
    """pool[layer, slot // S, slot % S] = row for every row with slot >= 0.

    k, v: [T, H, D]; slots: [T] integer tensor on the pool's device.
    """
    if use_hip:
        from .hip_paged_decode import kv_append

        kv_append(pool, layer_idx, k, v, slots)
        return
    if slots.numel() and not bool((slots >= 0).all()):
        keep = slots >= 0
        slots, k, v = slots[keep], k[keep], v[keep]
    S = pool.block_size
    blocks = torch.div(slots, S, rounding_mode="floor")
    offsets = slots % S
    pool.k[layer_idx, blocks, offsets] = k.to(pool.dtype)
    pool.v[layer_idx, blocks, offsets] = v.to(pool.dtype)


class KVCacheCausalSelfAttention(nn.Module):
    def __init__(self, n_embd: int, n_head: int, block_size: int, dropout: float = 0.0):
        super().__init__()
        if n_embd % n_head != 0:
            raise ValueError(f"n_embd {n_embd} is not divisible by n_head {n_head}")
        self.n_embd = n_embd
        self.n_head = n_head
        self.head_size = n_embd // n_head
        self.block_size = block_size
        self.dropout = dropout
        self.prefill_fastpath_enabled = False
        self.prefill_prefix_fastpath_enabled = False
        self.prefill_hip = False
        self.decode_attention_backend = "reference"
        # HIP backends: append and attend in one call (see the module docstring).
        self.fused_decode_append = True
        self.qkv = nn.Linear(n_embd, 3 * n_embd, bias=False)
        self.register_buffer("tril", torch.tril(torch.ones(block_size, block_size)))
        self.attn_dropout = nn.Dropout(dropout)
        self.project = nn.Linear(n_embd, n_embd)
        self.resid_dropout = nn.Dropout(dropout)

    # ------------------------------------------------------------- helpers

    @property
    def _hip(self) -> bool:
        return self.decode_attention_backend in HIP_BACKENDS

    def _qkv_heads(self, x: Tensor):
        """[B, T, C] -> q, k, v as [B, T, H, D] views of one projection output."""
        B, T, C = x.shape
        q, k, v = self.qkv(x).split(C, dim=-1)
        shape = (B, T, self.n_head, self.head_size)
        return q.view(shape), k.view(shape), v.view(shape)

    def _finish(self, out: Tensor) -> Tensor:
        return self.resid_dropout(self.project(out))

    def _write_chunk_kv(self, k: Tensor, v: Tensor, pool: KVBlockPool, layer_idx: int,
                        slot_mapping) -> None:
        slots = torch.as_tensor(slot_mapping, dtype=torch.long, device=pool.k.device)
        write_kv_rows(pool, layer_idx, k, v, slots, use_hip=self._hip)

    def _dense_prefill(self, q: Tensor, k: Tensor, v: Tensor, start: int, pool: KVBlockPool,
                       seq, layer_idx: int) -> Tensor:
        """Causal attention of chunk queries (positions start..start+T-1) over the
        cached prefix [0, start) and the chunk itself; float32 arithmetic."""
        _, T, H, D = q.shape
        keys, values = k, v
        if start > 0:
            S = pool.block_size
            n_blocks = (start + S - 1) // S
            ids = seq.block_table[:n_blocks]
            if len(ids) != n_blocks:
                raise RuntimeError("incomplete KV block table for prefix")
            idx = torch.tensor(ids, device=q.device, dtype=torch.long)
            prefix_k = pool.k[layer_idx].index_select(0, idx).reshape(-1, H, D)[:start]
            prefix_v = pool.v[layer_idx].index_select(0, idx).reshape(-1, H, D)[:start]
            keys = torch.cat((prefix_k[None].to(k.dtype), k), dim=1)
            values = torch.cat((prefix_v[None].to(v.dtype), v), dim=1)
        q_pos = start + torch.arange(T, device=q.device)
        k_pos = torch.arange(start + T, device=q.device)
        mask = k_pos[None, :] <= q_pos[:, None]
        out = F.scaled_dot_product_attention(
            q.transpose(1, 2).float().contiguous(), keys.transpose(1, 2).float().contiguous(),
            values.transpose(1, 2).float().contiguous(), attn_mask=mask, dropout_p=0.0)
        return out.transpose(1, 2).reshape(1, T, H * D).to(q.dtype)

    def _hip_prefill(self, q: Tensor, start: int, pool: KVBlockPool, seq, layer_idx: int,
                     table: Tensor | None) -> Tensor:
        """Chunk queries [1, T, H, D] at positions start.. through the paged
        prefill kernel; the chunk's KV is already in the pool."""
        from .hip_paged_decode import paged_prefill_hip

        _, T, H, D = q.shape
        if torch.is_grad_enabled() and q.requires_grad:
            raise RuntimeError("hip prefill is inference-only; run under torch.inference_mode()")
        if table is None:
            n_blocks = -(-(start + T) // pool.block_size)
            ids = seq.block_table[:n_blocks]
            if len(ids) != n_blocks:
                raise RuntimeError("incomplete KV block table for prefix")
            table = torch.tensor(ids, dtype=torch.long, device=q.device)
        out = paged_prefill_hip(q[0], pool, table, start, layer_idx)
        return out.reshape(1, T, H * D)

    # ------------------------------------------------------------- prefill

    def forward_prefill(self, x: Tensor, context: PrefillRuntimeContext) -> Tensor:
        """Whole-prompt prefill (B == 1) from position 0."""
        B, T, C = x.shape
        assert B == 1
        assert len(context.slot_mapping) == T
        q, k, v = self._qkv_heads(x)
        self._write_chunk_kv(k[0], v[0], context.kv_pool, context.layer_idx, context.slot_mapping)
        if self.prefill_hip:
            if context.start_pos != 0:
                raise ValueError("whole-prompt prefill starts at position 0")
            out = self._hip_prefill(q, 0, context.kv_pool, context.seq_state,
                                    context.layer_idx, context.block_table)
            return self._finish(out)
        out = self._dense_prefill(q, k, v, 0, context.kv_pool, context.seq_state, context.layer_idx)
        return self._finish(out)

    def forward_prefill_chunk(self, x: Tensor, context: PrefillChunkContext) -> Tensor:
        B, T, C = x.shape
        assert B == 1
        assert T == context.num_tokens
        q, k, v = self._qkv_heads(x)
        pool, layer = context.kv_pool, context.layer_idx
        self._write_chunk_kv(k[0], v[0], pool, layer, context.slot_mapping)
        start = context.start_pos
        if self.prefill_hip:
            out = self._hip_prefill(q, start, pool, context.seq_state, layer, context.block_table)
            return self._finish(out)
        if self.prefill_fastpath_enabled and (start == 0 or self.prefill_prefix_fastpath_enabled):
            out = self._dense_prefill(q, k, v, start, pool, context.seq_state, layer)
            return self._finish(out)
        rows = [paged_attention_online(q=q[0, i], pool=pool, seq=context.seq_state, layer_idx=layer,
                                       context_length=start + i + 1) for i in range(T)]
        out = torch.stack(rows, dim=0).reshape(1, T, C)
        return self._finish(out)

    # -------------------------------------------------------------- decode

    def forward_decode(self, x: Tensor, kv_context: KVRuntimeContext | None = None) -> Tensor:
        """Serial one-token decode (B == 1) of one sequence."""
        B, T, C = x.shape
        assert B == 1 and T == 1
        q, k, v = self._qkv_heads(x)
        ctx = kv_context
        slots = torch.tensor([ctx.physical_slot], dtype=torch.long, device=ctx.kv_pool.k.device)
        write_kv_rows(ctx.kv_pool, ctx.layer_idx, k[0], v[0], slots, use_hip=self._hip)
        out = paged_attention_online(q=q[0, 0], pool=ctx.kv_pool, seq=ctx.seq_state,
                                     layer_idx=ctx.layer_idx, context_length=ctx.context_length)
        return self._finish(out.reshape(1, 1, C))

    def forward_decode_batch(self, x: Tensor, metadata: DecodeBatchMetadata, kv_pool: KVBlockPool,
                             layer_idx: int) -> Tensor:
        B, T, C = x.shape
        assert T == 1
        q, k, v = self._qkv_heads(x)
        q, k, v = q[:, 0], k[:, 0], v[:, 0]            # [B, H, D], row stride 3C
        backend = self.decode_attention_backend
        if backend == "reference":
            write_kv_rows(kv_pool, layer_idx, k, v, metadata.slot_mapping, use_hip=False)
            out = paged_attention_batch_online_v1(q=q, pool=kv_pool, block_tables=metadata.block_tables,
                                                  context_lengths=metadata.context_lengths,
                                                  layer_idx=layer_idx)
        elif backend in HIP_BACKENDS:
            if torch.is_grad_enabled() and q.requires_grad:
                raise RuntimeError(f"{backend} is inference-only; run under torch.inference_mode()")
            from . import hip_paged_decode as hpd

            if self.fused_decode_append:
                # Row b's new K/V is sequence b's last token: the fused call's contract.
                out = hpd.paged_attention_batch_append_hip(q, kv_pool, metadata.block_tables,
                                                           metadata.context_lengths, layer_idx, k, v,
                                                           metadata.slot_mapping)
            else:
                # The new token's K/V must be in the pool before attention reads it.
                hpd.kv_append(kv_pool, layer_idx, k, v, metadata.slot_mapping)
                out = hpd.paged_attention_batch_hip(q=q, pool=kv_pool, block_tables=metadata.block_tables,
                                                    context_lengths=metadata.context_lengths,
                                                    layer_idx=layer_idx)
        else:
            raise ValueError(f"unknown decode attention backend: {backend}")
        return self._finish(out.reshape(B, 1, C))

    # -------------------------------------------------- dense (no paging)

    def forward(self, x: Tensor, kv_cache: KVCache | None = None) -> Tensor:
        """Dense causal attention over an optional contiguous KVCache."""
        B, T, C = x.shape
        past = 0 if kv_cache is None else kv_cache.length
        if past + T > self.block_size:
            raise ValueError(f"sequence length {past + T} exceeds block_size {self.block_size}")
        if kv_cache is not None and past + T > kv_cache.k.size(2):
            raise ValueError(f"KV cache capacity exceeded: end={past + T}, capacity={kv_cache.k.size(2)}")
        q, k, v = (t.transpose(1, 2) for t in self._qkv_heads(x))   # [B, H, T, D]
        if kv_cache is not None:
            kv_cache.k[:, :, past:past + T].copy_(k)
            kv_cache.v[:, :, past:past + T].copy_(v)
            k, v = kv_cache.k[:, :, :past + T], kv_cache.v[:, :, :past + T]
            kv_cache.length = past + T
        att = (q @ k.transpose(-2, -1).contiguous()) * (1.0 / math.sqrt(self.head_size))
        if kv_cache is not None or T > 1:
            att = att.masked_fill(self.tril[past:past + T, :past + T] == 0, float("-inf"))
        att = self.attn_dropout(F.softmax(att, dim=-1))
        out = (att @ v.contiguous()).transpose(1, 2).reshape(B, T, C)
        return self._finish(out)
