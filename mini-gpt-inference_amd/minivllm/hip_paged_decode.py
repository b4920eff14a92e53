"""MI355X HIP paged KV backend: fused decode attention, KV append and paged
prefill attention.

Drop-in for minivllm/triton_paged_decode.py. Inputs match
paged_attention_batch_online_v1:
    q:               [B, H, D] (arbitrary strides)
    pool.k / pool.v: [L, N, S, H, D]
    block_tables:    [B, M] (logical -> physical; -1 only in the unused tail)
    context_lengths: [B] (>= 1, include the KV written this step)

Both entry points validate on the host exactly like
paged_attention_batch_triton_v0 (minivllm/triton_paged_decode.py:109-144):
ValueError for contract violations, RuntimeError when the HIP library or its
PyTorch binding is unavailable. The checks, allocations and launches run in
the binding (csrc/torch_ops.cpp), which calls the C ABI of
libminivllm_hip.so. Nothing reads device data on the host (no .item()); the
kernels launch on torch's current stream, so the KV append is ordered before
the attention that reads it. There is no fallback: without the library or a
GPU these functions raise.

Beyond the Triton v0 backend: float32, bfloat16 and float16; head_dim up to
512; any block size; a split of long and ragged contexts over many
wavefronts (all sequences' blocks dealt out evenly) with a merge pass.

paged_prefill_hip is the prefill counterpart (the reference's per-token
loop, minivllm/attention.py:269-299, and its sdpa_v2 gather,
minivllm/attention.py:229-267): causal attention of one chunk's queries over
the sequence's cached prefix and the chunk itself, read from the pool.
"""
from __future__ import annotations

import torch

from . import _native
from .kv_block_pool import KVBlockPool


def paged_attention_batch_hip(q: torch.Tensor, pool: KVBlockPool, block_tables: torch.Tensor,
                              context_lengths: torch.Tensor, layer_idx: int, *,
                              split_tokens: int = 0) -> torch.Tensor:
    """One fused decode-attention pass over the paged pool; caller already wrote new KV.

    Returns a fresh [B, H, D] tensor of q.dtype. ``split_tokens`` = 0 lets
    the library split the work (evenly over a fixed number of wavefronts
    when contexts span several partitions); > 0 cuts every context into
    partitions of that many tokens.

    Validation (ValueError, the messages of the Triton v0 backend's checks),
    allocation and the launch happen in the _hip_ops binding
    (csrc/torch_ops.cpp).
    """
    return _native.ops().paged_decode(q, pool.k, pool.v, block_tables, context_lengths, int(layer_idx),
                                      int(split_tokens))


def paged_attention_batch_append_hip(q: torch.Tensor, pool: KVBlockPool, block_tables: torch.Tensor,
                                     context_lengths: torch.Tensor, layer_idx: int, k: torch.Tensor,
                                     v: torch.Tensor, slot_mapping: torch.Tensor, *,
                                     split_tokens: int = 0) -> torch.Tensor:
    """One decode step's KV write and attention as one call: kv_append of the
    B rows k[b], v[b] ([B, H, D]) into slot_mapping[b], then
    paged_attention_batch_hip, on the current stream.

    Where the library can (bf16/f16/f32 rows of the pool's dtype, head dim
    contiguous, 16-byte aligned, the fast attention path) the write runs inside
    the attention launch, by the wavefront that streams each sequence's last
    block, before it reads that block: one launch fewer per layer. The pool and
    the output are bit-identical to the two calls, given the decode step's
    invariant that a slot some context reads is the slot of its own row's last
    position (``context_lengths[b] - 1``); negative slots are skipped.
    """
    return _native.ops().paged_decode_append(q, pool.k, pool.v, block_tables, context_lengths, int(layer_idx),
                                             k, v, slot_mapping, int(split_tokens))


def kv_append(pool: KVBlockPool, layer_idx: int, k: torch.Tensor, v: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
    """Scatters rows k[t], v[t] ([T, H, D], any strides) into pool slots slot_mapping[t].

    pool.k[layer, s // S, s % S] = k[t] (same for v) for every s >= 0; rows
    with a negative slot are skipped. Bit-exact when k/v share the pool dtype.
    """
    _native.ops().kv_append(pool.k, pool.v, int(layer_idx), k, v, slot_mapping)


def paged_prefill_hip(q: torch.Tensor, pool: KVBlockPool, block_table: torch.Tensor,
                      start_pos: int, layer_idx: int) -> torch.Tensor:
    """Causal attention of a chunk's queries through the paged pool.

    q: [T, H, D] (any strides), query row t at absolute position start_pos + t.
    block_table: [n] integer tensor of the sequence's physical blocks,
    n >= ceil((start_pos + T) / S). The chunk's own K/V must already be in
    the pool (kv_append on the same stream). Returns a fresh [T, H, D]
    tensor of q.dtype with out[t] = softmax(q[t] K[0..start_pos+t]^T / sqrt(D)) V.
    """
    return _native.ops().paged_prefill(q, pool.k, pool.v, block_table, int(start_pos), int(layer_idx))
