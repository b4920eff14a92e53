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
ValueError for contract violations, RuntimeError when the HIP library is
unavailable. Nothing reads device data on the host (no .item()); the kernels
launch on torch's current stream, so the KV append is ordered before the
attention that reads it. There is no fallback: without the library or a GPU
these functions raise.

Beyond the Triton v0 backend: float32, bfloat16 and float16; head_dim up to
512; any block size; a split of long and ragged contexts over many
wavefronts (all sequences' blocks dealt out evenly) with a merge pass.

paged_prefill_hip is the prefill counterpart (the reference's per-token
loop, minivllm/attention.py:269-299, and its sdpa_v2 gather,
minivllm/attention.py:229-267): causal attention of one chunk's queries over
the sequence's cached prefix and the chunk itself, read from the pool.
"""
from __future__ import annotations

import math

import torch

from . import _native
from .kv_block_pool import KVBlockPool

_FLOATS = (torch.float32, torch.bfloat16, torch.float16)
_INDEX = (torch.int32, torch.int64)


def _check_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{what} must be on a GPU device for the HIP backend")


def paged_attention_batch_hip(q: torch.Tensor, pool: KVBlockPool, block_tables: torch.Tensor,
                              context_lengths: torch.Tensor, layer_idx: int, *,
                              split_tokens: int = 0) -> torch.Tensor:
    """One fused decode-attention pass over the paged pool; caller already wrote new KV.

    Returns a fresh [B, H, D] tensor of q.dtype. ``split_tokens`` = 0 lets
    the library split the work (evenly over a fixed number of wavefronts
    when contexts span several partitions); > 0 cuts every context into
    partitions of that many tokens.
    """
    lib = _native.lib()
    _check_device(q, "q")
    if q.ndim != 3:
        raise ValueError("q must have shape [B,H,D]")
    b, h, d = q.shape
    if b == 0 or h == 0 or d == 0:
        raise ValueError("q dimensions must be nonzero")
    if d > 512:
        raise ValueError("HIP backend supports head_dim <= 512")
    s = pool.block_size
    if s <= 0:
        raise ValueError("block_size must be positive")
    if q.dtype not in _FLOATS:
        raise ValueError("q must be float32, bfloat16 or float16")
    if pool.k.dtype != q.dtype or pool.v.dtype != q.dtype:
        raise ValueError("KV pool dtype must match q dtype")
    if pool.k.ndim != 5 or pool.v.shape != pool.k.shape:
        raise ValueError("KV tensors must have matching [L,P,S,H,D] shape")
    if tuple(pool.k.shape[2:]) != (s, h, d):
        raise ValueError("KV head dimensions or block size do not match q")
    if block_tables.ndim != 2 or block_tables.shape[0] != b:
        raise ValueError("block_tables must have shape [B,M]")
    if tuple(context_lengths.shape) != (b,):
        raise ValueError("context_lengths must have shape [B]")
    if block_tables.dtype not in _INDEX:
        raise ValueError("block_tables must contain integer indices")
    if context_lengths.dtype not in _INDEX:
        raise ValueError("context_lengths must be integer")
    if not 0 <= layer_idx < pool.k.shape[0]:
        raise ValueError("layer_idx outside KV pool")
    if any(x.device != q.device for x in (pool.k, pool.v, block_tables, context_lengths)):
        raise ValueError("all inputs must reside on same GPU device")
    if block_tables.shape[1] < 1:
        raise ValueError("block_tables need at least one block column")

    L, N, S, H, D = pool.k.shape
    M = block_tables.shape[1]
    out = torch.empty((b, h, d), dtype=q.dtype, device=q.device)
    ws_bytes = int(lib.mgi_paged_decode_workspace_bytes(b, h, d, S, M, int(split_tokens)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    status = lib.mgi_paged_decode(
        out.data_ptr(), _native.strides(out),
        q.data_ptr(), _native.strides(q),
        pool.k.data_ptr(), pool.v.data_ptr(), _native.strides(pool.k), _native.strides(pool.v),
        _native.DTYPE_CODES[q.dtype],
        block_tables.data_ptr(), _native.strides(block_tables), _native.ITYPE_CODES[block_tables.dtype],
        context_lengths.data_ptr(), context_lengths.stride(0),
        _native.ITYPE_CODES[context_lengths.dtype],
        b, h, d, S, N, M, L, int(layer_idx),
        1.0 / math.sqrt(d), int(split_tokens),
        ws.data_ptr() if ws is not None else None, ws_bytes,
        _native.stream_handle(q.device),
    )
    _native.check(status)
    return out


def kv_append(pool: KVBlockPool, layer_idx: int, k: torch.Tensor, v: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
    """Scatters rows k[t], v[t] ([T, H, D], any strides) into pool slots slot_mapping[t].

    pool.k[layer, s // S, s % S] = k[t] (same for v) for every s >= 0; rows
    with a negative slot are skipped. Bit-exact when k/v share the pool dtype.
    """
    lib = _native.lib()
    _check_device(pool.k, "KV pool")
    if k.ndim != 3 or v.shape != k.shape:
        raise ValueError("k and v must have matching shape [T,H,D]")
    T, h, d = k.shape
    if pool.k.ndim != 5 or pool.v.shape != pool.k.shape:
        raise ValueError("KV tensors must have matching [L,P,S,H,D] shape")
    L, N, S, H, D = pool.k.shape
    if (h, d) != (H, D):
        raise ValueError("k/v head dimensions do not match the KV pool")
    if pool.k.dtype not in _FLOATS or pool.v.dtype != pool.k.dtype:
        raise ValueError("KV pool must be float32, bfloat16 or float16")
    if k.dtype not in _FLOATS or v.dtype != k.dtype:
        raise ValueError("k and v must share a float dtype")
    if slot_mapping.ndim != 1 or slot_mapping.shape[0] != T:
        raise ValueError("slot_mapping must have shape [T]")
    if slot_mapping.dtype not in _INDEX:
        raise ValueError("slot_mapping must contain integer slots")
    if not 0 <= layer_idx < L:
        raise ValueError("layer_idx outside KV pool")
    if any(x.device != pool.k.device for x in (pool.v, k, v, slot_mapping)):
        raise ValueError("all inputs must reside on same GPU device")
    if T == 0:
        return
    status = lib.mgi_kv_append(
        pool.k.data_ptr(), pool.v.data_ptr(), _native.strides(pool.k), _native.strides(pool.v),
        _native.DTYPE_CODES[pool.k.dtype],
        k.data_ptr(), v.data_ptr(), _native.strides(k), _native.strides(v),
        _native.DTYPE_CODES[k.dtype],
        slot_mapping.data_ptr(), slot_mapping.stride(0), _native.ITYPE_CODES[slot_mapping.dtype],
        T, H, D, S, N, L, int(layer_idx),
        _native.stream_handle(pool.k.device),
    )
    _native.check(status)


def paged_prefill_hip(q: torch.Tensor, pool: KVBlockPool, block_table: torch.Tensor,
                      start_pos: int, layer_idx: int) -> torch.Tensor:
    """Causal attention of a chunk's queries through the paged pool.

    q: [T, H, D] (any strides), query row t at absolute position start_pos + t.
    block_table: [n] integer tensor of the sequence's physical blocks,
    n >= ceil((start_pos + T) / S). The chunk's own K/V must already be in
    the pool (kv_append on the same stream). Returns a fresh [T, H, D]
    tensor of q.dtype with out[t] = softmax(q[t] K[0..start_pos+t]^T / sqrt(D)) V.
    """
    lib = _native.lib()
    _check_device(q, "q")
    if q.ndim != 3:
        raise ValueError("q must have shape [T,H,D]")
    t, h, d = q.shape
    if h == 0 or d == 0:
        raise ValueError("q dimensions must be nonzero")
    if d > 512:
        raise ValueError("HIP backend supports head_dim <= 512")
    if q.dtype not in _FLOATS:
        raise ValueError("q must be float32, bfloat16 or float16")
    if pool.k.dtype != q.dtype or pool.v.dtype != q.dtype:
        raise ValueError("KV pool dtype must match q dtype")
    if pool.k.ndim != 5 or pool.v.shape != pool.k.shape:
        raise ValueError("KV tensors must have matching [L,P,S,H,D] shape")
    L, N, S, H, D = pool.k.shape
    if (H, D) != (h, d):
        raise ValueError("KV head dimensions do not match q")
    if block_table.ndim != 1 or block_table.dtype not in _INDEX:
        raise ValueError("block_table must be a 1-D integer tensor")
    if start_pos < 0:
        raise ValueError("start_pos must be non-negative")
    if block_table.shape[0] < -(-(start_pos + t) // S):
        raise ValueError("block_table shorter than ceil((start_pos + T) / S)")
    if not 0 <= layer_idx < L:
        raise ValueError("layer_idx outside KV pool")
    if any(x.device != q.device for x in (pool.k, pool.v, block_table)):
        raise ValueError("all inputs must reside on same GPU device")
    out = torch.empty((t, h, d), dtype=q.dtype, device=q.device)
    if t == 0:
        return out
    ws_bytes = int(lib.mgi_paged_prefill_workspace_bytes(int(start_pos), t, h, d, _native.DTYPE_CODES[q.dtype]))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    status = lib.mgi_paged_prefill(
        out.data_ptr(), _native.strides(out),
        q.data_ptr(), _native.strides(q),
        pool.k.data_ptr(), pool.v.data_ptr(), _native.strides(pool.k), _native.strides(pool.v),
        _native.DTYPE_CODES[q.dtype],
        block_table.data_ptr(), block_table.stride(0), _native.ITYPE_CODES[block_table.dtype],
        block_table.shape[0], int(start_pos), t,
        h, d, S, N, L, int(layer_idx),
        1.0 / math.sqrt(d),
        ws.data_ptr() if ws is not None else None, ws_bytes,
        _native.stream_handle(q.device),
    )
    _native.check(status)
    return out
