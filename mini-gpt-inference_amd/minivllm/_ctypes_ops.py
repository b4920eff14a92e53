"""The eager path's four calls through ctypes, for when the _hip_ops
extension (csrc/torch_ops.cpp) cannot be loaded but libminivllm_hip.so can,
for example after a PyTorch update that the extension was not rebuilt for.

Same functions, arguments, checks (in the same order), exception types and
messages as the extension; the checks follow paged_attention_batch_triton_v0
(minivllm/triton_paged_decode.py:109-144). Outputs and workspaces come from
PyTorch's caching allocator, and the C ABI runs on the current HIP stream,
so results are bit-identical to the extension's. Only the host cost per call
differs (the argument marshalling: about 9 against 5 us).
"""
from __future__ import annotations

import math

import torch

from . import _native

_FLOATS = (torch.float32, torch.bfloat16, torch.float16)
_INDEX = (torch.int32, torch.int64)


def _check_pool(kp: torch.Tensor, vp: torch.Tensor) -> None:
    if kp.ndim != 5 or vp.shape != kp.shape:
        raise ValueError("KV tensors must have matching [L,P,S,H,D] shape")


def kv_append(kp: torch.Tensor, vp: torch.Tensor, layer_idx: int, k: torch.Tensor, v: torch.Tensor,
              slots: torch.Tensor) -> None:
    """Rows k[t], v[t] into pool slots slots[t] (negative slots skipped)."""
    if not kp.is_cuda:
        raise ValueError("KV pool must be on a GPU device for the HIP backend")
    if k.ndim != 3 or v.shape != k.shape:
        raise ValueError("k and v must have matching shape [T,H,D]")
    _check_pool(kp, vp)
    L, N, S, H, D = kp.shape
    T = k.shape[0]
    if S <= 0:
        raise ValueError("block_size must be positive")
    if k.shape[1] != H or k.shape[2] != D:
        raise ValueError("k/v head dimensions do not match the KV pool")
    if kp.dtype not in _FLOATS or vp.dtype != kp.dtype:
        raise ValueError("KV pool must be float32, bfloat16 or float16")
    if k.dtype not in _FLOATS or v.dtype != k.dtype:
        raise ValueError("k and v must share a float dtype")
    if slots.ndim != 1 or slots.shape[0] != T:
        raise ValueError("slot_mapping must have shape [T]")
    if slots.dtype not in _INDEX:
        raise ValueError("slot_mapping must contain integer slots")
    if not 0 <= layer_idx < L:
        raise ValueError("layer_idx outside KV pool")
    if any(x.device != kp.device for x in (vp, k, v, slots)):
        raise ValueError("all inputs must reside on same GPU device")
    if T == 0:
        return
    lib = _native.lib()
    _native.check(lib.mgi_kv_append(
        kp.data_ptr(), vp.data_ptr(), _native.strides(kp), _native.strides(vp), _native.DTYPE_CODES[kp.dtype],
        k.data_ptr(), v.data_ptr(), _native.strides(k), _native.strides(v), _native.DTYPE_CODES[k.dtype],
        slots.data_ptr(), slots.stride(0), _native.ITYPE_CODES[slots.dtype],
        T, H, D, S, N, L, int(layer_idx), _native.stream_handle(kp.device)))


def _check_decode(q: torch.Tensor, kp: torch.Tensor, vp: torch.Tensor, bt: torch.Tensor, cl: torch.Tensor,
                  layer_idx: int) -> int:
    """paged_decode's checks; returns the block-table width M."""
    if not q.is_cuda:
        raise ValueError("q must be on a GPU device for the HIP backend")
    if q.ndim != 3:
        raise ValueError("q must have shape [B,H,D]")
    b, h, d = q.shape
    if b == 0 or h == 0 or d == 0:
        raise ValueError("q dimensions must be nonzero")
    if d > 512:
        raise ValueError("HIP backend supports head_dim <= 512")
    if q.dtype not in _FLOATS:
        raise ValueError("q must be float32, bfloat16 or float16")
    if kp.dtype != q.dtype or vp.dtype != q.dtype:
        raise ValueError("KV pool dtype must match q dtype")
    _check_pool(kp, vp)
    L, N, S = kp.shape[:3]
    if S <= 0:
        raise ValueError("block_size must be positive")
    if kp.shape[3] != h or kp.shape[4] != d:
        raise ValueError("KV head dimensions or block size do not match q")
    if bt.ndim != 2 or bt.shape[0] != b:
        raise ValueError("block_tables must have shape [B,M]")
    if cl.ndim != 1 or cl.shape[0] != b:
        raise ValueError("context_lengths must have shape [B]")
    if bt.dtype not in _INDEX:
        raise ValueError("block_tables must contain integer indices")
    if cl.dtype not in _INDEX:
        raise ValueError("context_lengths must be integer")
    if not 0 <= layer_idx < L:
        raise ValueError("layer_idx outside KV pool")
    if any(x.device != q.device for x in (kp, vp, bt, cl)):
        raise ValueError("all inputs must reside on same GPU device")
    M = bt.shape[1]
    if M < 1:
        raise ValueError("block_tables need at least one block column")
    return M


def paged_decode(q: torch.Tensor, kp: torch.Tensor, vp: torch.Tensor, bt: torch.Tensor, cl: torch.Tensor,
                 layer_idx: int, split_tokens: int) -> torch.Tensor:
    """[B, H, D] decode attention output of q's dtype."""
    M = _check_decode(q, kp, vp, bt, cl, layer_idx)
    b, h, d = q.shape
    L, N, S = kp.shape[:3]
    lib = _native.lib()
    out = torch.empty((b, h, d), dtype=q.dtype, device=q.device)
    ws_bytes = int(lib.mgi_paged_decode_workspace_bytes(b, h, d, S, M, int(split_tokens)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    _native.check(lib.mgi_paged_decode(
        out.data_ptr(), _native.strides(out), q.data_ptr(), _native.strides(q),
        kp.data_ptr(), vp.data_ptr(), _native.strides(kp), _native.strides(vp), _native.DTYPE_CODES[q.dtype],
        bt.data_ptr(), _native.strides(bt), _native.ITYPE_CODES[bt.dtype],
        cl.data_ptr(), cl.stride(0), _native.ITYPE_CODES[cl.dtype],
        b, h, d, S, N, M, L, int(layer_idx), 1.0 / math.sqrt(d), int(split_tokens),
        ws.data_ptr() if ws is not None else None, ws_bytes, _native.stream_handle(q.device)))
    return out


def paged_decode_append(q: torch.Tensor, kp: torch.Tensor, vp: torch.Tensor, bt: torch.Tensor,
                        cl: torch.Tensor, layer_idx: int, k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor,
                        split_tokens: int) -> torch.Tensor:
    """kv_append of the B rows k[b], v[b] into slots[b], then paged_decode, as one call."""
    M = _check_decode(q, kp, vp, bt, cl, layer_idx)
    b, h, d = q.shape
    L, N, S = kp.shape[:3]
    if k.ndim != 3 or v.shape != k.shape:
        raise ValueError("k and v must have matching shape [T,H,D]")
    if k.shape[0] != b:
        raise ValueError("k and v must hold one row per sequence")
    if k.shape[1] != h or k.shape[2] != d:
        raise ValueError("k/v head dimensions do not match the KV pool")
    if k.dtype not in _FLOATS or v.dtype != k.dtype:
        raise ValueError("k and v must share a float dtype")
    if slots.ndim != 1 or slots.shape[0] != b:
        raise ValueError("slot_mapping must have shape [B]")
    if slots.dtype not in _INDEX:
        raise ValueError("slot_mapping must contain integer slots")
    if any(x.device != q.device for x in (k, v, slots)):
        raise ValueError("all inputs must reside on same GPU device")
    lib = _native.lib()
    out = torch.empty((b, h, d), dtype=q.dtype, device=q.device)
    ws_bytes = int(lib.mgi_paged_decode_workspace_bytes(b, h, d, S, M, int(split_tokens)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    _native.check(lib.mgi_paged_decode_append(
        out.data_ptr(), _native.strides(out), q.data_ptr(), _native.strides(q),
        kp.data_ptr(), vp.data_ptr(), _native.strides(kp), _native.strides(vp), _native.DTYPE_CODES[q.dtype],
        k.data_ptr(), v.data_ptr(), _native.strides(k), _native.strides(v), _native.DTYPE_CODES[k.dtype],
        slots.data_ptr(), slots.stride(0), _native.ITYPE_CODES[slots.dtype],
        bt.data_ptr(), _native.strides(bt), _native.ITYPE_CODES[bt.dtype],
        cl.data_ptr(), cl.stride(0), _native.ITYPE_CODES[cl.dtype],
        b, h, d, S, N, M, L, int(layer_idx), 1.0 / math.sqrt(d), int(split_tokens),
        ws.data_ptr() if ws is not None else None, ws_bytes, _native.stream_handle(q.device)))
    return out


def paged_prefill(q: torch.Tensor, kp: torch.Tensor, vp: torch.Tensor, bt: torch.Tensor, start_pos: int,
                  layer_idx: int) -> torch.Tensor:
    """[T, H, D] causal attention of a chunk's rows over the pool."""
    if not q.is_cuda:
        raise ValueError("q must be on a GPU device for the HIP backend")
    if q.ndim != 3:
        raise ValueError("q must have shape [T,H,D]")
    t, h, d = q.shape
    if h == 0 or d == 0:
        raise ValueError("q dimensions must be nonzero")
    if d > 512:
        raise ValueError("HIP backend supports head_dim <= 512")
    if q.dtype not in _FLOATS:
        raise ValueError("q must be float32, bfloat16 or float16")
    if kp.dtype != q.dtype or vp.dtype != q.dtype:
        raise ValueError("KV pool dtype must match q dtype")
    _check_pool(kp, vp)
    L, N, S = kp.shape[:3]
    if S <= 0:
        raise ValueError("block_size must be positive")
    if kp.shape[3] != h or kp.shape[4] != d:
        raise ValueError("KV head dimensions do not match q")
    if bt.ndim != 1 or bt.dtype not in _INDEX:
        raise ValueError("block_table must be a 1-D integer tensor")
    if start_pos < 0:
        raise ValueError("start_pos must be non-negative")
    if bt.shape[0] < (start_pos + t + S - 1) // S:
        raise ValueError("block_table shorter than ceil((start_pos + T) / S)")
    if not 0 <= layer_idx < L:
        raise ValueError("layer_idx outside KV pool")
    if any(x.device != q.device for x in (kp, vp, bt)):
        raise ValueError("all inputs must reside on same GPU device")
    out = torch.empty((t, h, d), dtype=q.dtype, device=q.device)
    if t == 0:
        return out
    lib = _native.lib()
    code = _native.DTYPE_CODES[q.dtype]
    ws_bytes = int(lib.mgi_paged_prefill_workspace_bytes(int(start_pos), t, h, d, code))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    _native.check(lib.mgi_paged_prefill(
        out.data_ptr(), _native.strides(out), q.data_ptr(), _native.strides(q),
        kp.data_ptr(), vp.data_ptr(), _native.strides(kp), _native.strides(vp), code,
        bt.data_ptr(), bt.stride(0), _native.ITYPE_CODES[bt.dtype], bt.shape[0], int(start_pos), t,
        h, d, S, N, L, int(layer_idx), 1.0 / math.sqrt(d),
        ws.data_ptr() if ws is not None else None, ws_bytes, _native.stream_handle(q.device)))
    return out
