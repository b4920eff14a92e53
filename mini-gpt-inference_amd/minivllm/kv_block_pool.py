"""Physical paged KV storage.

API of minivllm/kv_block_pool.py:32-152 (KVBlockPool): two tensors ``k`` and
``v`` of shape [n_layer, num_blocks, block_size, n_head, head_dim], created
with ``torch.empty`` (contents start undefined, so every reader must mask
slots past a sequence's length). Element strides are therefore
(N*S*H*D, S*H*D, H*D, D, 1): one physical block of one layer is a
contiguous [S, H, D] slab, and one token of one layer is a contiguous [H, D]
row -- the layout the HIP kernels read in place.
"""
from __future__ import annotations

import torch

from .sequence import SequenceState


def make_kv(seq_tag: int, logical_pos: int, n_layer: int, n_head: int, head_dim: int):
    """Deterministic per-(sequence, position) K/V of shape [n_layer, n_head, head_dim].

    Same values as minivllm/kv_block_pool.py:5-29: an arange pattern offset by
    ``seq_tag * 10000 + logical_pos * 100`` (V is K + 0.5).
    """
    base = torch.arange(n_layer * n_head * head_dim, dtype=torch.float32)
    base = base.reshape(n_layer, n_head, head_dim)
    shift = seq_tag * 10000 + logical_pos * 100
    return base + shift, base + (shift + 0.5)


class KVBlockPool:
    def __init__(self, n_layer: int, num_blocks: int, block_size: int, n_head: int,
                 head_dim: int, device="cpu", dtype=torch.float32):
        self.n_layer = n_layer
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.n_head = n_head
        self.head_dim = head_dim
        self.dtype = dtype
        shape = (n_layer, num_blocks, block_size, n_head, head_dim)
        self.k = torch.empty(shape, dtype=dtype, device=device)
        self.v = torch.empty(shape, dtype=dtype, device=device)

    @property
    def device(self) -> torch.device:
        return self.k.device

    def write(self, physical_block: int, block_offset: int, k_new: torch.Tensor,
              v_new: torch.Tensor) -> None:
        """Writes one token slot in every layer; k_new/v_new are [L, H, D]."""
        expected = (self.n_layer, self.n_head, self.head_dim)
        assert tuple(k_new.shape) == expected
        assert tuple(v_new.shape) == expected
        self.k[:, physical_block, block_offset].copy_(k_new)
        self.v[:, physical_block, block_offset].copy_(v_new)

    def write_layer(self, layer_idx: int, physical_block: int, block_offset: int,
                    k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Writes one token slot of one layer; k_new/v_new are [H, D]."""
        self.k[layer_idx, physical_block, block_offset].copy_(k_new)
        self.v[layer_idx, physical_block, block_offset].copy_(v_new)

    def gather_sequence(self, seq: SequenceState) -> tuple[torch.Tensor, torch.Tensor]:
        """Logical K/V of `seq` on the host: two [L, seq.length, H, D] tensors."""
        length = seq.length
        S = self.block_size
        k_out = torch.empty((self.n_layer, length, self.n_head, self.head_dim), dtype=self.dtype)
        v_out = torch.empty_like(k_out)
        for logical, physical in enumerate(seq.block_table):
            lo = logical * S
            hi = min(lo + S, length)
            if hi <= lo:
                break
            k_out[:, lo:hi].copy_(self.k[:, physical, : hi - lo])
            v_out[:, lo:hi].copy_(self.v[:, physical, : hi - lo])
        return k_out, v_out
