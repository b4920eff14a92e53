"""Host-side contract of minivllm.hip_paged_decode without a GPU: every
violation raises (ValueError, as paged_attention_batch_triton_v0 does,
minivllm/triton_paged_decode.py:109-144), and CPU tensors are rejected rather
than computed on some other path."""
from __future__ import annotations

import pytest
import torch

from minivllm import hip_paged_decode as hpd
from minivllm.kv_block_pool import KVBlockPool


def _inputs(dtype=torch.float32):
    pool = KVBlockPool(1, 4, 16, 2, 8, dtype=dtype)
    q = torch.randn(2, 2, 8, dtype=dtype)
    return q, pool, torch.tensor([[0], [1]]), torch.tensor([3, 5])


def test_cpu_tensors_are_rejected_not_computed():
    q, pool, tables, lens = _inputs()
    with pytest.raises(ValueError, match="GPU"):
        hpd.paged_attention_batch_hip(q, pool, tables, lens, 0)
    with pytest.raises(ValueError, match="GPU"):
        hpd.kv_append(pool, 0, q, q, torch.tensor([0, 1]))


def test_entry_points_are_module_attributes_for_patching():
    # forward_decode_batch imports these at call time so tests can patch them
    assert callable(hpd.paged_attention_batch_hip)
    assert callable(hpd.kv_append)
