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
    with pytest.raises(ValueError, match="GPU"):
        hpd.paged_prefill_hip(q, pool, torch.tensor([0, 1]), 0, 0)


def test_hip_prefill_mode_on_cpu_raises_instead_of_falling_back():
    from minivllm.block_manager import BlockManager
    from minivllm.model import MiniGPT
    from minivllm.model_runner import ModelRunner
    from minivllm.sequence import SequenceState

    torch.manual_seed(0)
    model = MiniGPT(n_embd=32, n_head=4, vocab_size=64, block_size=64, n_layer=1).eval()
    model.set_prefill_fastpath_mode("hip")
    bm = BlockManager(8, 4)
    pool = KVBlockPool(1, 8, 4, 4, 8)
    runner = ModelRunner(model, pool, bm)
    seq = SequenceState(seq_id="s", prompt_tokens=list(range(1, 10)), max_tokens=12)
    with torch.inference_mode(), pytest.raises(ValueError, match="GPU"):
        runner.prefill_chunk(seq, 0, 9)


def test_unknown_prefill_mode_is_rejected():
    from minivllm.model import MiniGPT

    model = MiniGPT(n_embd=32, n_head=4, vocab_size=64, block_size=64, n_layer=1)
    with pytest.raises(ValueError, match="mode must be"):
        model.set_prefill_fastpath_mode("flash")


def test_entry_points_are_module_attributes_for_patching():
    # forward_decode_batch / forward_prefill_chunk import these at call time
    # so tests can patch them
    assert callable(hpd.paged_attention_batch_hip)
    assert callable(hpd.kv_append)
    assert callable(hpd.paged_prefill_hip)
