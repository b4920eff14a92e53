"""KV-aware MiniGPT (minivllm/model.py:16-283).

Modules are created in the reference's order (token embedding, position
embedding, blocks, final LayerNorm, LM head) with the same shapes and
attribute names, so a given torch seed yields the same weights and the
reference's state dicts load unchanged.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor, nn
from torch.utils.checkpoint import checkpoint

from .attention import DECODE_BACKENDS, PREFILL_MODES, KVCache
from .block import TransformerBlock
from .decode_batch_metadata import DecodeBatchMetadata
from .kv_block_pool import KVBlockPool
from .kv_runtime import KVRuntimeContext, PrefillChunkContext, PrefillRuntimeContext


class MiniGPT(nn.Module):
    def __init__(self, n_embd: int, n_head: int, vocab_size: int, block_size: int,
                 dropout: float = 0.0, n_layer: int = 1, enable_activation_checkpointing: bool = False):
        super().__init__()
        self.block_size = block_size
        self.vocab_size = vocab_size
        self.n_layer = n_layer
        self.token_embedding_table = nn.Embedding(num_embeddings=vocab_size, embedding_dim=n_embd)
        self.position_embedding_table = nn.Embedding(num_embeddings=block_size, embedding_dim=n_embd)
        self.blocks = nn.Sequential(*[TransformerBlock(n_embd=n_embd, n_head=n_head, block_size=block_size,
                                                       dropout=dropout) for _ in range(n_layer)])
        self.layer_norm = nn.LayerNorm(n_embd)
        self.language_model_head = nn.Linear(n_embd, vocab_size)
        self.enable_activation_checkpointing = enable_activation_checkpointing

    # -------------------------------------------------------- backend knobs

    def set_prefill_fastpath(self, enabled: bool) -> None:
        """First-chunk SDPA only (the v1 boolean API)."""
        if not isinstance(enabled, bool):
            raise TypeError("enabled must be bool")
        for block in self.blocks:
            block.attn.prefill_fastpath_enabled = enabled
            block.attn.prefill_prefix_fastpath_enabled = False
            block.attn.prefill_hip = False

    def set_prefill_fastpath_mode(self, mode: str) -> None:
        """'reference', 'sdpa_v1' (first chunk), 'sdpa_v2' (prefix-aware) or
        'hip' (every chunk through the paged prefill kernel of
        libminivllm_hip.so, any model dtype; GPU only)."""
        if mode not in PREFILL_MODES:
            raise ValueError("mode must be reference, sdpa_v1, sdpa_v2 or hip")
        for block in self.blocks:
            block.attn.prefill_fastpath_enabled = mode != "reference"
            block.attn.prefill_prefix_fastpath_enabled = mode in ("sdpa_v2", "hip")
            block.attn.prefill_hip = mode == "hip"

    def set_decode_attention_backend(self, backend: str) -> None:
        """'reference' (PyTorch) or 'hip' (MI355X kernels; 'triton_v0' is an alias).

        Constraints of the HIP backend (GPU tensors, supported dtypes) are
        validated at dispatch and never bypassed.
        """
        if backend not in DECODE_BACKENDS:
            raise ValueError("decode backend must be reference, hip or triton_v0")
        for block in self.blocks:
            block.attn.decode_attention_backend = backend

    # ------------------------------------------------------------ execution

    def _embed(self, input_ids: Tensor, positions: Tensor) -> Tensor:
        return self.token_embedding_table(input_ids) + self.position_embedding_table(positions)

    def _head(self, x: Tensor) -> Tensor:
        return self.language_model_head(self.layer_norm(x))

    def forward(self, idx: Tensor, kv_caches: list[KVCache] | None = None, targets: Tensor | None = None):
        """Dense full-sequence forward with optional contiguous KV caches."""
        B, T = idx.shape
        past = kv_caches[0].length if kv_caches is not None else 0
        if past + T > self.block_size:
            raise ValueError(f"sequence length {past + T} exceeds block_size {self.block_size}")
        x = self._embed(idx, torch.arange(past, past + T, device=idx.device))
        for i, block in enumerate(self.blocks):
            if self.enable_activation_checkpointing and self.training and torch.is_grad_enabled():
                x = checkpoint(block, x, use_reentrant=False, preserve_rng_state=True)
                continue
            if kv_caches is None:
                x = block(x)
            else:
                a = block.attn(block.layer_norm_1(x), kv_cache=kv_caches[i])
                x = block._mlp(x + a)
        logits = self._head(x)
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.reshape(B * T, -1), targets.reshape(B * T))
        return logits, loss

    def prefill(self, input_ids: Tensor, contexts: list[PrefillRuntimeContext]) -> Tensor:
        T = input_ids.shape[1]
        start = contexts[0].start_pos
        x = self._embed(input_ids, torch.arange(start, start + T, device=input_ids.device))
        for i, block in enumerate(self.blocks):
            x = block.forward_prefill(x, contexts[i])
        return self._head(x)

    def prefill_chunk(self, input_ids: Tensor, contexts: list[PrefillChunkContext]) -> Tensor:
        T = input_ids.shape[1]
        start = contexts[0].start_pos
        x = self._embed(input_ids, torch.arange(start, start + T, device=input_ids.device))
        for i, block in enumerate(self.blocks):
            x = block.forward_prefill_chunk(x, contexts[i])
        return self._head(x)

    def decode_batch(self, input_ids: Tensor, metadata: DecodeBatchMetadata, kv_pool: KVBlockPool) -> Tensor:
        """One batched decode step: input_ids [B, 1] -> logits [B, 1, vocab]."""
        x = self._embed(input_ids, metadata.positions.unsqueeze(1))
        for i, block in enumerate(self.blocks):
            x = block.forward_decode_batch(x, metadata=metadata, kv_pool=kv_pool, layer_idx=i)
        return self._head(x)

    def decode(self, input_ids: Tensor, contexts: list[KVRuntimeContext]) -> Tensor:
        assert len(contexts) == self.n_layer
        pos = torch.tensor([[contexts[0].logical_pos]], device=input_ids.device, dtype=torch.long)
        x = self._embed(input_ids, pos)
        for i, block in enumerate(self.blocks):
            x = block.forward_decode(x, contexts[i])
        return self._head(x)
