"""Pre-LN transformer block of MiniGPT (minivllm/block.py:6-102):
x + attn(LN1(x)), then x + ffn(LN2(x)), for each execution mode."""
from __future__ import annotations

from torch import Tensor, nn

from .attention import KVCacheCausalSelfAttention
from .decode_batch_metadata import DecodeBatchMetadata
from .feed_forward import FeedForward
from .kv_block_pool import KVBlockPool
from .kv_runtime import KVRuntimeContext, PrefillChunkContext, PrefillRuntimeContext


class TransformerBlock(nn.Module):
    def __init__(self, n_embd: int, n_head: int, block_size: int, dropout: float = 0.0):
        super().__init__()
        if n_embd <= 0:
            raise ValueError("n_embd must be > 0")
        if n_head <= 0:
            raise ValueError("n_head must be > 0")
        self.attn = KVCacheCausalSelfAttention(n_embd, n_head, block_size, dropout)
        self.ffn = FeedForward(n_embd, dropout)
        self.layer_norm_1 = nn.LayerNorm(n_embd)
        self.layer_norm_2 = nn.LayerNorm(n_embd)

    def _mlp(self, x: Tensor) -> Tensor:
        return x + self.ffn(self.layer_norm_2(x))

    def forward_prefill(self, x: Tensor, context: PrefillRuntimeContext) -> Tensor:
        return self._mlp(x + self.attn.forward_prefill(self.layer_norm_1(x), context))

    def forward_prefill_chunk(self, x: Tensor, context: PrefillChunkContext) -> Tensor:
        return self._mlp(x + self.attn.forward_prefill_chunk(self.layer_norm_1(x), context))

    def forward_decode(self, x: Tensor, kv_context: KVRuntimeContext) -> Tensor:
        return self._mlp(x + self.attn.forward_decode(self.layer_norm_1(x), kv_context=kv_context))

    def forward_decode_batch(self, x: Tensor, metadata: DecodeBatchMetadata, kv_pool: KVBlockPool,
                             layer_idx: int) -> Tensor:
        h = self.attn.forward_decode_batch(self.layer_norm_1(x), metadata=metadata, kv_pool=kv_pool,
                                           layer_idx=layer_idx)
        return self._mlp(x + h)

    def forward(self, x: Tensor) -> Tensor:
        return self._mlp(x + self.attn(self.layer_norm_1(x)))
