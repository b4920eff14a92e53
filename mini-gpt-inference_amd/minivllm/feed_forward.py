"""Position-wise MLP (minivllm/feed_forward.py:3-28): Linear(C, 4C) -> GELU ->
Linear(4C, C) -> Dropout. Dense GEMMs stay on PyTorch (hipBLASLt)."""
from __future__ import annotations

from torch import Tensor, nn


class FeedForward(nn.Module):
    def __init__(self, n_embd: int, dropout: float = 0.0):
        super().__init__()
        if n_embd <= 0:
            raise ValueError("n_embd must be > 0")
        if not 0.0 <= dropout <= 1.0:
            raise ValueError("dropout must be in [0, 1]")
        self.network = nn.Sequential(
            nn.Linear(n_embd, 4 * n_embd),
            nn.GELU(),
            nn.Linear(4 * n_embd, n_embd),
            nn.Dropout(dropout),
        )

    def forward(self, x: Tensor) -> Tensor:
        return self.network(x)
