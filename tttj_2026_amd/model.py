"""Caller-side model contract: the pre-LN block stack whose forward this package replaces.

``make_optimized_transformer`` accepts any ``nn.Module`` shaped like the organizer model in
``benchmarks/torch_transformer_benchmark.py:29-172``: a ``.config`` with the seven fields of
``TransformerConfig`` and the parameter tree ``layers.{i}.norm1 / attention.{q,k,v,out}_proj /
norm2 / ffn_in / ffn_out`` plus ``final_norm``.  This module provides that type for callers who do
not have the organizer file, with the same field names, parameter names and module-construction
order (so that ``torch.manual_seed(s)`` followed by construction yields the same default-initialised
weights).  Its ``forward`` is the eager PyTorch path: it is the baseline the optimized module is
timed against, not part of the optimized path.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass(frozen=True)
class TransformerConfig:
    """Shape contract of the block stack (torch_transformer_benchmark.py:29-56)."""

    batch_size: int
    seq_len: int
    d_model: int
    num_heads: int
    ffn_dim: int
    num_layers: int
    causal: bool

    def validate(self) -> None:
        for name in ("batch_size", "seq_len", "d_model", "num_heads", "ffn_dim", "num_layers"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.d_model % self.num_heads != 0:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by num_heads ({self.num_heads})"
            )

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    @property
    def tokens(self) -> int:
        return self.batch_size * self.seq_len


class BaselineSelfAttention(nn.Module):
    """Multi-head self-attention with explicit masks (torch_transformer_benchmark.py:59-122).

    Construction order q, k, v, out matters for seeded initialisation (:72-75).
    """

    def __init__(self, d_model: int, num_heads: int) -> None:
        super().__init__()
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_proj = nn.Linear(d_model, d_model, bias=True)
        self.k_proj = nn.Linear(d_model, d_model, bias=True)
        self.v_proj = nn.Linear(d_model, d_model, bias=True)
        self.out_proj = nn.Linear(d_model, d_model, bias=True)

    def _heads(self, t: torch.Tensor) -> torch.Tensor:
        b, s, _ = t.shape
        return t.reshape(b, s, self.num_heads, self.head_dim).permute(0, 2, 1, 3).contiguous()

    def forward(
        self,
        x: torch.Tensor,
        valid_token_mask: Optional[torch.Tensor] = None,
        causal: bool = False,
    ) -> torch.Tensor:
        b, s, _ = x.shape
        q, k, v = (self._heads(p(x)) for p in (self.q_proj, self.k_proj, self.v_proj))
        # Eager semantics (:97-117): scores in the activation dtype, scaled, masked with -inf,
        # softmax in fp32, probabilities cast back, then P.V.
        scores = torch.matmul(q, k.transpose(-2, -1)) * self.scale
        if causal:
            upper = torch.ones((s, s), device=x.device, dtype=torch.bool).triu(diagonal=1)
            scores = scores.masked_fill(upper, float("-inf"))
        if valid_token_mask is not None:
            scores = scores.masked_fill(~valid_token_mask[:, None, None, :], float("-inf"))
        probs = torch.softmax(scores.float(), dim=-1).to(x.dtype)
        ctx = torch.matmul(probs, v).permute(0, 2, 1, 3).reshape(b, s, self.d_model)
        out = self.out_proj(ctx)
        if valid_token_mask is not None:
            out = out.masked_fill(~valid_token_mask[..., None], 0)
        return out


class BaselineTransformerBlock(nn.Module):
    """Pre-LN block (torch_transformer_benchmark.py:125-145); construction order :128-132."""

    def __init__(self, d_model: int, num_heads: int, ffn_dim: int) -> None:
        super().__init__()
        self.norm1 = nn.LayerNorm(d_model)
        self.attention = BaselineSelfAttention(d_model, num_heads)
        self.norm2 = nn.LayerNorm(d_model)
        self.ffn_in = nn.Linear(d_model, ffn_dim)
        self.ffn_out = nn.Linear(ffn_dim, d_model)

    def forward(self, x, valid_token_mask, causal):
        x = x + self.attention(self.norm1(x), valid_token_mask, causal)
        x = x + self.ffn_out(F.gelu(self.ffn_in(self.norm2(x)), approximate="none"))
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x


class BaselineTransformer(nn.Module):
    """Block stack + final LayerNorm (torch_transformer_benchmark.py:148-172)."""

    def __init__(self, config: TransformerConfig) -> None:
        super().__init__()
        config.validate()
        self.config = config
        self.layers = nn.ModuleList(
            BaselineTransformerBlock(config.d_model, config.num_heads, config.ffn_dim)
            for _ in range(config.num_layers)
        )
        self.final_norm = nn.LayerNorm(config.d_model)

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None):
        for layer in self.layers:
            x = layer(x, valid_token_mask, self.config.causal)
        x = self.final_norm(x)
        if valid_token_mask is not None:
            x = x.masked_fill(~valid_token_mask[..., None], 0)
        return x
