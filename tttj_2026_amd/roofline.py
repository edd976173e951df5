"""Algorithmic FLOP and byte accounting for the forward pass (FMA = 2 FLOPs, fp16 = 2 bytes).

Per layer: ``8*T*D^2 + 4*T*D*F + 4*D*sum_b P_b`` with ``P_b = l_b^2`` (non-causal) or
``l_b (l_b + 1) / 2`` (causal), ``T`` the token count.  "Dense" uses ``l_b = S`` for every
sequence; "useful" uses the valid lengths of a right-padded mask, so skipped padded work is never
counted as done.
"""

from __future__ import annotations

from typing import Optional, Sequence

from .model import TransformerConfig

MI355X_FP16_DENSE_TFLOPS = 2516.6   # 256 CUs x 4 SIMDs x 1024 FLOP/clk x 2.4 GHz
MI355X_HBM_GBPS = 8000.0


def _pairs(length: int, causal: bool) -> int:
    return length * (length + 1) // 2 if causal else length * length


def layer_flops(cfg: TransformerConfig, lengths: Optional[Sequence[int]] = None) -> dict:
    lens = [cfg.seq_len] * cfg.batch_size if lengths is None else list(lengths)
    t = sum(lens)
    d, f = cfg.d_model, cfg.ffn_dim
    pairs = sum(_pairs(l, cfg.causal) for l in lens)
    out = {
        "qkv": 2 * t * d * 3 * d,
        "out_proj": 2 * t * d * d,
        "ffn_in": 2 * t * d * f,
        "ffn_out": 2 * t * f * d,
        "attention": 4 * d * pairs,
    }
    out["gemm"] = out["qkv"] + out["out_proj"] + out["ffn_in"] + out["ffn_out"]
    out["total"] = out["gemm"] + out["attention"]
    return out


def forward_flops(cfg: TransformerConfig, lengths: Optional[Sequence[int]] = None) -> int:
    return cfg.num_layers * layer_flops(cfg, lengths)["total"]


def param_count(cfg: TransformerConfig) -> int:
    d, f = cfg.d_model, cfg.ffn_dim
    per_layer = 4 * d + 4 * (d * d + d) + (f * d + f) + (d * f + d)
    return cfg.num_layers * per_layer + 2 * d


def min_bytes(cfg: TransformerConfig) -> int:
    """Weights once + x in + y out (+ a byte mask), fp16."""
    t = cfg.tokens
    return 2 * param_count(cfg) + 2 * 2 * t * cfg.d_model + t


def layernorm_bytes(rows: int, d: int) -> int:
    """Standalone LayerNorm: read x, write y (fp16), read gamma and beta."""
    return 2 * rows * d * 2 + 2 * d * 2


def gemm_bytes(m: int, n: int, k: int, residual: bool) -> int:
    """Compulsory traffic of Y = X W^T (+b) (+residual): X, W, b, Y (and the residual) once."""
    return 2 * (m * k + n * k + n + m * n + (m * n if residual else 0))
