"""MI355X-native (gfx950) optimized forward pass for the pre-LN transformer block stack.

Drop-in for the reference's ``make_optimized_transformer(model)`` / ``forward(x, valid_token_mask)``
(optimized_transformer.py:69-93): hand-written HIP kernels behind a C ABI (include/tttj_amd.h),
loaded with ctypes; PyTorch-ROCm provides device memory and streams.
"""

from .model import BaselineTransformer, TransformerConfig
from .optimized_transformer import (
    PLAN_AUTO,
    PLAN_FUSED_LN,
    PLAN_LAYERWISE,
    PLAN_MEGAKERNEL,
    IMPLEMENTED_CASE_LAYERS,
    IMPLEMENTED_CASES,
    GraphedOptimizedTransformer,
    OptimizedTransformer,
    case_number_for_model,
    check_supported,
    make_optimized_transformer,
    pack_model_weights,
)

__all__ = [
    "BaselineTransformer",
    "TransformerConfig",
    "OptimizedTransformer",
    "GraphedOptimizedTransformer",
    "make_optimized_transformer",
    "pack_model_weights",
    "check_supported",
    "case_number_for_model",
    "IMPLEMENTED_CASES",
    "IMPLEMENTED_CASE_LAYERS",
    "PLAN_AUTO",
    "PLAN_LAYERWISE",
    "PLAN_MEGAKERNEL",
    "PLAN_FUSED_LN",
]
