"""The five benchmark workloads and their seeded synthetic inputs.

Input protocol (deliberately host-generated so every provider sees identical bits):
``torch.manual_seed(1234)`` then the model is built on the CPU in fp32 (default nn.Linear /
nn.LayerNorm init), the GPU copy is ``.half()``.  ``x`` is drawn from a CPU ``torch.Generator``
seeded with ``1234 + index`` and quantised to fp16.  Masked workloads draw right-padded prefix
lengths ``l ~ U{S/2 .. S}`` from the same generator and zero ``x`` at padded rows, as
``generate_random_case`` does (benchmarks/torch_transformer_benchmark.py:234-272).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Optional, Tuple

import torch

from .model import BaselineTransformer, TransformerConfig

SEED = 1234


@dataclass(frozen=True)
class Workload:
    name: str
    config: TransformerConfig
    masked: bool          # right-padded valid_token_mask with l ~ U{S/2..S}
    description: str


def _cfg(b, s, d, h, f, l, causal):
    return TransformerConfig(batch_size=b, seq_len=s, d_model=d, num_heads=h, ffn_dim=f,
                             num_layers=l, causal=causal)


WORKLOADS: Dict[str, Workload] = {
    "C1": Workload("C1", _cfg(4, 128, 256, 4, 1024, 2, False), False,
                   "2 layers, D256 H4 (hd64) F1024, B4 S128, non-causal, no mask"),
    "C2": Workload("C2", _cfg(1, 64, 256, 8, 1024, 4, True), False,
                   "4 layers, D256 H8 (hd32) F1024, B1 S64, causal, no mask"),
    "C3": Workload("C3", _cfg(8, 512, 512, 8, 2048, 6, False), True,
                   "6 layers, D512 H8 (hd64) F2048, B8 S512, non-causal, right-padded mask"),
    "C4": Workload("C4", _cfg(8, 1024, 1024, 16, 4096, 8, True), True,
                   "8 layers, D1024 H16 (hd64) F4096, B8 S1024, causal, right-padded mask"),
    "C5": Workload("C5", _cfg(2, 4096, 1024, 16, 4096, 12, True), False,
                   "12 layers, D1024 H16 (hd64) F4096, B2 S4096, causal, no mask"),
}
WORKLOAD_ORDER = ("C1", "C2", "C3", "C4", "C5")

# The reference's own shape table (optimized_transformer.py:22-42): case -> (batch, seq, d_model,
# heads); every case is causal with ffn_dim = d_model and 4 layers (2 for case 14).  The HIP path
# is not limited to these shapes; they are parity and timing cases.
REFERENCE_CASES: Dict[int, Tuple[int, int, int, int]] = {
    1: (64, 128, 128, 4), 2: (1, 128, 128, 4), 3: (4, 128, 128, 4), 4: (16, 128, 128, 4),
    5: (128, 128, 128, 4), 6: (10000, 128, 128, 4), 7: (64, 128, 32, 4), 8: (64, 128, 1024, 4),
    9: (64, 128, 128, 1), 10: (64, 128, 128, 2), 11: (64, 128, 128, 16), 12: (64, 32, 128, 4),
    13: (64, 1024, 128, 4), 14: (32, 100000, 1024, 16),
}
REFERENCE_CASE_LAYERS: Dict[int, int] = {n: 2 if n == 14 else 4 for n in REFERENCE_CASES}


def reference_case_config(case: int, batch: Optional[int] = None,
                          seq: Optional[int] = None) -> TransformerConfig:
    """TransformerConfig of reference case ``case`` (optionally with a smaller batch / seq)."""
    b, s, d, h = REFERENCE_CASES[case]
    return _cfg(b if batch is None else batch, s if seq is None else seq, d, h, d,
                REFERENCE_CASE_LAYERS[case], True)


def build_model(config: TransformerConfig, seed: int = SEED) -> BaselineTransformer:
    """Seeded fp32 CPU model in reference construction order (regression.py:30-44)."""
    torch.manual_seed(seed)
    return BaselineTransformer(config).eval()


def make_inputs(config: TransformerConfig, masked: bool, seed: int,
                min_valid: Optional[int] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Return ``(x16, mask)`` on the CPU: x fp16 ``[B,S,D]``, mask bool ``[B,S]`` or ``None``."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=gen)
    mask = None
    if masked:
        lo = config.seq_len // 2 if min_valid is None else min_valid
        lengths = torch.randint(lo, config.seq_len + 1, (config.batch_size,), generator=gen)
        mask = torch.arange(config.seq_len)[None, :] < lengths[:, None]
        x = x.masked_fill(~mask[..., None], 0)
    return x.half(), mask


def workload_inputs(name: str) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    w = WORKLOADS[name]
    return make_inputs(w.config, w.masked, SEED + 1 + WORKLOAD_ORDER.index(name))
