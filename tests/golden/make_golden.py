#!/usr/bin/env python3
"""Write the golden fixtures that only the reference itself can pin.

Two properties of the reference are fixed by its RNG consumption order and by nothing the
mathematics can check: (1) the default-initialised weights that ``torch.manual_seed(s)`` followed by
``BaselineTransformer(config)`` produces (module construction order,
benchmarks/torch_transformer_benchmark.py:62-75,126-132,149-160), and (2) the ``(x, mask)`` pair
``generate_random_case`` draws (:234-272).  This script imports the reference module in the build
container (it is never present on the GPU box), evaluates those two functions on tiny shapes, and
stores inputs and outputs as plain arrays in ``reference_init_and_inputs.npz``.  Nothing of the
reference's source is stored.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import importlib.util
import pathlib
import sys

import numpy as np
import torch

REF = pathlib.Path("/root/reference/benchmarks/torch_transformer_benchmark.py")
OUT = pathlib.Path(__file__).with_name("reference_init_and_inputs.npz")

# (name, batch, seq, d_model, heads, ffn, layers, causal, seed, padding_ratio)
CASES = [
    ("tiny_causal", 2, 6, 16, 2, 24, 2, True, 1234, 0.5),
    ("tiny_noncausal", 3, 5, 8, 2, 32, 1, False, 77, 0.0),
]


def main() -> int:
    spec = importlib.util.spec_from_file_location("reference_benchmark", REF)
    ref = importlib.util.module_from_spec(spec)
    sys.modules["reference_benchmark"] = ref
    spec.loader.exec_module(ref)
    arrays = {}
    for name, b, s, d, h, f, layers, causal, seed, pad in CASES:
        cfg = ref.TransformerConfig(batch_size=b, seq_len=s, d_model=d, num_heads=h, ffn_dim=f,
                                    num_layers=layers, causal=causal)
        torch.manual_seed(seed)
        model = ref.BaselineTransformer(cfg)
        for key, value in model.state_dict().items():
            arrays[f"{name}/param/{key}"] = value.detach().numpy().astype(np.float32)
        x, mask = ref.generate_random_case(cfg, torch.device("cpu"), torch.float32,
                                           seed=seed + 1, padding_ratio=pad, input_scale=1.0)
        arrays[f"{name}/x"] = x.numpy().astype(np.float32)
        arrays[f"{name}/mask"] = mask.numpy().astype(np.bool_)
        arrays[f"{name}/meta"] = np.array([b, s, d, h, f, layers, int(causal), seed], np.int64)
        arrays[f"{name}/padding_ratio"] = np.array([pad], np.float64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({len(arrays)} arrays)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
