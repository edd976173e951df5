#!/usr/bin/env python3
"""Write the golden fixtures that only the reference itself can pin.

Three properties of the reference are fixed by its own code and by nothing the mathematics can
check: (1) the default-initialised weights that ``torch.manual_seed(s)`` followed by
``BaselineTransformer(config)`` produces (module construction order,
benchmarks/torch_transformer_benchmark.py:62-75,126-132,149-160), (2) the ``(x, mask)`` pair
``generate_random_case`` draws (:234-272), and (3) what ``BaselineTransformer.forward``
(:85-172) returns for given weights, inputs and mask -- the residual order, the points where
padded rows are zeroed and the mask semantics.  This script imports the reference module in the
build container (it is never present on the GPU box), evaluates those functions on tiny shapes,
and stores inputs and outputs as plain arrays in ``reference_init_and_inputs.npz``.  Nothing of
the reference's source is stored.

Cases beyond the first two give the forward non-default LayerNorm affine parameters (default
init, weight 1 and bias 0, hides affine mistakes) and masks the reference's generator does not
draw: a non-prefix mask and a fully padded sequence.  For those the weights used by the forward
are stored under ``{case}/fwd_param/`` and the forward's inputs under ``{case}/fwd_x`` /
``{case}/fwd_mask``; ``{case}/param/`` always holds the seeded default init and ``{case}/x`` /
``{case}/mask`` the generator's own draw.
The forward is evaluated in float32 (``y_fp32``) and on a float64 copy of the module
(``y_fp64``), both in eval mode without gradients.

Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import copy
import importlib.util
import pathlib
import sys

import numpy as np
import torch

REF = pathlib.Path("/root/reference/benchmarks/torch_transformer_benchmark.py")
OUT = pathlib.Path(__file__).with_name("reference_init_and_inputs.npz")

# (name, batch, seq, d_model, heads, ffn, layers, causal, seed, padding_ratio, extra)
# extra: None, or (ln_perturb_seed, mask kind) with mask kind "generated" (generate_random_case's
# own prefix mask), "nonprefix" (holes inside each sequence, key 0 always valid) or
# "empty_seq" (generated prefix mask with the last sequence fully padded).
CASES = [
    ("tiny_causal", 2, 6, 16, 2, 24, 2, True, 1234, 0.5, None),
    ("tiny_noncausal", 3, 5, 8, 2, 32, 1, False, 77, 0.0, None),
    ("masked_noncausal_ln", 3, 7, 16, 4, 40, 2, False, 2024, 0.6, (31, "empty_seq")),
    ("nonprefix_causal_ln", 2, 8, 16, 2, 24, 2, True, 4242, 0.0, (32, "nonprefix")),
]


def _perturb_layer_norms(model: torch.nn.Module, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.add_(0.3 * torch.randn(p.shape, generator=g, dtype=p.dtype))


def _nonprefix_mask(batch: int, seq: int) -> torch.Tensor:
    mask = torch.ones(batch, seq, dtype=torch.bool)
    for b in range(batch):
        for s in range(1, seq):
            if (3 * s + b) % 5 == 2:  # a few holes per sequence; key 0 stays valid
                mask[b, s] = False
    return mask


def main() -> int:
    spec = importlib.util.spec_from_file_location("reference_benchmark", REF)
    ref = importlib.util.module_from_spec(spec)
    sys.modules["reference_benchmark"] = ref
    spec.loader.exec_module(ref)
    arrays = {}
    for name, b, s, d, h, f, layers, causal, seed, pad, extra in CASES:
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
        if extra is not None:
            ln_seed, kind = extra
            _perturb_layer_norms(model, ln_seed)
            for key, value in model.state_dict().items():
                arrays[f"{name}/fwd_param/{key}"] = value.detach().numpy().astype(np.float32)
            if kind == "nonprefix":
                mask = _nonprefix_mask(b, s)
                x = x.masked_fill(~mask[..., None], 0)
            elif kind == "empty_seq":
                mask = mask.clone()
                mask[-1] = False
                x = x.masked_fill(~mask[..., None], 0)
            arrays[f"{name}/fwd_x"] = x.numpy().astype(np.float32)
            arrays[f"{name}/fwd_mask"] = mask.numpy().astype(np.bool_)
        model.eval()
        with torch.no_grad():
            y32 = model(x, mask)
            y64 = copy.deepcopy(model).double()(x.double(), mask)
        arrays[f"{name}/y_fp32"] = y32.numpy().astype(np.float32)
        arrays[f"{name}/y_fp64"] = y64.numpy().astype(np.float64)
        arrays[f"{name}/meta"] = np.array([b, s, d, h, f, layers, int(causal), seed], np.int64)
        arrays[f"{name}/padding_ratio"] = np.array([pad], np.float64)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({len(arrays)} arrays)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
