"""Fused-LayerNorm layer-wise plan (LN1 / LN2 computed inside the QKV / ffn_in tiles) against the
fp32 oracle and the plain layer-wise plan.

Same gate as the end-to-end tests (max-abs <= 2e-2, mean-abs <= 2e-3, padded rows bitwise +0.0,
repeated calls bit-identical), on the megakernel's case list: ragged S, d_model up to 512 (a K
ring that wraps), head dims 32 and 64, prefix / non-prefix / empty masks, perturbed LN affines.
"""

import copy

import pytest
import torch

from oracle import transformer_oracle as O
from tttj_2026_amd import PLAN_FUSED_LN, PLAN_LAYERWISE, make_optimized_transformer
from tttj_2026_amd.configs import build_model, make_inputs
from tttj_2026_amd.model import TransformerConfig

pytestmark = pytest.mark.gpu

CASES = [
    # (B, S, D, H, F, L, causal, mask kind)
    (1, 64, 256, 8, 1024, 4, True, None),          # C2 shape
    (4, 128, 256, 4, 1024, 2, False, None),        # C1 shape
    (3, 200, 256, 4, 512, 2, True, "prefix"),
    (2, 77, 256, 8, 256, 3, False, "nonprefix"),
    (2, 256, 512, 8, 2048, 2, True, "prefix"),     # D = 512: the W ring wraps
    (5, 33, 128, 4, 128, 1, True, "empty"),
]


def _mask(kind, b, s, seed):
    if kind is None:
        return None
    g = torch.Generator().manual_seed(seed)
    if kind == "prefix":
        lens = torch.randint(max(1, s // 2), s + 1, (b,), generator=g)
        return torch.arange(s)[None, :] < lens[:, None]
    if kind == "empty":
        lens = torch.randint(1, s + 1, (b,), generator=g)
        lens[1] = 0
        return torch.arange(s)[None, :] < lens[:, None]
    m = torch.rand(b, s, generator=g) > 0.3
    m[:, 0] = True
    return m


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}S{c[1]}D{c[2]}H{c[3]}F{c[4]}L{c[5]}"
                                             f"{'c' if c[6] else 'n'}-{c[7]}" for c in CASES])
def test_fused_ln_parity(device, case):
    b, s, d, h, f, l, causal, kind = case
    cfg = TransformerConfig(b, s, d, h, f, l, causal)
    model = build_model(cfg, seed=41)
    with torch.no_grad():
        g = torch.Generator().manual_seed(42)
        for name, p in model.named_parameters():
            if "norm" in name:
                p.add_(0.2 * torch.randn(p.shape, generator=g))
    x16, _ = make_inputs(cfg, False, 43)
    mask = _mask(kind, b, s, 44)
    if mask is not None:
        x16 = x16.masked_fill(~mask[..., None], 0)
    gm = copy.deepcopy(model).half().to(device).eval()
    fz = make_optimized_transformer(copy.deepcopy(gm), plan=PLAN_FUSED_LN)
    lw = make_optimized_transformer(copy.deepcopy(gm), plan=PLAN_LAYERWISE)
    xd = x16.to(device)
    md = None if mask is None else mask.to(device)
    print(f"[fused-ln] case {case}", flush=True)
    with torch.inference_mode():
        y1 = fz(xd, md).clone()
        y2 = fz(xd, md)
        ylw = lw(xd, md)
    torch.cuda.synchronize()
    ref = O.forward(O.params_fp32(gm), x16.float(), mask, h, causal)
    res = O.check_tolerance(y1, ref, mask)
    assert res["passed"], res
    assert torch.equal(y1, y2)
    assert (y1.float() - ylw.float()).abs().max().item() <= 2e-2


def test_fused_ln_graph_replay(device):
    cfg = TransformerConfig(1, 64, 256, 8, 1024, 4, True)
    gm = build_model(cfg, seed=45).half().to(device).eval()
    eager = make_optimized_transformer(copy.deepcopy(gm), plan=PLAN_FUSED_LN)
    graphed = make_optimized_transformer(copy.deepcopy(gm), plan=PLAN_FUSED_LN, graphed=True)
    x16, _ = make_inputs(cfg, False, 46)
    xd = x16.to(device)
    with torch.inference_mode():
        want = eager(xd, None).clone()
        for _ in range(3):
            got = graphed(xd, None)
            torch.cuda.synchronize()
            assert torch.equal(got, want)
            eager(xd, None)
            torch.cuda.synchronize()
