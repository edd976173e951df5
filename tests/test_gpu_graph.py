"""HIP-graph replay of the whole forward (GraphedOptimizedTransformer) against the eager module
and the fp32 oracle.

Each graph is replayed several times with eager work and synchronisations in between, and every
replay is compared bit for bit with the eager module on the same inputs (same kernels, same
order).  New contents written into the captured input allocation must be picked up by the next
replay; a different allocation must fall back to the eager path and leave the static output alone.
"""

import copy

import pytest
import torch

from oracle import transformer_oracle as O
from tttj_2026_amd import PLAN_LAYERWISE, PLAN_MEGAKERNEL, make_optimized_transformer
from tttj_2026_amd.configs import build_model, make_inputs
from tttj_2026_amd.model import TransformerConfig

pytestmark = pytest.mark.gpu

CASES = [
    # (B, S, D, H, F, L, causal, masked, plan)
    (2, 256, 512, 8, 2048, 2, False, True, PLAN_LAYERWISE),
    (1, 64, 256, 8, 1024, 4, True, False, PLAN_LAYERWISE),
    (1, 64, 256, 8, 1024, 4, True, False, PLAN_MEGAKERNEL),
    (3, 100, 256, 4, 512, 2, True, True, PLAN_MEGAKERNEL),
]


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}S{c[1]}D{c[2]}L{c[5]}{'c' if c[6] else 'n'}"
                                             f"{'-mask' if c[7] else ''}-plan{c[8]}" for c in CASES])
def test_graph_replay_matches_eager(device, case):
    b, s, d, h, f, l, causal, masked, plan = case
    cfg = TransformerConfig(b, s, d, h, f, l, causal)
    gm = build_model(cfg, seed=21).half().to(device).eval()
    eager = make_optimized_transformer(copy.deepcopy(gm), plan=plan)
    graphed = make_optimized_transformer(copy.deepcopy(gm), plan=plan, graphed=True)
    x1, m1 = make_inputs(cfg, masked, 31, min_valid=max(1, s // 2))
    x2, _ = make_inputs(cfg, False, 32)
    if m1 is not None:
        x2 = x2.masked_fill(~m1[..., None], 0)
    xd = x1.to(device)
    md = None if m1 is None else m1.to(device)
    print(f"[graph] case {case}", flush=True)
    p32 = O.params_fp32(gm)
    with torch.inference_mode():
        want1 = eager(xd, md).clone()
        for i in range(4):
            got = graphed(xd, md)
            torch.cuda.synchronize()
            assert graphed.captured
            assert torch.equal(got, want1), f"replay {i} differs from eager"
            # eager work between replays
            _ = eager(xd, md)
            torch.cuda.synchronize()
        res = O.check_tolerance(got, O.forward(p32, x1.float(), m1, h, causal), m1)
        assert res["passed"], res
        # new contents in the captured allocation are read by the next replay
        xd.copy_(x2.to(device))
        want2 = eager(xd, md).clone()
        got2 = graphed(xd, md)
        torch.cuda.synchronize()
        assert torch.equal(got2, want2)
        res2 = O.check_tolerance(got2, O.forward(p32, x2.float(), m1, h, causal), m1)
        assert res2["passed"], res2
        # another allocation falls back to the eager module; the static output is untouched
        static_before = got2.clone()
        other = x1.to(device)
        y_other = graphed(other, None if md is None else md.clone())
        torch.cuda.synchronize()
        assert y_other.data_ptr() != got2.data_ptr()
        assert torch.equal(y_other, want1)
        assert torch.equal(got2, static_before)
    if plan == PLAN_MEGAKERNEL:
        assert eager.megakernel_status(b, s) == 0
        assert graphed.module.megakernel_status(b, s) == 0
