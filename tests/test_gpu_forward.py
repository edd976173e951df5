"""End-to-end parity of make_optimized_transformer(model)(x, mask) against the fp32 CPU oracle.

Gate (the acceptance bar): over the whole [B,S,D] fp16 output, max|d| <= 2e-2 and
mean|d| <= 2e-3 against the oracle run in fp32 on the fp16-rounded weights and inputs, padded rows
bitwise +0.0, and two consecutive calls bit-identical (the reference's repeat check,
benchmarks/regression.py:123-134).
"""

import copy

import pytest
import torch

from oracle import transformer_oracle as O
from tttj_2026_amd import PLAN_LAYERWISE, make_optimized_transformer, ops
from tttj_2026_amd.configs import WORKLOADS, WORKLOAD_ORDER, build_model, make_inputs, workload_inputs
from tttj_2026_amd.model import TransformerConfig

pytestmark = pytest.mark.gpu


def _run(model_cpu, x16, mask, device, perturb_ln=False, **kw):
    cfg = model_cpu.config
    if perturb_ln:
        g = torch.Generator().manual_seed(99)
        with torch.no_grad():
            for name, p in model_cpu.named_parameters():
                if "norm" in name:
                    p.add_(0.25 * torch.randn(p.shape, generator=g))
    gpu_model = copy.deepcopy(model_cpu).half().to(device).eval()
    opt = make_optimized_transformer(copy.deepcopy(gpu_model), **kw)
    xd = x16.to(device)
    md = None if mask is None else mask.to(device)
    with torch.inference_mode():
        y1 = opt(xd, md).clone()
        y2 = opt(xd, md)
    torch.cuda.synchronize()
    ref = O.forward(O.params_fp32(gpu_model), x16.float(), mask, cfg.num_heads, cfg.causal)
    res = O.check_tolerance(y1, ref, mask)
    res["repeat_identical"] = bool(torch.equal(y1, y2))
    return res, gpu_model, y1, ref


# Eager PyTorch fp16 (the reference's baseline module, fp16 weights and activations) against the
# same fp32 oracle: the error floor of fp16 arithmetic on each workload.  The optimized forward
# keeps the scores, softmax statistics and every accumulation in fp32, so it must stay within
# this floor plus a small margin (it is below the floor where eager rounds the scores to fp16).
FLOOR_MARGIN_MAX, FLOOR_MARGIN_MEAN = 2e-3, 2e-4


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", WORKLOAD_ORDER)
def test_workload_parity(device, name):
    w = WORKLOADS[name]
    model = build_model(w.config)
    x16, mask = workload_inputs(name)
    print(f"[parity] {name} {w.description}", flush=True)
    res, gpu_model, _, ref = _run(model, x16, mask, device)
    with torch.inference_mode():
        eager = gpu_model(x16.to(device), None if mask is None else mask.to(device))
    torch.cuda.synchronize()
    floor = O.check_tolerance(eager, ref, mask, max_abs=1.0, mean_abs=1.0)
    print(f"[parity] {name} optimized {res}", flush=True)
    print(f"[floor] {name} eager fp16 max_abs {floor['max_abs']:.5f} mean_abs {floor['mean_abs']:.3e}"
          f"  optimized max_abs {res['max_abs']:.5f} mean_abs {res['mean_abs']:.3e}", flush=True)
    assert res["passed"], res
    assert res["repeat_identical"]
    assert res["max_abs"] <= floor["max_abs"] + FLOOR_MARGIN_MAX, (res, floor)
    assert res["mean_abs"] <= floor["mean_abs"] + FLOOR_MARGIN_MEAN, (res, floor)


def _lengths_mask(lengths, seq):
    return torch.arange(seq)[None, :] < torch.tensor(lengths)[:, None]


# Packed variable-length rows (tt_forward_packs_rows): shapes whose four projections run on MFMA
# tiles, with right-padded lengths that are not multiples of 8 (and 0 and S), non-prefix masks
# with a fully padded sequence, an all-valid mask (bit-identical to no mask) and S not a multiple
# of 8.
@pytest.mark.parametrize("kind", ["prefix", "nonprefix", "allvalid"])
@pytest.mark.parametrize("b,s,d,h,f,causal", [
    (4, 512, 512, 8, 2048, False),
    (4, 512, 512, 16, 2048, True),     # head_dim 32
    (4, 300, 512, 8, 2048, True),      # S % 8 != 0
])
def test_packed_rows_masks(device, kind, b, s, d, h, f, causal):
    from tttj_2026_amd import _lib
    assert _lib.forward_packs_rows(b, s, d, h, f), "shape expected to run on packed rows"
    cfg = TransformerConfig(b, s, d, h, f, 2, causal)
    model = build_model(cfg, seed=31)
    x16, _ = make_inputs(cfg, False, 32)
    g = torch.Generator().manual_seed(33)
    if kind == "prefix":
        mask = _lengths_mask([s - 3, 0, 77, s][:b], s)
    elif kind == "nonprefix":
        mask = torch.rand(b, s, generator=g) > 0.35
        mask[1] = False
        mask[2, : s // 2] = True
    else:
        mask = torch.ones(b, s, dtype=torch.bool)
    x16 = x16.masked_fill(~mask[..., None], 0)
    res, gm, y1, _ = _run(model, x16, mask, device)
    print(f"[packed] {kind} {(b, s, d, h, f, causal)} {res}", flush=True)
    assert res["passed"], res
    assert res["repeat_identical"]
    # the padded forward (every token computed, padded tiles skipped) gives the same bits: packed
    # and padded rows run the same tiles' arithmetic, and every padded token's Q / K / V^T is
    # +0.0 in both
    opt = make_optimized_transformer(copy.deepcopy(gm))
    lib = _lib.load()
    _lib.check(lib.tt_forward_packing_override(0), "packing override")
    try:
        with torch.inference_mode():
            y_pad = opt(x16.to(device), mask.to(device))
        torch.cuda.synchronize()
    finally:
        lib.tt_forward_packing_override(-1)
    assert torch.equal(y_pad, y1)
    if kind == "allvalid":
        with torch.inference_mode():
            y0 = opt(x16.to(device), None)
        assert torch.equal(y0, y1)


# More than 2^20 tokens: the packed-row set-up takes its three-launch path (mask summary, maps,
# V^T clear) instead of the one-launch kernel.  Packed against padded forward bitwise, padded rows
# +0.0, and a few sequences against the oracle (sequences are independent, so each is checked on
# its own).
@pytest.mark.timeout(600)
def test_packed_rows_long_batch(device):
    from tttj_2026_amd import _lib
    b, s, d, h, f = 2048, 520, 64, 1, 64
    assert b * s > (1 << 20)
    assert _lib.forward_packs_rows(b, s, d, h, f), "shape expected to run on packed rows"
    cfg = TransformerConfig(b, s, d, h, f, 1, True)
    model = build_model(cfg, seed=41)
    x16, _ = make_inputs(cfg, False, 42)
    g = torch.Generator().manual_seed(43)
    lengths = torch.randint(0, s + 1, (b,), generator=g)
    lengths[:3] = torch.tensor([0, s, 7])
    mask = torch.arange(s)[None, :] < lengths[:, None]
    x16 = x16.masked_fill(~mask[..., None], 0)
    gm = copy.deepcopy(model).half().to(device).eval()
    opt = make_optimized_transformer(copy.deepcopy(gm))
    xd, md = x16.to(device), mask.to(device)
    lib = _lib.load()
    with torch.inference_mode():
        y = opt(xd, md)
        _lib.check(lib.tt_forward_packing_override(0), "packing override")
        try:
            y_pad = opt(xd, md)
        finally:
            lib.tt_forward_packing_override(-1)
    torch.cuda.synchronize()
    assert torch.equal(y, y_pad)
    assert bool((y.cpu()[~mask] == 0).all()) and not torch.signbit(y.cpu()[~mask]).any()
    params = O.params_fp32(gm)
    for i in (0, 1, 2, 1000, b - 1):
        ref = O.forward(params, x16[i:i + 1].float(), mask[i:i + 1], h, True)
        res = O.check_tolerance(y[i:i + 1], ref, mask[i:i + 1])
        print(f"[packed-long] seq {i} len {int(lengths[i])} {res}", flush=True)
        assert res["passed"], (i, res)


# The reference's input-scale sweep (benchmarks/benchmark_steps_1_2.py:28) on the C1 (layer-wise,
# LayerNorm folded into the projections), C2 (persistent megakernel) and C3 (masked, packed rows)
# shapes.
INPUT_SCALES = (1.0e-4, 1.0e-3, 3.0e-3, 1.0e-2, 0.1, 1.0, 10.0, 100.0, 1000.0)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("name", ["C1", "C2", "C3"])
def test_input_scale_sweep(device, name):
    w = WORKLOADS[name]
    model = build_model(w.config)
    x16, mask = workload_inputs(name)
    gpu_model = copy.deepcopy(model).half().to(device).eval()
    opt = make_optimized_transformer(copy.deepcopy(gpu_model))
    p32 = O.params_fp32(gpu_model)
    md = None if mask is None else mask.to(device)
    for scale in INPUT_SCALES:
        xs = (x16.float() * scale).half()
        with torch.inference_mode():
            y = opt(xs.to(device), md)
        torch.cuda.synchronize()
        ref = O.forward(p32, xs.float(), mask, w.config.num_heads, w.config.causal)
        res = O.check_tolerance(y, ref, mask)
        print(f"[scale] {name} x{scale:g} {res}", flush=True)
        assert res["passed"], (scale, res)


@pytest.mark.parametrize("offset", [30.0, 200.0])
@pytest.mark.parametrize("name", ["C1", "C2", "C3"])
def test_large_row_mean(device, name, offset):
    """Rows whose mean is far larger than their spread (|mean| = 30 or 200, std 1): the LayerNorms
    folded into the projections (C1 layer-wise, C2 megakernel) compute rstd (x W'^T - mean c) + b',
    a difference of two large terms.  At these magnitudes the fp16 residual stream itself is
    coarse (ulp 1/64 at 30, 1/8 at 200), which eager fp16 pays too, so the bar is eager fp16's
    error against the same fp32 oracle: a cancellation in the fold would exceed it."""
    w = WORKLOADS[name]
    model = build_model(w.config)
    x16, mask = workload_inputs(name)
    g = torch.Generator().manual_seed(77)
    off = offset * torch.sign(torch.randn(x16.shape[0], x16.shape[1], 1, generator=g))
    xs = (x16.float() + off).half()
    if mask is not None:
        xs = xs.masked_fill(~mask[..., None], 0)
    res, gm, _, ref = _run(model, xs, mask, device)
    with torch.inference_mode():
        eager = gm(xs.to(device), None if mask is None else mask.to(device))
    torch.cuda.synchronize()
    floor = O.check_tolerance(eager, ref, mask, max_abs=1e9, mean_abs=1e9)
    print(f"[rowmean] {name} +-{offset:g}: optimized max {res['max_abs']:.4f} mean "
          f"{res['mean_abs']:.3e}; eager fp16 max {floor['max_abs']:.4f} mean "
          f"{floor['mean_abs']:.3e}", flush=True)
    assert res["finite"] and res["padded_zero"] and res["repeat_identical"], res
    assert res["max_abs"] <= 1.25 * floor["max_abs"] + 2e-3, (res, floor)
    assert res["mean_abs"] <= 1.25 * floor["mean_abs"] + 2e-4, (res, floor)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hd", [32, 64])
def test_nonprefix_mask_and_perturbed_norms(device, causal, hd):
    cfg = TransformerConfig(3, 96, 256, 256 // hd, 512, 2, causal)
    model = build_model(cfg, seed=7)
    x16, _ = make_inputs(cfg, False, 8)
    g = torch.Generator().manual_seed(9)
    mask = torch.rand(3, 96, generator=g) > 0.3
    mask[1] = False          # a fully padded sequence
    mask[2, :50] = True
    x16 = x16.masked_fill(~mask[..., None], 0)
    res, _, _, _ = _run(model, x16, mask, device, perturb_ln=True)
    assert res["passed"], res
    assert res["repeat_identical"]


@pytest.mark.parametrize("scale", [1e-3, 1.0, 30.0])
def test_input_scales(device, scale):
    cfg = TransformerConfig(2, 128, 512, 8, 2048, 2, True)
    model = build_model(cfg, seed=3)
    x16, mask = make_inputs(cfg, True, 4)
    x16 = (x16.float() * scale).half()
    res, _, _, _ = _run(model, x16, mask, device)
    assert res["passed"], res


@pytest.mark.parametrize("plan", ["auto", "layerwise"])
@pytest.mark.parametrize("b,s,d,h,f,causal,masked", [
    (1, 64, 256, 8, 1024, True, False),      # C2 shape: ffn_out K = 1024 over 4 tiles
    (2, 96, 256, 4, 2048, True, True),       # padded rows, K = 2048
    (4, 128, 512, 8, 2048, False, True),
    (3, 40, 128, 2, 512, False, False),      # partial row tile, K = 512
])
def test_few_tokens_long_k(device, plan, b, s, d, h, f, causal, masked):
    """Few tokens and long K (small grids, partial row tiles, padded rows), both plans."""
    from tttj_2026_amd import PLAN_AUTO
    cfg = TransformerConfig(b, s, d, h, f, 2, causal)
    model = build_model(cfg, seed=11)
    x16, mask = make_inputs(cfg, masked, 12)
    res, _, _, _ = _run(model, x16, mask, device,
                        plan=PLAN_AUTO if plan == "auto" else PLAN_LAYERWISE)
    assert res["passed"], res
    assert res["repeat_identical"]


def test_runtime_shape_differs_from_config(device):
    """Any (B, S) works at run time; only d_model/heads/ffn/layers come from the config."""
    cfg = TransformerConfig(4, 128, 256, 4, 1024, 2, False)
    model = build_model(cfg, seed=5)
    run_cfg = TransformerConfig(3, 77, 256, 4, 1024, 2, False)
    x16, mask = make_inputs(run_cfg, True, 6, min_valid=10)
    res, _, _, _ = _run(model, x16, mask, device, plan=PLAN_LAYERWISE)
    assert res["passed"], res


def test_eager_fp16_floor_and_no_mask_equivalence(device):
    name = "C1"
    w = WORKLOADS[name]
    model = build_model(w.config)
    x16, _ = workload_inputs(name)
    gpu_model = copy.deepcopy(model).half().to(device).eval()
    opt = make_optimized_transformer(copy.deepcopy(gpu_model))
    xd = x16.to(device)
    with torch.inference_mode():
        eager = gpu_model(xd, None)
        a = opt(xd, None)
        b = opt(xd, torch.ones(x16.shape[:2], dtype=torch.bool, device=device))
    ref = O.forward(O.params_fp32(gpu_model), x16.float(), None, w.config.num_heads, w.config.causal)
    floor = O.check_tolerance(eager, ref, None)
    ours = O.check_tolerance(a, ref, None)
    print(f"[floor] eager fp16 {floor}  optimized {ours}", flush=True)
    assert ours["passed"]
    assert torch.equal(a, b)


def test_stage_parity_layer0(device):
    """Layer-0 intermediates of the kernel chain vs the oracle's stages (numerics localisation,
    after benchmarks/benchmark_steps_1_2.py:73-117)."""
    cfg = TransformerConfig(2, 128, 512, 8, 2048, 1, False)
    model = build_model(cfg, seed=21)
    x16, mask = make_inputs(cfg, True, 22)
    gm = copy.deepcopy(model).half().to(device)
    p32 = O.params_fp32(gm)
    stages = {}
    O.forward(p32, x16.float(), mask, cfg.num_heads, cfg.causal, stages=stages)
    L = gm.layers[0]
    xd, md = x16.to(device), mask.to(device)
    ln1 = ops.layernorm(xd, L.norm1.weight, L.norm1.bias)
    att = L.attention
    wqkv = torch.cat([att.q_proj.weight, att.k_proj.weight, att.v_proj.weight])
    bqkv = torch.cat([att.q_proj.bias, att.k_proj.bias, att.v_proj.bias])
    q, k, vt = ops.qkv_projection(ln1, wqkv, bqkv, cfg.num_heads)
    ctx = ops.attention(q, k, vt, md, cfg.causal)
    x1 = ops.linear(ctx, att.out_proj.weight, att.out_proj.bias, "resid_masked", residual=xd, valid=md)
    ln2 = ops.layernorm(x1, L.norm2.weight, L.norm2.bias)
    hmid = ops.linear(ln2, L.ffn_in.weight, L.ffn_in.bias, "gelu")
    x2 = ops.linear(hmid, L.ffn_out.weight, L.ffn_out.bias, "masked_resid", residual=x1, valid=md)
    torch.cuda.synchronize()
    v = mask
    hd = 512 // 8
    checks = {
        "ln1": (ln1, stages["ln1"], 1e-2),
        "q": (q.permute(0, 2, 1, 3).reshape(2, 128, 512), stages["q"], 2e-2),
        "ctx": (ctx, stages["ctx"], 2e-2),
        "x1": (x1, x16.float() + stages["attn_out"], 3e-2),
        "gelu": (hmid, stages["gelu"], 2e-2),
        "block_out": (x2, stages["block_out"], 4e-2),
    }
    for name, (got, want, tol) in checks.items():
        err = (got.float().cpu()[v] - want[v]).abs().max().item()
        assert err <= tol, (name, err)
    assert (x2.cpu()[~v].view(torch.int16) == 0).all()
    del hd


# ---------------------------------------------------------------- folded LayerNorm
def test_pack_derived_segments(device):
    """Segments 12-17 written by tt_pack_derived: W' = fp16(W * gamma) exactly, c = row sums of
    W' and b' = b + W beta (fp32, against float64 sums of the same fp16 values)."""
    from tttj_2026_amd import _lib
    from tttj_2026_amd.optimized_transformer import pack_model_weights

    cfg = TransformerConfig(1, 8, 128, 4, 320, 2, True)
    model = build_model(cfg, seed=31)
    g = torch.Generator().manual_seed(32)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name:
                p.add_(0.3 * torch.randn(p.shape, generator=g))
    gm = model.half().to(device)
    packed = pack_model_weights(gm)
    torch.cuda.synchronize()
    offs, stride, _, _ = _lib.weight_layout(128, 320, 2)
    P = packed.cpu()
    D, F = 128, 320
    for l in range(2):
        base = l * stride
        seg = lambda i, n: P[base + offs[i]: base + offs[i] + n]
        fp32 = lambda i, n: seg(i, 2 * n).view(torch.float32)
        for (w_i, g_i, b_i, bias_i, wp_i, c_i, bp_i, rows) in (
                (2, 0, 1, 3, 12, 13, 14, 3 * D), (8, 6, 7, 9, 15, 16, 17, F)):
            W = seg(w_i, rows * D).view(rows, D)
            gam, bet, bias = seg(g_i, D), seg(b_i, D), seg(bias_i, rows)
            Wp = seg(wp_i, rows * D).view(rows, D)
            assert torch.equal(Wp, (W.float() * gam.float()).half())
            c_ref = Wp.double().sum(1)
            b_ref = bias.double() + (W.double() * bet.double()).sum(1)
            assert torch.allclose(fp32(c_i, rows).double(), c_ref, atol=1e-4, rtol=1e-5)
            assert torch.allclose(fp32(bp_i, rows).double(), b_ref, atol=1e-4, rtol=1e-5)


@pytest.mark.parametrize("shape", [(2, 64, 256, 4, 1024, 3, False, False),
                                   (3, 100, 512, 8, 2048, 2, True, True),
                                   (1, 32, 96, 3, 160, 2, True, False)],
                         ids=["D256", "D512-masked", "D96-small-kernel"])
def test_folded_layernorm_large_input_perturbed_norms(device, shape):
    """The folded LayerNorm (statistics from the producer's partial slots, W' and the epilogue
    correction) at input scale 30 with non-default LayerNorm parameters: the gate still holds,
    so the single-pass partial statistics and the rstd (acc - mean c) form do not cancel badly."""
    b, s, d, h, f, l, causal, masked = shape
    cfg = TransformerConfig(b, s, d, h, f, l, causal)
    model = build_model(cfg, seed=41)
    x16, mask = make_inputs(cfg, masked, 42, min_valid=max(1, s // 2))
    x16 = (x16.float() * 30.0).half()
    print(f"[fold] {shape}", flush=True)
    res, _, _, _ = _run(model, x16, mask if masked else None, device, perturb_ln=True)
    print(f"[fold] {shape} {res}", flush=True)
    assert res["passed"], res
    assert res["repeat_identical"]


def test_every_tile_perturbed_norms(device):
    """Every GEMM tile configuration forced in turn (with tile 5, the narrow kernel, the
    LayerNorms are folded and its statistics slots are 32 columns wide): each forward passes the
    gate with perturbed LayerNorm parameters."""
    from tttj_2026_amd import _lib

    lib = _lib.load()
    cfg = TransformerConfig(2, 128, 512, 8, 1024, 2, True)
    model = build_model(cfg, seed=51)
    g = torch.Generator().manual_seed(53)
    with torch.no_grad():  # perturbed once (_run's perturb_ln would accumulate over the loop)
        for name, p in model.named_parameters():
            if "norm" in name:
                p.add_(0.25 * torch.randn(p.shape, generator=g))
    x16, mask = make_inputs(cfg, True, 52, min_valid=64)
    try:
        for tile in range(11):
            assert lib.tt_gemm_tile_override(tile) == 0
            res, _, _, _ = _run(model, x16, mask, device)
            print(f"[fold] tile {tile} {res}", flush=True)
            assert res["passed"], (tile, res)
    finally:
        lib.tt_gemm_tile_override(-1)


@pytest.mark.parametrize("name", ["C1", "C2"])
def test_folded_layernorm_matches_fused_ln_plan(device, name):
    """At the few-token workloads the layer-wise plan folds the LayerNorms; its output agrees
    with the fused-LN plan (LayerNorm computed in LDS from the unfolded weights) far inside the
    gate, with perturbed LayerNorm parameters."""
    from tttj_2026_amd import PLAN_FUSED_LN

    w = WORKLOADS[name]
    model = build_model(w.config, seed=61)
    g = torch.Generator().manual_seed(62)
    with torch.no_grad():
        for pname, p in model.named_parameters():
            if "norm" in pname:
                p.add_(0.25 * torch.randn(p.shape, generator=g))
    x16, mask = workload_inputs(name)
    res_a, _, ya, ref = _run(model, x16, mask, device, plan=PLAN_LAYERWISE)
    res_b, _, yb, _ = _run(model, x16, mask, device, plan=PLAN_FUSED_LN)
    print(f"[fold] {name} layerwise {res_a} fused_ln {res_b}", flush=True)
    assert res_a["passed"] and res_b["passed"]
    assert (ya.float() - yb.float()).abs().max().item() <= 1e-2


# ---------------------------------------------------------------- captured stages of the fused plans
@pytest.mark.parametrize("plan_name,shape", [
    ("megakernel", (2, 64, 256, 8, 1024, True, True)),      # hd 32, causal, padded
    ("megakernel", (1, 64, 256, 4, 1024, False, False)),    # hd 64
    ("fused_ln", (2, 100, 128, 4, 512, True, True)),
    ("layerwise", (4, 128, 256, 4, 1024, False, True)),     # LayerNorm folded (narrow tiles)
    ("layerwise", (2, 256, 512, 8, 2048, True, False)),     # MFMA tiles; LN2 overwrites ctx
    ("layerwise", (4, 512, 512, 16, 2048, True, True)),     # packed variable-length rows
], ids=["mk-hd32-causal-mask", "mk-hd64", "fusedln-causal-mask", "lw-fold-mask", "lw-mfma-causal",
        "lw-packed-mask"])
def test_captured_stages(device, plan_name, shape):
    """Per-stage parity inside the fused plans (after benchmarks/benchmark_steps_1_2.py:73-117 and
    the CAPTURE slots of kernels/fused_megakernel.py:224-238): the last layer's Q / K / V, attention
    context and GELU activations left in the workspace by one 1-layer forward, against the
    oracle's stages.  The in-LDS LayerNorms of the megakernel and the fused-LN tiles are never
    stored on their own; Q / K / V and the GELU input depend on them directly."""
    from tttj_2026_amd import PLAN_FUSED_LN, PLAN_MEGAKERNEL
    plans = {"megakernel": PLAN_MEGAKERNEL, "fused_ln": PLAN_FUSED_LN, "layerwise": PLAN_LAYERWISE}
    b, s, d, h, f, causal, masked = shape
    cfg = TransformerConfig(b, s, d, h, f, 1, causal)
    model = build_model(cfg, seed=41)
    with torch.no_grad():  # non-default LayerNorm affine parameters
        g = torch.Generator().manual_seed(42)
        for name, p in model.named_parameters():
            if "norm" in name:
                p.add_(0.2 * torch.randn(p.shape, generator=g))
    x16, mask = make_inputs(cfg, masked, 43)
    gm = copy.deepcopy(model).half().to(device).eval()
    mod = make_optimized_transformer(copy.deepcopy(gm), plan=plans[plan_name])
    print(f"[stages] {plan_name} {shape}", flush=True)
    with torch.inference_mode():
        mod(x16.to(device), None if mask is None else mask.to(device))
        got = mod.captured_stages(b, s)
        got = {k: (None if v is None else v.float().cpu()) for k, v in got.items()}
    st = {}
    O.forward(O.params_fp32(gm), x16.float(), mask, h, causal, stages=st)
    v = torch.ones(b, s, dtype=torch.bool) if mask is None else mask
    heads_to_rows = lambda t: t.permute(0, 2, 1, 3).reshape(b, s, d)  # [B,H,S,hd] -> [B,S,D]
    checks = {"q": (heads_to_rows(got["q"]), st["q"]), "k": (heads_to_rows(got["k"]), st["k"]),
              "v": (heads_to_rows(got["v"]), st["v"]), "hidden": (got["hidden"], st["gelu"])}
    if got["ctx"] is not None:
        checks["ctx"] = (got["ctx"], st["ctx"])
    elif plan_name != "layerwise" or d <= 256:
        raise AssertionError("the fused plans keep the context")
    for name, (a, want) in checks.items():
        err = (a[v] - want[v]).abs().max().item()
        assert err <= 2e-2, (name, err)
