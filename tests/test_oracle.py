"""CPU tests that pin the oracle (oracle/transformer_oracle.py) before anything is checked against it.

Pins, in order of strength:
  * golden fixtures written by importing the reference itself (tests/golden/make_golden.py):
    seeded default-init weights and generate_random_case outputs;
  * a scalar-loop float64 restatement (bruteforce_forward) on tiny shapes, including causal,
    ragged right-padded masks, non-prefix masks and a fully padded sequence;
  * closed forms and invariants: GELU vs math.erf, LayerNorm shift invariance, single-head
    unmasked attention vs a textbook softmax(QK^T/sqrt(d))V, permutation equivariance of
    non-causal unmasked attention, the causal prefix property, all-valid mask == None;
  * the FLOP accounting against the closed-form totals of the benchmark table.
"""

import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import transformer_oracle as O
from tttj_2026_amd import roofline
from tttj_2026_amd.configs import WORKLOADS, build_model, make_inputs
from tttj_2026_amd.model import BaselineTransformer, TransformerConfig

GOLDEN = pathlib.Path(__file__).parent / "golden" / "reference_init_and_inputs.npz"


def _tiny(causal, layers=2, d=16, h=2, f=24, b=2, s=6):
    return TransformerConfig(b, s, d, h, f, layers, causal)


def _params(cfg, seed=1234, perturb=False):
    m = build_model(cfg, seed)
    p = O.params_fp32(m)
    if perturb:  # non-default LayerNorm affine parameters expose affine bugs
        g = torch.Generator().manual_seed(seed + 5)
        for k in p:
            if "norm" in k:
                p[k] = p[k] + 0.3 * torch.randn(p[k].shape, generator=g)
    return p


# ---------------------------------------------------------------- golden fixtures (reference)
@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def _golden_cases(golden):
    return sorted({k.split("/")[0] for k in golden.files})


def test_golden_init_matches_reference(golden):
    for case in _golden_cases(golden):
        b, s, d, h, f, layers, causal, seed = (int(v) for v in golden[f"{case}/meta"])
        cfg = TransformerConfig(b, s, d, h, f, layers, bool(causal))
        model = build_model(cfg, seed)
        sd = model.state_dict()
        keys = [k[len(case) + 7:] for k in golden.files if k.startswith(f"{case}/param/")]
        assert sorted(keys) == sorted(sd.keys())
        for k in keys:
            np.testing.assert_array_equal(sd[k].numpy(), golden[f"{case}/param/{k}"], err_msg=k)


def test_golden_generate_random_case_matches_reference(golden):
    for case in _golden_cases(golden):
        b, s, d, h, f, layers, causal, seed = (int(v) for v in golden[f"{case}/meta"])
        pad = float(golden[f"{case}/padding_ratio"][0])
        x, mask = O.generate_random_case(b, s, d, seed + 1, pad)
        np.testing.assert_array_equal(x.numpy(), golden[f"{case}/x"])
        np.testing.assert_array_equal(mask.numpy(), golden[f"{case}/mask"])


def _golden_forward_params(golden, case):
    """The weights the reference forward ran with: the LayerNorm-perturbed set where the case
    has one, else the seeded default init."""
    pre = f"{case}/fwd_param/" if any(k.startswith(f"{case}/fwd_param/") for k in golden.files) \
        else f"{case}/param/"
    return {k[len(pre):]: torch.from_numpy(golden[k]) for k in golden.files if k.startswith(pre)}


def _golden_forward_inputs(golden, case):
    """(x, mask) the reference forward ran on: the case's own mask where it has one, else the
    generator's draw."""
    xk, mk = (f"{case}/fwd_x", f"{case}/fwd_mask") if f"{case}/fwd_x" in golden.files \
        else (f"{case}/x", f"{case}/mask")
    return torch.from_numpy(golden[xk]), torch.from_numpy(golden[mk])


def test_golden_forward_oracle_vs_bruteforce(golden):
    """The fixture inputs through both restatements (weights are the reference's own)."""
    for case in _golden_cases(golden):
        b, s, d, h, f, layers, causal, seed = (int(v) for v in golden[f"{case}/meta"])
        p = _golden_forward_params(golden, case)
        x, mask = _golden_forward_inputs(golden, case)
        out = O.forward(p, x, mask, h, bool(causal)).double().numpy()
        bf = O.bruteforce_forward(p, x, mask, h, bool(causal))
        np.testing.assert_allclose(out, bf, atol=2e-5, rtol=0)


def test_golden_forward_matches_reference_output(golden):
    """Both restatements against the reference BaselineTransformer's own forward output
    (float64 module copy and float32), on causal and non-causal cases, prefix and non-prefix
    masks, a fully padded sequence and perturbed LayerNorm parameters."""
    cases = _golden_cases(golden)
    assert {"masked_noncausal_ln", "nonprefix_causal_ln"} <= set(cases)
    for case in cases:
        b, s, d, h, f, layers, causal, seed = (int(v) for v in golden[f"{case}/meta"])
        p = _golden_forward_params(golden, case)
        x, mask = _golden_forward_inputs(golden, case)
        y64 = golden[f"{case}/y_fp64"]
        y32 = golden[f"{case}/y_fp32"]
        out = O.forward(p, x, mask, h, bool(causal))
        np.testing.assert_allclose(out.double().numpy(), y64, atol=1e-5, rtol=0, err_msg=case)
        np.testing.assert_allclose(out.numpy(), y32, atol=1e-5, rtol=0, err_msg=case)
        # the reference rounds its softmax to fp32 even in a float64 module (scores.float(),
        # torch_transformer_benchmark.py:111), so the float64 brute force differs by ~1e-7
        bf = O.bruteforce_forward(p, x, mask, h, bool(causal))
        np.testing.assert_allclose(bf, y64, atol=1e-6, rtol=0, err_msg=case)
        # padded rows are exactly zero in the reference output and in the oracle's
        assert (y64[~mask.numpy()] == 0).all() and (out[~mask] == 0).all()


# ---------------------------------------------------------------- brute force
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("mask_kind", ["none", "prefix", "nonprefix", "empty_row"])
def test_oracle_matches_bruteforce(causal, mask_kind):
    cfg = _tiny(causal, b=3, s=7)
    p = _params(cfg, perturb=True)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(3, 7, 16, generator=g) * 1.7
    mask = None
    if mask_kind == "prefix":
        mask = torch.arange(7)[None, :] < torch.tensor([7, 4, 1])[:, None]
    elif mask_kind == "nonprefix":
        mask = torch.rand(3, 7, generator=g) > 0.4
        mask[:, 2] = True
    elif mask_kind == "empty_row":
        mask = torch.arange(7)[None, :] < torch.tensor([5, 0, 3])[:, None]
    out = O.forward(p, x, mask, 2, causal)
    bf = O.bruteforce_forward(p, x, mask, 2, causal)
    assert torch.isfinite(out).all()
    np.testing.assert_allclose(out.double().numpy(), bf, atol=2e-5, rtol=0)
    if mask is not None:
        assert (out[~mask] == 0).all()


def test_oracle_matches_module_fp32():
    cfg = _tiny(True, b=2, s=9, d=32, h=2, f=64, layers=3)
    model = build_model(cfg)
    x, mask = make_inputs(cfg, True, 5, min_valid=3)
    with torch.no_grad():
        ref = model(x.float(), mask)
    out = O.forward(O.params_fp32(model), x.float(), mask, 2, True)
    assert (out - ref).abs().max() < 1e-5


# ---------------------------------------------------------------- closed forms / invariants
def test_gelu_matches_math_erf():
    xs = torch.linspace(-8, 8, 161, dtype=torch.float64)
    ref = torch.tensor([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.tolist()],
                       dtype=torch.float64)
    assert torch.allclose(O.gelu_erf(xs), ref, atol=1e-12)
    # erf-GELU differs from the tanh approximation by up to ~5e-4: make sure we did not use it
    tanh = 0.5 * xs * (1 + torch.tanh(math.sqrt(2 / math.pi) * (xs + 0.044715 * xs ** 3)))
    assert (O.gelu_erf(xs) - tanh).abs().max() > 1e-4


def test_layernorm_shift_invariance_and_moments():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 64, generator=g, dtype=torch.float64)
    w, b = torch.ones(64, dtype=torch.float64), torch.zeros(64, dtype=torch.float64)
    y = O.layer_norm(x, w, b)
    assert torch.allclose(O.layer_norm(x + 123.0, w, b), y, atol=1e-9)
    assert torch.allclose(y.mean(-1), torch.zeros(5, dtype=torch.float64), atol=1e-12)
    # biased variance with eps: var(y) = var(x) / (var(x) + eps)
    v = x.var(-1, unbiased=False)
    assert torch.allclose(y.var(-1, unbiased=False), v / (v + O.LN_EPS), atol=1e-12)


def test_single_head_attention_is_textbook():
    g = torch.Generator().manual_seed(4)
    d, s = 8, 6
    names = ("q", "k", "v", "out")
    p = {f"a.{n}_proj.weight": torch.randn(d, d, generator=g) for n in names}
    p.update({f"a.{n}_proj.bias": torch.randn(d, generator=g) for n in names})
    x = torch.randn(1, s, d, generator=g, dtype=torch.float32)
    out = O.attention(x, p, "a.", 1, None, False)
    q = x[0] @ p["a.q_proj.weight"].T + p["a.q_proj.bias"]
    k = x[0] @ p["a.k_proj.weight"].T + p["a.k_proj.bias"]
    v = x[0] @ p["a.v_proj.weight"].T + p["a.v_proj.bias"]
    import scipy.special

    att = scipy.special.softmax((q @ k.T).numpy() / math.sqrt(d), axis=-1) @ v.numpy()
    ref = att @ p["a.out_proj.weight"].numpy().T + p["a.out_proj.bias"].numpy()
    np.testing.assert_allclose(out[0].numpy(), ref, atol=1e-4)


def test_permutation_equivariance_noncausal():
    cfg = _tiny(False, b=1, s=8)
    p = _params(cfg, perturb=True)
    x = torch.randn(1, 8, 16, generator=torch.Generator().manual_seed(9))
    perm = torch.randperm(8, generator=torch.Generator().manual_seed(10))
    y = O.forward(p, x, None, 2, False)
    yp = O.forward(p, x[:, perm], None, 2, False)
    assert torch.allclose(yp, y[:, perm], atol=1e-5)


def test_causal_prefix_property():
    cfg = _tiny(True, b=1, s=8)
    p = _params(cfg)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(1, 8, 16, generator=g)
    x2 = x.clone()
    x2[:, 5:] = torch.randn(1, 3, 16, generator=g)
    y, y2 = O.forward(p, x, None, 2, True), O.forward(p, x2, None, 2, True)
    assert torch.allclose(y[:, :5], y2[:, :5], atol=1e-6)
    assert not torch.allclose(y[:, 5:], y2[:, 5:], atol=1e-3)
    # and the non-causal model does see the future
    yn, yn2 = O.forward(p, x, None, 2, False), O.forward(p, x2, None, 2, False)
    assert not torch.allclose(yn[:, :5], yn2[:, :5], atol=1e-3)


def test_all_valid_mask_equals_none():
    cfg = _tiny(True, b=2, s=5)
    p = _params(cfg)
    x = torch.randn(2, 5, 16, generator=torch.Generator().manual_seed(13))
    a = O.forward(p, x, None, 2, True)
    b = O.forward(p, x, torch.ones(2, 5, dtype=torch.bool), 2, True)
    assert torch.equal(a, b)


def test_check_tolerance_gate():
    ref = torch.zeros(1, 2, 4)
    mask = torch.tensor([[True, False]])
    good = torch.zeros(1, 2, 4, dtype=torch.float16)
    assert O.check_tolerance(good, ref, mask)["passed"]
    neg_zero = good.clone()
    neg_zero[0, 1, 0] = -0.0
    assert not O.check_tolerance(neg_zero, ref, mask)["padded_zero"]
    off = good.clone()
    off[0, 0, 0] = 0.03
    assert not O.check_tolerance(off, ref, mask)["passed"]


# ---------------------------------------------------------------- accounting
@pytest.mark.parametrize("name,gflop", [("C1", 1.745), ("C2", 0.411), ("C3", 180.39),
                                        ("C4", 1786.84), ("C5", 3298.74)])
def test_dense_flops_table(name, gflop):
    cfg = WORKLOADS[name].config
    assert abs(roofline.forward_flops(cfg) / 1e9 - gflop) / gflop < 2e-3


def test_param_count_matches_module():
    for name in ("C1", "C2"):
        cfg = WORKLOADS[name].config
        model = BaselineTransformer(cfg)
        assert roofline.param_count(cfg) == sum(p.numel() for p in model.parameters())
