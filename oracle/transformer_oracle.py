"""CPU fp32 restatement of the reference forward pass -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

This is the oracle the HIP path is checked against.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker (or as the
timed CPU baseline); the optimized package never imports or calls it.

It restates ``BaselineTransformer.forward`` (benchmarks/torch_transformer_benchmark.py:85-172)
as explicit fp32 arithmetic on a flat parameter dict keyed by the reference's state-dict names
(``layers.{i}.norm1.weight`` ...).  Every formula is written out (LayerNorm with biased variance and
eps 1e-5, exact-erf GELU, max-subtracted softmax) rather than delegated to the nn modules, so the
restatement is independent of the module code it checks.  ``bruteforce_forward`` is a second,
loop-level float64 restatement for tiny shapes that pins this one.
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import numpy as np
import torch

LN_EPS = 1e-5


def layer_norm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float = LN_EPS):
    """nn.LayerNorm over the last dim (torch_transformer_benchmark.py:128,130,160)."""
    mu = x.mean(dim=-1, keepdim=True)
    var = ((x - mu) ** 2).mean(dim=-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + eps) * w + b


def linear(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """nn.Linear: x W^T + b (:72-75,131-132)."""
    return torch.matmul(x, w.t()) + b


def gelu_erf(x: torch.Tensor) -> torch.Tensor:
    """F.gelu(approximate="none") (:141): 0.5 x (1 + erf(x / sqrt 2))."""
    return 0.5 * x * (1.0 + torch.erf(x * (1.0 / math.sqrt(2.0))))


def attention(xn: torch.Tensor, p: Dict[str, torch.Tensor], prefix: str, heads: int,
              mask: Optional[torch.Tensor], causal: bool, stages: Optional[dict] = None):
    """BaselineSelfAttention.forward (:85-122) in fp32."""
    bsz, s, d = xn.shape
    hd = d // heads
    scale = hd ** -0.5

    def split(t):  # [B,S,D] -> [B,H,S,hd] (:77-83)
        return t.reshape(bsz, s, heads, hd).permute(0, 2, 1, 3)

    q = linear(xn, p[prefix + "q_proj.weight"], p[prefix + "q_proj.bias"])
    k = linear(xn, p[prefix + "k_proj.weight"], p[prefix + "k_proj.bias"])
    v = linear(xn, p[prefix + "v_proj.weight"], p[prefix + "v_proj.bias"])
    scores = torch.matmul(split(q), split(k).transpose(-2, -1)) * scale          # :97
    neg = torch.tensor(float("-inf"))
    if causal:                                                                      # :99-103
        ki = torch.arange(s)
        scores = torch.where(ki[None, :] > ki[:, None], neg, scores)
    if mask is not None:                                                            # :105-108
        scores = torch.where(mask[:, None, None, :], scores, neg)
    row_max = scores.amax(dim=-1, keepdim=True)                                     # :111
    e = torch.exp(scores - row_max)
    probs = e / e.sum(dim=-1, keepdim=True)
    ctx = torch.matmul(probs, split(v)).permute(0, 2, 1, 3).reshape(bsz, s, d)     # :112-117
    out = linear(ctx, p[prefix + "out_proj.weight"], p[prefix + "out_proj.bias"])  # :118
    if mask is not None:                                                            # :120-121
        out = torch.where(mask[..., None], out, torch.zeros(()))
    if stages is not None:
        stages.update(q=q, k=k, v=v, probs=probs, ctx=ctx, attn_out=out)
    return out


def forward(params: Dict[str, torch.Tensor], x: torch.Tensor, mask: Optional[torch.Tensor],
            heads: int, causal: bool, stages: Optional[dict] = None) -> torch.Tensor:
    """BaselineTransformer.forward (:162-172); x fp32 [B,S,D], mask bool [B,S] or None.

    ``stages`` (optional dict) receives layer-0 intermediates for stage-level checks.
    """
    x = x.float()
    n_layers = 1 + max(int(k.split(".")[1]) for k in params if k.startswith("layers."))
    zero = torch.zeros(())
    for i in range(n_layers):
        pre = f"layers.{i}."
        st = stages if (stages is not None and i == 0) else None
        h = layer_norm(x, params[pre + "norm1.weight"], params[pre + "norm1.bias"])
        if st is not None:
            st["ln1"] = h
        x = x + attention(h, params, pre + "attention.", heads, mask, causal, st)   # :140
        h = layer_norm(x, params[pre + "norm2.weight"], params[pre + "norm2.bias"])
        a = gelu_erf(linear(h, params[pre + "ffn_in.weight"], params[pre + "ffn_in.bias"]))
        x = x + linear(a, params[pre + "ffn_out.weight"], params[pre + "ffn_out.bias"])  # :141
        if mask is not None:                                                        # :143-144
            x = torch.where(mask[..., None], x, zero)
        if st is not None:
            st.update(ln2=h, gelu=a, block_out=x)
    x = layer_norm(x, params["final_norm.weight"], params["final_norm.bias"])        # :169
    if mask is not None:                                                            # :170-171
        x = torch.where(mask[..., None], x, zero)
    return x


def params_fp32(model: torch.nn.Module) -> Dict[str, torch.Tensor]:
    """State dict of a (possibly fp16, possibly GPU) model as fp32 CPU tensors.

    Taking the fp16 parameters upcast to fp32 makes the measured error kernel error, not weight
    quantisation error.
    """
    return {k: v.detach().float().cpu() for k, v in model.state_dict().items()}


# --------------------------------------------------------------------------------------------
# Loop-level float64 restatement for tiny shapes (pins the vectorised oracle above).
# --------------------------------------------------------------------------------------------

def _ln64(row, w, b):
    n = len(row)
    mu = sum(row) / n
    var = sum((v - mu) ** 2 for v in row) / n
    inv = 1.0 / math.sqrt(var + LN_EPS)
    return [(row[i] - mu) * inv * w[i] + b[i] for i in range(n)]


def _lin64(row, w, b):
    return [sum(row[k] * w[n][k] for k in range(len(row))) + b[n] for n in range(len(w))]


def bruteforce_forward(params: Dict[str, torch.Tensor], x: torch.Tensor,
                       mask: Optional[torch.Tensor], heads: int, causal: bool) -> np.ndarray:
    """Scalar-loop float64 forward for B*S*D small enough to loop over (seconds)."""
    p = {k: v.double().tolist() for k, v in params.items()}
    xs = x.double().tolist()
    bsz, s, d = len(xs), len(xs[0]), len(xs[0][0])
    hd = d // heads
    valid = [[True] * s for _ in range(bsz)] if mask is None else mask.tolist()
    n_layers = 1 + max(int(k.split(".")[1]) for k in p if k.startswith("layers."))
    for i in range(n_layers):
        pre = f"layers.{i}."
        w = lambda name: p[pre + name]
        for bi in range(bsz):
            seq = xs[bi]
            ln = [_ln64(r, w("norm1.weight"), w("norm1.bias")) for r in seq]
            q = [_lin64(r, w("attention.q_proj.weight"), w("attention.q_proj.bias")) for r in ln]
            k = [_lin64(r, w("attention.k_proj.weight"), w("attention.k_proj.bias")) for r in ln]
            v = [_lin64(r, w("attention.v_proj.weight"), w("attention.v_proj.bias")) for r in ln]
            ctx = [[0.0] * d for _ in range(s)]
            for h in range(heads):
                c0 = h * hd
                for qi in range(s):
                    allowed = [kj for kj in range(s)
                               if valid[bi][kj] and not (causal and kj > qi)]
                    if not allowed:       # every key masked: softmax is NaN in the reference
                        for dd in range(hd):
                            ctx[qi][c0 + dd] = float("nan")
                        continue
                    sc = {kj: sum(q[qi][c0 + t] * k[kj][c0 + t] for t in range(hd)) / math.sqrt(hd)
                          for kj in allowed}
                    m = max(sc.values())
                    z = sum(math.exp(vv - m) for vv in sc.values())
                    for dd in range(hd):
                        ctx[qi][c0 + dd] = sum(math.exp(sc[kj] - m) / z * v[kj][c0 + dd]
                                               for kj in allowed)
            att = [_lin64(r, w("attention.out_proj.weight"), w("attention.out_proj.bias"))
                   for r in ctx]
            seq = [[seq[si][c] + (att[si][c] if valid[bi][si] else 0.0) for c in range(d)]
                   for si in range(s)]
            ln2 = [_ln64(r, w("norm2.weight"), w("norm2.bias")) for r in seq]
            hid = [[0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0)))
                    for t in _lin64(r, w("ffn_in.weight"), w("ffn_in.bias"))] for r in ln2]
            ff = [_lin64(r, w("ffn_out.weight"), w("ffn_out.bias")) for r in hid]
            xs[bi] = [[(seq[si][c] + ff[si][c]) if valid[bi][si] else 0.0 for c in range(d)]
                      for si in range(s)]
    out = np.zeros((bsz, s, d))
    for bi in range(bsz):
        for si in range(s):
            r = _ln64(xs[bi][si], p["final_norm.weight"], p["final_norm.bias"])
            out[bi, si] = r if valid[bi][si] else [0.0] * d
    return out


def check_tolerance(out16: torch.Tensor, ref: torch.Tensor, mask: Optional[torch.Tensor],
                    max_abs: float = 2e-2, mean_abs: float = 2e-3) -> dict:
    """The acceptance gate: max|d| <= 2e-2, mean|d| <= 2e-3 over [B,S,D], padded rows +0.0."""
    o = out16.detach().float().cpu()
    r = ref.detach().float().cpu()
    err = (o - r).abs()
    res = {
        "max_abs": float(err.max()) if err.numel() else 0.0,
        "mean_abs": float(err.mean()) if err.numel() else 0.0,
        "finite": bool(torch.isfinite(o).all()),
    }
    pad_ok = True
    if mask is not None and (~mask).any():
        padded = out16.detach().cpu()[~mask.cpu()]
        # bitwise +0.0: value zero and sign bit clear
        bits = padded.view(torch.int16) if padded.dtype == torch.float16 else padded.float().view(torch.int32)
        pad_ok = bool((bits == 0).all())
    res["padded_zero"] = pad_ok
    res["passed"] = (res["finite"] and res["max_abs"] <= max_abs and res["mean_abs"] <= mean_abs
                     and pad_ok)
    return res


def generate_random_case(batch: int, seq: int, d_model: int, seed: int, padding_ratio: float,
                         input_scale: float = 1.0, dtype=torch.float32):
    """CPU restatement of the reference input generator (torch_transformer_benchmark.py:234-272).

    One generator seeded with ``seed`` draws ``x ~ N(0,1) [B,S,D]`` first, then (only when
    ``padding_ratio > 0``) the right-padded prefix lengths ``U{max(1, round(S(1-r))) .. S}``;
    ``x`` is zeroed at padded positions.  With ``padding_ratio <= 0`` the mask is all-valid.
    """
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, seq, d_model, generator=gen, dtype=dtype) * input_scale
    if padding_ratio <= 0:
        return x, torch.ones(batch, seq, dtype=torch.bool)
    min_valid = max(1, int(round(seq * (1.0 - padding_ratio))))
    lengths = torch.randint(min_valid, seq + 1, (batch,), generator=gen)
    mask = torch.arange(seq)[None, :] < lengths[:, None]
    return x.masked_fill(~mask[..., None], 0), mask
