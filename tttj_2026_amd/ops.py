"""Per-kernel entry points over the C ABI, taking and returning torch tensors.

These are the building blocks ``tt_transformer_fwd`` chains; they are exposed for stage-level
parity tests and for callers that want one fused op (e.g. a GEMM with its epilogue) on its own.
Every function launches on the current stream of the input's device and raises on any error.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _half(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.float16 or t.device.type != "cuda":
        raise ValueError(f"{name} must be a CUDA float16 tensor")
    return t.contiguous()


def _mask(m: Optional[torch.Tensor], numel: int) -> Optional[torch.Tensor]:
    if m is None:
        return None
    if m.dtype != torch.bool or m.numel() != numel:
        raise ValueError(f"mask must be bool with {numel} elements")
    return m.contiguous()


def layernorm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
              valid: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    x = _half(x, "x")
    d = x.shape[-1]
    rows = x.numel() // d
    valid = _mask(valid, rows)
    y = torch.empty_like(x)
    rc = _lib.load().tt_layernorm_fwd(x.data_ptr(), _half(weight, "weight").data_ptr(),
                                      _half(bias, "bias").data_ptr(), _ptr(valid), y.data_ptr(),
                                      rows, d, eps, _stream(x))
    _lib.check(rc, "tt_layernorm_fwd")
    return y


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, epilogue: str = "bias",
           residual: Optional[torch.Tensor] = None, valid: Optional[torch.Tensor] = None,
           out: Optional[torch.Tensor] = None, seq: int = 0) -> torch.Tensor:
    """``epilogue`` in {"bias", "gelu", "resid_masked", "masked_resid"} (see tt_linear_fwd).
    ``seq`` (rows per sequence, with ``valid``) only changes the order tiles are visited in."""
    if epilogue not in ("bias", "gelu", "resid_masked", "masked_resid"):
        raise ValueError(f"unknown epilogue {epilogue!r}")
    x = _half(x, "x")
    weight = _half(weight, "weight")
    k = x.shape[-1]
    m = x.numel() // k
    n = weight.shape[0]
    if weight.shape[1] != k:
        raise ValueError("weight must be [N, K]")
    if residual is not None:
        residual = _half(residual, "residual")
        if residual.numel() != m * n:
            raise ValueError("residual must be [M, N]")
    valid = _mask(valid, m)
    y = out if out is not None else torch.empty(*x.shape[:-1], n, dtype=x.dtype, device=x.device)
    rc = _lib.load().tt_linear_fwd(x.data_ptr(), weight.data_ptr(), _half(bias, "bias").data_ptr(),
                                   _ptr(residual), _ptr(valid), y.data_ptr(), m, n, k,
                                   _lib.EPILOGUES[epilogue], 0, int(seq), 0, _stream(x))
    _lib.check(rc, "tt_linear_fwd")
    return y


def qkv_projection(x: torch.Tensor, wqkv: torch.Tensor, bqkv: torch.Tensor,
                   heads: int, valid: Optional[torch.Tensor] = None
                   ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """x [B,S,D] -> (q [B,H,S,hd], k [B,H,S,hd], vt [B,H,hd,Sp]) with Sp = S rounded up to 64.
    With ``valid`` ([B,S] bool), tokens whose mask is False get +0.0 in q, k and vt."""
    x = _half(x, "x")
    b, s, d = x.shape
    valid = _mask(valid, b * s)
    hd = d // heads
    sp = (s + 63) // 64 * 64
    plane = b * s * d
    buf = torch.empty(2 * plane + b * d * sp, dtype=torch.float16, device=x.device)
    rc = _lib.load().tt_linear_fwd(x.data_ptr(), _half(wqkv, "wqkv").data_ptr(),
                                   _half(bqkv, "bqkv").data_ptr(), None, _ptr(valid), buf.data_ptr(),
                                   b * s, 3 * d, d, _lib.EPILOGUES["qkv"], b, s, heads,
                                   _stream(x))
    _lib.check(rc, "tt_linear_fwd(qkv)")
    q = buf[:plane].view(b, heads, s, hd)
    k = buf[plane:2 * plane].view(b, heads, s, hd)
    vt = buf[2 * plane:].view(b, heads, hd, sp)
    return q, k, vt


def mask_info(mask: Optional[torch.Tensor], batch: int, seq: int, device) -> torch.Tensor:
    info = torch.empty(2 * batch, dtype=torch.int32, device=device)
    mask = _mask(mask, batch * seq)
    rc = _lib.load().tt_mask_info(_ptr(mask), info.data_ptr(), batch, seq,
                                  torch.cuda.current_stream(device).cuda_stream)
    _lib.check(rc, "tt_mask_info")
    return info


def attention(q: torch.Tensor, k: torch.Tensor, vt: torch.Tensor, mask: Optional[torch.Tensor],
              causal: bool, out: Optional[torch.Tensor] = None,
              prescaled: bool = False) -> torch.Tensor:
    """q, k [B,H,S,hd], vt [B,H,hd,Sp] (views from qkv_projection) -> ctx [B,S,H*hd].

    `out`, if given, is a contiguous fp16 [B,S,H*hd] tensor on the same device that receives ctx.
    `prescaled`: q already holds Q * hd^-1/2 * log2(e) (the forward's own Q,
    tt_attention_fwd_prescaled); otherwise the kernel applies the factor when it loads q.
    """
    b, h, s, hd = q.shape
    if k.shape != q.shape or vt.shape[:3] != (b, h, hd) or vt.shape[3] != (s + 63) // 64 * 64:
        raise ValueError("inconsistent q/k/vt shapes")
    for t, name in ((q, "q"), (k, "k"), (vt, "vt")):
        if not t.is_contiguous() or t.dtype != torch.float16:
            raise ValueError(f"{name} must be contiguous fp16")
    mask = _mask(mask, b * s)
    info = mask_info(mask, b, s, q.device) if mask is not None else None
    if out is None:
        ctx = torch.empty(b, s, h * hd, dtype=torch.float16, device=q.device)
    elif (out.shape != (b, s, h * hd) or out.dtype != torch.float16 or not out.is_contiguous()
          or out.device != q.device):
        raise ValueError("out must be a contiguous fp16 [B,S,H*hd] tensor on q's device")
    else:
        ctx = out
    fn = _lib.load().tt_attention_fwd_prescaled if prescaled else _lib.load().tt_attention_fwd
    rc = fn(q.data_ptr(), k.data_ptr(), vt.data_ptr(), _ptr(mask), _ptr(info), ctx.data_ptr(), b,
            s, h, hd, int(causal), _stream(q))
    _lib.check(rc, "tt_attention_fwd")
    return ctx
