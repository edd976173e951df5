"""Per-kernel parity of the HIP path (through the C ABI) against fp32 references on the same inputs.

Tolerances: the kernels read fp16 inputs, accumulate in fp32 and round the output to fp16 once,
so the references are computed in fp32 (on the CPU, from the same fp16 inputs) and the gate is a
few fp16 ulps of the output magnitude (stated per test).  Padded rows must be bitwise +0.0.
"""

import math

import pytest
import torch

from oracle import transformer_oracle as O
from tttj_2026_amd import _lib, ops

pytestmark = pytest.mark.gpu


def _rand(shape, seed, scale=1.0, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).half().to(device)


def _bits_zero(t):
    return bool((t.contiguous().view(torch.int16) == 0).all())


# ---------------------------------------------------------------- LayerNorm
@pytest.mark.parametrize("rows,d", [(1, 256), (3, 512), (1000, 1024), (77, 96), (5, 8192), (4096, 256),
                                    (8192, 1024), (20001, 512), (6000, 2048)])
def test_layernorm(device, rows, d):
    x = _rand((rows, d), 1, scale=3.0) + 0.5
    w = _rand((d,), 2, scale=0.3) + 1.0
    b = _rand((d,), 3, scale=0.3)
    valid = (torch.arange(rows) % 3 != 1).to(device)
    y = ops.layernorm(x, w, b, valid)
    torch.cuda.synchronize()
    ref = O.layer_norm(x.float().cpu(), w.float().cpu(), b.float().cpu())
    got = y.float().cpu()
    v = valid.cpu()
    err = (got[v] - ref[v]).abs().max().item()
    assert err <= 4e-3 * max(1.0, ref.abs().max().item()), err
    assert _bits_zero(y.cpu()[~v])
    y2 = ops.layernorm(x, w, b, None)
    assert (y2.float().cpu() - ref).abs().max().item() <= 4e-3 * max(1.0, ref.abs().max().item())


# ---------------------------------------------------------------- GEMM + epilogues
def _linear_ref(x, w, b):
    return x.float().cpu() @ w.float().cpu().t() + b.float().cpu()


GEMM_SHAPES = [(64, 768, 256), (100, 64, 64), (512, 1024, 256), (4096, 1536, 512),
               (8192, 1024, 4096), (1, 128, 128), (300, 3072, 1024), (200, 512, 64),
               (130, 256, 192)]


@pytest.mark.parametrize("tile", [-1, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10])
@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
def test_linear_bias_all_tiles(device, m, n, k, tile):
    if tile >= 0 and m * n * k > 2 ** 31:
        pytest.skip("large shape covered by the automatic tile")
    lib = _lib.load()
    x = _rand((m, k), 10 + m, 1.0)
    w = _rand((n, k), 11 + n, 1.0 / math.sqrt(k))
    b = _rand((n,), 12, 0.5)
    _lib.check(lib.tt_gemm_tile_override(tile), "override")
    try:
        y = ops.linear(x, w, b, "bias")
        torch.cuda.synchronize()
    finally:
        lib.tt_gemm_tile_override(-1)
    ref = _linear_ref(x, w, b)
    err = (y.float().cpu() - ref).abs().max().item()
    assert err <= 2e-3 * max(1.0, ref.abs().max().item()), (err, tile)


@pytest.mark.parametrize("m,n,k", [(512, 1024, 256), (8192, 4096, 1024), (37, 2048, 512)])
def test_linear_gelu(device, m, n, k):
    x = _rand((m, k), 20, 1.0)
    w = _rand((n, k), 21, 1.0 / math.sqrt(k))
    b = _rand((n,), 22, 0.5)
    y = ops.linear(x, w, b, "gelu")
    ref = O.gelu_erf(_linear_ref(x, w, b))
    err = (y.float().cpu() - ref).abs().max().item()
    assert err <= 2e-3 * max(1.0, ref.abs().max().item()), err


@pytest.mark.parametrize("mode", ["resid_masked", "masked_resid"])
@pytest.mark.parametrize("m,n,k", [(512, 256, 256), (4096, 512, 2048), (8192, 1024, 1024)])
def test_linear_residual_epilogues(device, mode, m, n, k):
    x = _rand((m, k), 30, 1.0)
    w = _rand((n, k), 31, 1.0 / math.sqrt(k))
    b = _rand((n,), 32, 0.5)
    r = _rand((m, n), 33, 2.0)
    valid = (torch.rand(m, generator=torch.Generator().manual_seed(34)) > 0.3).to(device)
    ref_branch = _linear_ref(x, w, b)
    rc, vc = r.float().cpu(), valid.cpu()[:, None]
    if mode == "resid_masked":
        ref = rc + torch.where(vc, ref_branch, torch.zeros(()))
    else:
        ref = torch.where(vc, rc + ref_branch, torch.zeros(()))
    y = ops.linear(x, w, b, mode, residual=r, valid=valid)
    err = (y.float().cpu() - ref).abs().max().item()
    assert err <= 3e-3 * max(1.0, ref.abs().max().item()), err
    if mode == "masked_resid":
        assert _bits_zero(y.cpu()[~valid.cpu()])
    # in place: residual aliases the output
    r2 = r.clone()
    ops.linear(x, w, b, mode, residual=r2, valid=valid, out=r2)
    assert torch.equal(r2, y)


def _padded_rows(m, seed):
    """Row mask with a long padded tail (whole tiles of every size masked), holes and a valid
    last-but-one block, so fully masked, partly masked and unmasked tiles all occur."""
    g = torch.Generator().manual_seed(seed)
    v = torch.rand(m, generator=g) > 0.2
    v[int(0.55 * m):] = False
    v[m - 70:m - 40] = True
    return v


@pytest.mark.parametrize("tile", [-1, 0, 2, 4, 5, 6, 7, 8, 9, 10])
@pytest.mark.parametrize("mode", ["bias", "gelu", "resid_masked", "masked_resid"])
@pytest.mark.parametrize("m,n,k,seq", [(1000, 512, 256, 0), (4096, 1024, 512, 0),
                                       (4096, 1024, 512, 512), (8192, 256, 256, 1024)])
def test_linear_masked_rows(device, m, n, k, seq, mode, tile):
    """With a row mask, masked rows get the mode's fill value bitwise (+0.0, or the residual for
    resid_masked) -- tiles of masked rows skip the MMA -- and valid rows match the reference."""
    lib = _lib.load()
    x = _rand((m, k), 90, 1.0)
    w = _rand((n, k), 91, 1.0 / math.sqrt(k))
    b = _rand((n,), 92, 0.5)
    r = _rand((m, n), 93, 2.0)
    if seq:   # right-padded sequences of random lengths (whole padded tiles at every tail)
        g = torch.Generator().manual_seed(94)
        lens = torch.randint(seq // 4, seq + 1, (m // seq,), generator=g)
        v = (torch.arange(seq)[None, :] < lens[:, None]).reshape(-1)
    else:
        v = _padded_rows(m, 94)
    vd = v.to(device)
    branch = _linear_ref(x, w, b)
    if mode == "gelu":
        branch = O.gelu_erf(branch)
    _lib.check(lib.tt_gemm_tile_override(tile), "override")
    try:
        if mode in ("bias", "gelu"):
            y = ops.linear(x, w, b, mode, valid=vd, seq=seq)
            ref = branch
        else:
            y = ops.linear(x, w, b, mode, residual=r, valid=vd, seq=seq)
            ref = r.float().cpu() + branch
        torch.cuda.synchronize()
    finally:
        lib.tt_gemm_tile_override(-1)
    got = y.cpu()
    err = (got.float()[v] - ref[v]).abs().max().item()
    assert err <= 3e-3 * max(1.0, ref[v].abs().max().item()), err
    if mode == "resid_masked":
        assert torch.equal(got[~v], r.cpu()[~v])
    else:
        assert _bits_zero(got[~v])


@pytest.mark.parametrize("tile", [-1, 0, 2, 4, 5, 6, 7, 8, 9, 10])
@pytest.mark.parametrize("b,s,d,h", [(4, 256, 512, 8), (3, 100, 256, 4), (2, 1024, 1024, 16),
                                     (4, 100, 32, 4), (2, 130, 96, 3), (3, 128, 128, 16),
                                     (2, 64, 1024, 4), (2, 72, 128, 1), (5, 3, 64, 2),
                                     (6, 12, 128, 4), (3, 40, 256, 2)])
def test_qkv_projection_masked_tokens(device, b, s, d, h, tile):
    """Masked tokens get +0.0 in Q, K and V^T (whole masked tiles skip the MMA); others match."""
    lib = _lib.load()
    x = _rand((b, s, d), 95)
    w = _rand((3 * d, d), 96, 1.0 / math.sqrt(d))
    bias = _rand((3 * d,), 97, 0.5)
    mask = _padded_rows(b * s, 98).reshape(b, s)
    _lib.check(lib.tt_gemm_tile_override(tile), "override")
    try:
        q, k, vt = ops.qkv_projection(x, w, bias, h, valid=mask.to(device))
        torch.cuda.synchronize()
    finally:
        lib.tt_gemm_tile_override(-1)
    hd = d // h
    ref = _linear_ref(x.reshape(-1, d), w, bias).reshape(b, s, 3, h, hd)
    ref = ref * mask[:, :, None, None, None]
    for got, want in ((q, ref[:, :, 0].permute(0, 2, 1, 3)), (k, ref[:, :, 1].permute(0, 2, 1, 3)),
                      (vt[..., :s], ref[:, :, 2].permute(0, 2, 3, 1))):
        err = (got.float().cpu() - want).abs().max().item()
        assert err <= 2e-3 * max(1.0, want.abs().max().item()), err
    qc, kc, vc = q.cpu(), k.cpu(), vt[..., :s].cpu()
    mb = ~mask
    assert _bits_zero(qc.permute(0, 2, 1, 3)[mb]) and _bits_zero(kc.permute(0, 2, 1, 3)[mb])
    assert _bits_zero(vc.permute(0, 3, 1, 2)[mb])


def test_linear_rejects_bad_shapes(device):
    x = _rand((64, 100), 1)
    w = _rand((64, 100), 2)
    b = _rand((64,), 3)
    with pytest.raises(ValueError):
        ops.linear(x, w, b)  # K = 100 is not a multiple of 8
    x = _rand((64, 64), 1)
    w = _rand((36, 64), 2)
    with pytest.raises(ValueError):
        ops.linear(x, w, _rand((36,), 3))  # N = 36 is not a multiple of 8


@pytest.mark.parametrize("mode", ["bias", "gelu", "resid_masked", "masked_resid"])
@pytest.mark.parametrize("m,n,k", [(1000, 96, 32), (37, 32, 32), (513, 40, 24), (256, 136, 200),
                                   (4096, 32, 96), (64, 64, 8)])
@pytest.mark.parametrize("masked", [False, True])
def test_linear_small_shapes(device, m, n, k, mode, masked):
    """N or K not a multiple of 64 (d_model 32, 96, ...): the vector-ALU kernel, same epilogues,
    masked rows filled bitwise as on the MFMA path."""
    x = _rand((m, k), 110 + m, 1.0)
    w = _rand((n, k), 111 + n, 1.0 / math.sqrt(k))
    b = _rand((n,), 112, 0.5)
    r = _rand((m, n), 113, 2.0)
    v = _padded_rows(m, 114) if (masked and m >= 128) else (torch.rand(m, generator=torch.Generator().manual_seed(3)) > 0.3 if masked else None)
    vd = None if v is None else v.to(device)
    branch = _linear_ref(x, w, b)
    if mode == "gelu":
        branch = O.gelu_erf(branch)
    if mode in ("bias", "gelu"):
        y = ops.linear(x, w, b, mode, valid=vd)
        ref = branch
    else:
        y = ops.linear(x, w, b, mode, residual=r, valid=vd)
        ref = r.float().cpu() + branch
    torch.cuda.synchronize()
    got = y.cpu()
    rows = torch.ones(m, dtype=torch.bool) if v is None else v
    err = (got.float()[rows] - ref[rows]).abs().max().item() if rows.any() else 0.0
    assert err <= 3e-3 * max(1.0, ref.abs().max().item()), err
    if v is not None and (~v).any():
        if mode == "resid_masked":
            assert torch.equal(got[~v], r.cpu()[~v])
        else:
            assert _bits_zero(got[~v])


# ---------------------------------------------------------------- QKV layout + attention
@pytest.mark.parametrize("b,s,d,h", [(2, 64, 256, 8), (1, 100, 128, 2), (3, 128, 512, 8),
                                     (11, 6, 64, 1), (9, 24, 512, 4), (4, 200, 256, 2)])
def test_qkv_projection_layout(device, b, s, d, h):
    x = _rand((b, s, d), 40)
    w = _rand((3 * d, d), 41, 1.0 / math.sqrt(d))
    bias = _rand((3 * d,), 42, 0.5)
    q, k, vt = ops.qkv_projection(x, w, bias, h)
    torch.cuda.synchronize()
    hd = d // h
    ref = _linear_ref(x.reshape(-1, d), w, bias).reshape(b, s, 3, h, hd)
    for got, want in ((q, ref[:, :, 0].permute(0, 2, 1, 3)), (k, ref[:, :, 1].permute(0, 2, 1, 3)),
                      (vt[..., :s], ref[:, :, 2].permute(0, 2, 3, 1))):
        err = (got.float().cpu() - want).abs().max().item()
        assert err <= 2e-3 * max(1.0, want.abs().max().item()), err


def _attention_ref(q, k, vt, mask, causal):
    """fp32 CPU softmax(q k^T / sqrt(hd)) v with -inf masks; rows with no key -> 0."""
    b, h, s, hd = q.shape
    qf, kf = q.float().cpu(), k.float().cpu()
    vf = vt[..., :s].float().cpu().transpose(-1, -2).contiguous()
    sc = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) / math.sqrt(hd)
    allowed = torch.ones(b, 1, s, s, dtype=torch.bool)
    if causal:
        allowed &= ~torch.ones(s, s, dtype=torch.bool).triu(1)
    if mask is not None:
        allowed &= mask.cpu()[:, None, None, :]
    sc = sc.masked_fill(~allowed, float("-inf"))
    p = torch.softmax(sc, dim=-1).nan_to_num(0.0)
    return torch.matmul(p, vf).permute(0, 2, 1, 3).reshape(b, s, h * hd)


def _masks(kind, b, s, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "none":
        return None
    if kind == "all":
        return torch.ones(b, s, dtype=torch.bool)
    if kind == "prefix":
        lens = torch.randint(max(1, s // 2), s + 1, (b,), generator=g)
        lens[0] = s
        return torch.arange(s)[None, :] < lens[:, None]
    if kind == "ragged_empty":
        lens = torch.randint(0, s + 1, (b,), generator=g)
        lens[-1] = 0
        return torch.arange(s)[None, :] < lens[:, None]
    m = torch.rand(b, s, generator=g) > 0.35  # non-prefix
    m[:, 0] = True
    return m


@pytest.mark.parametrize("hd", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("s", [1, 37, 64, 128, 200, 512])
@pytest.mark.parametrize("mask_kind", ["none", "prefix", "nonprefix", "ragged_empty"])
def test_attention(device, hd, causal, s, mask_kind):
    b, h = 3, 2
    q = _rand((b, h, s, hd), 50 + s, 1.5)
    k = _rand((b, h, s, hd), 51 + s, 1.5)
    sp = (s + 63) // 64 * 64
    vt = _rand((b, h, hd, sp), 52 + s, 1.0)
    vt[..., s:] = float("nan")  # padding columns must never be read into the result
    mask = _masks(mask_kind, b, s, 53 + s)
    mdev = None if mask is None else mask.to(device)
    ctx = ops.attention(q, k, vt, mdev, causal)
    torch.cuda.synchronize()
    ref = _attention_ref(q, k, vt, mask, causal)
    got = ctx.float().cpu()
    assert torch.isfinite(got).all()
    if mask is not None:
        assert _bits_zero(ctx.cpu()[~mask])
        got, ref = got[mask], ref[mask]
    if got.numel():
        err = (got - ref).abs().max().item()
        assert err <= 6e-3, err


@pytest.mark.parametrize("hd", [8, 32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("s", [200, 2100])
@pytest.mark.parametrize("mask_kind", ["none", "prefix", "nonprefix"])
def test_attention_prescaled_entry(device, hd, causal, s, mask_kind):
    """tt_attention_fwd_prescaled (Q already multiplied by hd^-1/2 log2 e and rounded once, the
    form the forward's QKV epilogue writes) against tt_attention_fwd, which applies the factor
    when it loads Q: the MFMA kernels round Q * factor to fp16 the same way, so the two agree
    bit for bit; the head_dim 8 / 16 kernel keeps Q * factor in fp32, so there they agree to
    rounding."""
    b, h = 2, 2
    q = _rand((b, h, s, hd), 90 + s, 1.5)
    k = _rand((b, h, s, hd), 91 + s, 1.5)
    vt = _rand((b, h, hd, (s + 63) // 64 * 64), 92 + s, 1.0)
    mask = _masks(mask_kind, b, s, 93 + s)
    mdev = None if mask is None else mask.to(device)
    f32 = lambda v: torch.tensor(v, dtype=torch.float32)
    factor = (f32(1.0) / torch.sqrt(f32(float(hd)))) * f32(1.4426950408889634)
    qs = (q.float() * factor.to(device)).half()
    a = ops.attention(q, k, vt, mdev, causal)
    c = ops.attention(qs, k, vt, mdev, causal, prescaled=True)
    torch.cuda.synchronize()
    if hd >= 32:
        assert torch.equal(a, c)
    else:
        assert (a.float() - c.float()).abs().max().item() <= 4e-3


@pytest.mark.parametrize("hd", [32, 64])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("s", [2048, 2100])
@pytest.mark.parametrize("mask_kind", ["none", "prefix", "nonprefix", "ragged_empty"])
def test_attention_long_ring(device, hd, causal, s, mask_kind):
    """Sequences of 2048 keys and more run the three-tile key ring (head_dim <= 64); 2100 ends in
    a partial tile."""
    b, h = 2, 2
    q = _rand((b, h, s, hd), 70 + s, 1.5)
    k = _rand((b, h, s, hd), 71 + s, 1.5)
    sp = (s + 63) // 64 * 64
    vt = _rand((b, h, hd, sp), 72 + s, 1.0)
    vt[..., s:] = float("nan")
    mask = _masks(mask_kind, b, s, 73 + s)
    ctx = ops.attention(q, k, vt, None if mask is None else mask.to(device), causal)
    torch.cuda.synchronize()
    ref = _attention_ref(q, k, vt, mask, causal)
    got = ctx.float().cpu()
    assert torch.isfinite(got).all()
    if mask is not None:
        assert _bits_zero(ctx.cpu()[~mask])
        got, ref = got[mask], ref[mask]
    if got.numel():
        assert (got - ref).abs().max().item() <= 6e-3


@pytest.mark.parametrize("b,s,h,hd,causal", [(2, 4096, 16, 64, True), (8, 1024, 16, 64, True),
                                              (8, 512, 8, 64, False), (1, 64, 8, 32, True)])
def test_attention_benchmark_shapes(device, b, s, h, hd, causal):
    q = _rand((b, h, s, hd), 60, 1.0)
    k = _rand((b, h, s, hd), 61, 1.0)
    vt = _rand((b, h, hd, (s + 63) // 64 * 64), 62, 1.0)
    mask = _masks("prefix", b, s, 63) if b == 8 else None
    # NaN-filled output: every (sequence, head, query tile) block must write its rows, so a block
    # order that skips or repeats a tile leaves NaN behind.
    ctx = torch.full((b, s, h * hd), float("nan"), dtype=torch.float16, device=device)
    ops.attention(q, k, vt, None if mask is None else mask.to(device), causal, out=ctx)
    torch.cuda.synchronize()
    assert torch.isfinite(ctx).all().item()
    # full fp32 reference for the first sequence (the full reference is large) ...
    sl = slice(0, 1)
    ref = _attention_ref(q[sl], k[sl], vt[sl], None if mask is None else mask[sl], causal)
    got = ctx[sl].float().cpu()
    if mask is not None:
        got, ref = got[mask[sl]], ref[mask[sl]]
    assert (got - ref).abs().max().item() <= 6e-3
    # ... and, for every sequence and head, the first and last row of every query tile
    rows = sorted({r for t in range(0, s, 128) for r in (t, min(t + 127, s - 1))})
    qf, kf = q.float().cpu(), k.float().cpu()
    vf = vt[..., :s].float().cpu()
    sc = torch.matmul(qf[:, :, rows], kf.transpose(-1, -2).contiguous()) / math.sqrt(hd)
    allowed = torch.ones(b, 1, len(rows), s, dtype=torch.bool)
    if causal:
        allowed &= torch.arange(s)[None, :] <= torch.tensor(rows)[:, None]
    if mask is not None:
        allowed &= mask[:, None, None, :]
    p = torch.softmax(sc.masked_fill(~allowed, float("-inf")), dim=-1).nan_to_num(0.0)
    ref = torch.matmul(p, vf.transpose(-1, -2).contiguous()).permute(0, 2, 1, 3).reshape(b, len(rows), h * hd)
    got = ctx[:, rows].float().cpu()
    if mask is not None:
        ref = ref * mask[:, rows, None]  # padded query rows are written as zeros
    assert (got - ref).abs().max().item() <= 6e-3


@pytest.mark.parametrize("causal", [False, True])
def test_attention_large_scores(device, causal):
    """Scores up to ~43 in the log2 domain, growing along the keys, so that the reference max of
    every row moves several times (lazy rescaling).  Through the C ABI, q arrives unscaled and the
    kernel rounds q hd^-1/2 log2(e) to fp16 when it loads it; that second rounding alone moves
    this output by up to ~3e-3 (fp64 model of it), within the bound of the other attention tests.
    The forward's Q comes out of the QKV epilogue already multiplied (one rounding, as unscaled Q
    would have)."""
    b, s, h, hd = 1, 2048, 2, 64
    g = torch.Generator().manual_seed(5)
    q = (torch.randn(b, h, s, hd, generator=g) * 2.0).half().to(device)
    k = (torch.randn(b, h, s, hd, generator=g)
         * torch.linspace(0.2, 3.0, s)[None, None, :, None]).half().to(device)
    vt = _rand((b, h, hd, s), 81, 1.0)
    got = ops.attention(q, k, vt, None, causal)
    torch.cuda.synchronize()
    ref = _attention_ref(q, k, vt, None, causal)
    assert (got.float().cpu() - ref).abs().max().item() <= 6e-3


def test_attention_rejects_head_dim(device):
    q = _rand((1, 1, 8, 48), 1)
    vt = _rand((1, 1, 48, 64), 2)
    with pytest.raises(ValueError):
        ops.attention(q, q, vt, None, False)


def test_mask_info(device):
    mask = torch.tensor([[1, 1, 1, 0, 0], [1, 0, 1, 0, 0], [0, 0, 0, 0, 0], [1, 1, 1, 1, 1]],
                        dtype=torch.bool)
    info = ops.mask_info(mask.to(device), 4, 5, device).cpu().tolist()
    assert info == [3, 3, 0, 5, 1, 0, 1, 1]
    info = ops.mask_info(None, 2, 7, device).cpu().tolist()
    assert info == [7, 7, 1, 1]


def test_gelu_epilogue_matches_exact_erf_gelu(device):
    """GELU epilogue on every fp16 pre-activation in [-12, 12]: the GEMM is arranged so that the
    accumulator equals the value exactly (x = [v, 0, ...], every weight row = e_0, bias 0), and the
    fp16 output must equal the correctly rounded exact-erf GELU (float64 math.erf) up to one fp16
    ulp, with at most 0.1% of values off by that ulp (values next to a rounding tie)."""
    vals = torch.arange(-(2 ** 15), 2 ** 15, dtype=torch.int32).to(torch.int16).view(torch.float16)
    vals = vals[torch.isfinite(vals) & (vals.float().abs() <= 12)]
    m, n, k = vals.numel(), 64, 64
    x = torch.zeros(m, k, dtype=torch.float16)
    x[:, 0] = vals
    w = torch.zeros(n, k, dtype=torch.float16)
    w[:, 0] = 1
    y = ops.linear(x.to(device), w.to(device), torch.zeros(n, dtype=torch.float16, device=device),
                   "gelu")
    torch.cuda.synchronize()
    got = y[:, 0].cpu()
    assert (y.cpu() == got[:, None]).all()           # every output column is the same function
    v64 = vals.double()
    exact = 0.5 * v64 * (1.0 + torch.erf(v64 / math.sqrt(2.0)))
    want = exact.half()
    ulp = (got.view(torch.int16).int() - want.view(torch.int16).int()).abs()
    ulp = torch.where((got == 0) & (want == 0), torch.zeros_like(ulp), ulp)  # +0 vs -0
    assert ulp.max().item() <= 1
    assert (ulp > 0).float().mean().item() < 1e-3
    err = (got.double() - exact).abs()
    half_ulp = (want.double().abs().clamp_min(2 ** -14) * 2 ** -11)
    assert (err <= half_ulp + 1e-6).all()
