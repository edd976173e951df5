"""CPU tests of the host side: C-ABI exports, layout bookkeeping, config validation, packing rules.

None of these launch a kernel; the library's bookkeeping exports run without a GPU.
"""

import ctypes
import pathlib
import re

import pytest
import torch

from tttj_2026_amd import _lib, check_supported, make_optimized_transformer
from tttj_2026_amd.configs import WORKLOADS, build_model
from tttj_2026_amd.model import TransformerConfig

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "tttj_amd.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(tt_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    # the Python binding declares exactly the header's functions
    assert sorted(_lib.SIGNATURES) == names


def test_version_and_error_channel():
    lib = _lib.load()
    assert b"gfx950" in lib.tt_version()
    rc = lib.tt_weight_layout(0, 1, 1, None, None, None, None)
    assert rc == _lib.TT_ERR_INVALID
    assert "bad shape" in _lib.last_error()


def test_weight_layout_matches_definition():
    for name in WORKLOADS:
        cfg = WORKLOADS[name].config
        d, f, n = cfg.d_model, cfg.ffn_dim, cfg.num_layers
        offs, stride, final, total = _lib.weight_layout(d, f, n)
        sizes = [d, d, 3 * d * d, 3 * d, d * d, d, d, d, f * d, f, d * f, d,
                 3 * d * d, 6 * d, 6 * d, f * d, 2 * f, 2 * f]
        assert len(offs) == len(sizes) == _lib.LAYER_SEGMENTS
        al = lambda v: (v + 63) // 64 * 64
        o = 0
        for i, s in enumerate(sizes):
            assert offs[i] == o and o % 64 == 0
            o += al(s)
        assert stride == o and final == n * stride and total == final + 2 * al(d)


def test_workspace_bytes_monotone_and_validated():
    small = _lib.workspace_bytes(1, 64, 256, 8, 1024)
    big = _lib.workspace_bytes(2, 4096, 1024, 16, 4096)
    assert 0 < small < big
    # C5 workspace: x, LN/ctx, Q, K, V^T, FFN hidden (fp16) ~ 144 MiB
    # activations (x', LN / context, Q, K, V^T, hidden) + partial LayerNorm statistics
    # (D / 4 float2 slots per token)
    assert big == pytest.approx((4 * 8192 * 1024 + 2 * 1024 * 4096 + 8192 * 4096) * 2
                                + 8192 * (1024 // 4) * 8, rel=1e-3)
    with pytest.raises(ValueError):
        _lib.workspace_bytes(1, 64, 240, 5, 1024)  # head_dim 48
    with pytest.raises(ValueError):  # the megakernel's attention tasks take head_dim 32 / 64
        _lib.workspace_bytes(1, 64, 256, 16, 1024, 2, _lib.PLAN_MEGAKERNEL)
    # megakernel: residual, context, Q/K/V^T, FFN hidden (fp16) + counters growing with layers
    m2 = _lib.workspace_bytes(1, 64, 256, 8, 1024, 2, _lib.PLAN_MEGAKERNEL)
    m64 = _lib.workspace_bytes(1, 64, 256, 8, 1024, 64, _lib.PLAN_MEGAKERNEL)
    assert (2 * 64 * 256 + 2 * 64 * 256 + 256 * 64 + 64 * 1024) * 2 < m2 < m64
    with pytest.raises(ValueError):  # the LayerNorm'd operand of the megakernel lives in LDS
        _lib.workspace_bytes(1, 64, 1024, 16, 4096, 2, _lib.PLAN_MEGAKERNEL)
    with pytest.raises(ValueError):
        _lib.workspace_bytes(1, 64, 256, 8, 1024, 2, 7)


def test_plan_resolution():
    # measured on MI355X: LN fused into the QKV / ffn_in tiles wins only for d_model <= 128 with
    # few tokens; C2 (64 tokens) runs the persistent megakernel, C1 layer-wise (narrow GEMM tiles)
    assert _lib.resolve_plan(1, 64, 256, 8, 1024, _lib.PLAN_AUTO) == _lib.PLAN_MEGAKERNEL     # C2
    assert _lib.resolve_plan(2, 32, 256, 4, 1024, _lib.PLAN_AUTO) == _lib.PLAN_MEGAKERNEL
    assert _lib.resolve_plan(1, 65, 256, 8, 1024, _lib.PLAN_AUTO) == _lib.PLAN_LAYERWISE
    assert _lib.resolve_plan(1, 64, 256, 16, 1024, _lib.PLAN_AUTO) == _lib.PLAN_LAYERWISE    # hd 16
    assert _lib.resolve_plan(4, 128, 256, 4, 1024, _lib.PLAN_AUTO) == _lib.PLAN_LAYERWISE     # C1
    assert _lib.resolve_plan(1, 128, 128, 4, 128, _lib.PLAN_AUTO) == _lib.PLAN_FUSED_LN       # case 2
    assert _lib.resolve_plan(1, 64, 256, 8, 1024, _lib.PLAN_MEGAKERNEL) == _lib.PLAN_MEGAKERNEL
    assert _lib.resolve_plan(1, 64, 256, 8, 1024, _lib.PLAN_LAYERWISE) == _lib.PLAN_LAYERWISE
    assert _lib.resolve_plan(8, 512, 512, 8, 2048, _lib.PLAN_AUTO) == _lib.PLAN_LAYERWISE     # C3
    assert _lib.resolve_plan(2, 4096, 1024, 16, 4096, _lib.PLAN_AUTO) == _lib.PLAN_LAYERWISE   # C5
    assert _lib.resolve_plan(1, 64, 1024, 16, 4096, _lib.PLAN_AUTO) == _lib.PLAN_LAYERWISE     # D > 512
    assert _lib.resolve_plan(2, 4096, 512, 8, 2048, _lib.PLAN_MEGAKERNEL) == _lib.PLAN_MEGAKERNEL
    # the reference's D = 128 cases: fused LN up to 2048 tokens (case 4), layer-wise beyond (case 1)
    assert _lib.resolve_plan(16, 128, 128, 4, 128, _lib.PLAN_AUTO) == _lib.PLAN_FUSED_LN
    assert _lib.resolve_plan(64, 128, 128, 4, 128, _lib.PLAN_AUTO) == _lib.PLAN_LAYERWISE
    # shapes the fused tiles do not take fall back to layer-wise (d_model 32: N = 96)
    assert _lib.resolve_plan(4, 128, 32, 4, 32, _lib.PLAN_AUTO) == _lib.PLAN_LAYERWISE
    with pytest.raises(ValueError):
        _lib.resolve_plan(1, 64, 256, 8, 1024, 7)


def _documented_auto_plan(b, s, d, h, f):
    """TT_PLAN_AUTO as include/tttj_amd.h documents it."""
    hd = d // h
    tiles64 = d % 64 == 0 and f % 64 == 0
    if b * s <= 64 and 256 <= d <= 512 and tiles64 and hd in (32, 64):
        return _lib.PLAN_MEGAKERNEL
    if tiles64 and d <= 128 and b * s <= 2048:
        return _lib.PLAN_FUSED_LN
    return _lib.PLAN_LAYERWISE


def test_auto_plan_matches_its_documentation():
    for b in (1, 2, 4, 16, 64):
        for s in (16, 32, 64, 100, 128):
            for d, h, f in ((128, 4, 128), (128, 2, 512), (256, 8, 1024), (256, 4, 1024),
                            (256, 16, 1024), (512, 8, 2048), (512, 16, 1536), (1024, 16, 4096),
                            (96, 3, 128), (256, 4, 1000), (576, 9, 2304)):
                got = _lib.resolve_plan(b, s, d, h, f, _lib.PLAN_AUTO)
                assert got == _documented_auto_plan(b, s, d, h, f), (b, s, d, h, f, got)


@pytest.mark.parametrize("kwargs,ok", [
    (dict(d_model=256, num_heads=8, ffn_dim=1024), True),     # hd 32
    (dict(d_model=1024, num_heads=16, ffn_dim=4096), True),   # hd 64
    (dict(d_model=128, num_heads=4, ffn_dim=128), True),      # the reference's own D=F shape
    (dict(d_model=256, num_heads=16, ffn_dim=1024), True),    # hd 16
    (dict(d_model=512, num_heads=4, ffn_dim=2048), True),     # hd 128
    (dict(d_model=1024, num_heads=4, ffn_dim=1024), True),    # hd 256 (reference case 8)
    (dict(d_model=32, num_heads=4, ffn_dim=32), True),        # hd 8, D = 32 (reference case 7)
    (dict(d_model=96, num_heads=3, ffn_dim=128), True),       # hd 32, D not a multiple of 64
    (dict(d_model=96, num_heads=2, ffn_dim=128), False),      # hd 48
    (dict(d_model=512, num_heads=1, ffn_dim=2048), False),    # hd 512
    (dict(d_model=256, num_heads=4, ffn_dim=1000), True),     # F a multiple of 8, not of 64
    (dict(d_model=256, num_heads=4, ffn_dim=1004), False),    # F not a multiple of 8
    (dict(d_model=12, num_heads=3, ffn_dim=16), False),       # hd 4, D not a multiple of 8
])
def test_check_supported(kwargs, ok):
    cfg = TransformerConfig(batch_size=2, seq_len=16, num_layers=2, causal=True, **kwargs)
    if ok:
        check_supported(cfg)
    else:
        with pytest.raises(ValueError, match="no optimized transformer"):
            check_supported(cfg)


def test_make_optimized_requires_gpu_fp16_params():
    model = build_model(WORKLOADS["C2"].config)  # fp32 on the CPU
    with pytest.raises(ValueError, match="CUDA float16"):
        make_optimized_transformer(model)


def test_c_abi_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    # null pointers and unsupported shapes are refused before any HIP call
    assert lib.tt_transformer_fwd(None, None, None, None, None, 0, 1, 64, 256, 8, 1024, 1, 1, 0,
                                  None) == _lib.TT_ERR_INVALID
    assert lib.tt_linear_fwd(None, None, None, None, None, None, 64, 64, 64, 0, 0, 0, 0,
                             None) == _lib.TT_ERR_INVALID
    assert lib.tt_attention_fwd(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                                None, None, ctypes.c_void_p(16), 1, 8, 1, 48, 0,
                                None) == _lib.TT_ERR_INVALID
    assert "head_dim" in _lib.last_error()
    assert lib.tt_gemm_tile_override(99) == _lib.TT_ERR_INVALID


def test_reference_case_table_is_supported():
    """Every shape of the reference's case table (optimized_transformer.py:22-42) passes the
    constructor's check, and the C ABI sizes its workspace (case 14: 3.2M tokens, > 2^31 GEMM
    operand elements) without refusing it."""
    from tttj_2026_amd.configs import REFERENCE_CASES, REFERENCE_CASE_LAYERS, reference_case_config
    assert len(REFERENCE_CASES) == 14 and REFERENCE_CASE_LAYERS[14] == 2 and REFERENCE_CASE_LAYERS[1] == 4
    for case in REFERENCE_CASES:
        cfg = reference_case_config(case)
        assert cfg.causal and cfg.ffn_dim == cfg.d_model
        check_supported(cfg)
        n = _lib.workspace_bytes(cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads,
                                 cfg.ffn_dim, cfg.num_layers)
        t = cfg.batch_size * cfg.seq_len
        assert n >= (5 * t * cfg.d_model + t * cfg.ffn_dim) * 2
    cfg = reference_case_config(14)
    assert cfg.batch_size * cfg.seq_len * cfg.d_model > 2 ** 31


def test_case_number_for_model_mirrors_reference():
    """case_number_for_model: the reference's table lookup (optimized_transformer.py:45-66) with its
    error message for shapes outside the table."""
    from tttj_2026_amd import IMPLEMENTED_CASES, case_number_for_model
    from tttj_2026_amd.configs import reference_case_config

    class Holder:  # only .config is read
        def __init__(self, config):
            self.config = config

    for case in IMPLEMENTED_CASES:
        assert case_number_for_model(Holder(reference_case_config(case))) == case
    with pytest.raises(ValueError, match="no optimized transformer is implemented for shape="):
        case_number_for_model(Holder(WORKLOADS["C5"].config))  # ffn_dim = 4 d_model
    with pytest.raises(ValueError, match="layers=3"):
        cfg = reference_case_config(1)
        case_number_for_model(Holder(TransformerConfig(cfg.batch_size, cfg.seq_len, cfg.d_model,
                                                       cfg.num_heads, cfg.ffn_dim, 3, True)))


def test_megakernel_health_check_raises_and_rearms(monkeypatch):
    """Host logic of the megakernel health word, with a stubbed status (no GPU): a non-zero word
    raises MegakernelWaitError after zero-filling the workspace, clearing the word and
    re-attaching it; a zero word does nothing."""
    from tttj_2026_amd import optimized_transformer as OT

    class _Stream:
        def synchronize(self):
            pass

    monkeypatch.setattr(OT.torch.cuda, "current_stream", lambda *a, **k: _Stream())
    cfg = TransformerConfig(1, 64, 256, 8, 1024, 4, True)
    mod = OT.OptimizedTransformer(build_model(cfg), plan=OT.PLAN_MEGAKERNEL)
    attached = []
    monkeypatch.setattr(mod, "_attach", lambda entry, b, s: attached.append((b, s)))
    ws = torch.full((64,), 7, dtype=torch.uint8)
    status = torch.zeros(1, dtype=torch.int32)
    entry = (ws, status, status.numpy())
    mod._check_mega_health(entry, 1, 64)            # healthy: nothing happens
    assert attached == [] and (ws == 7).all()
    status[0] = 1                                   # the kernel reported an expired wait
    with pytest.raises(OT.MegakernelWaitError):
        mod._check_mega_health(entry, 1, 64)
    assert (ws == 0).all() and int(status[0]) == 0 and attached == [(1, 64)]
    mod._check_mega_health(entry, 1, 64)            # re-armed
    assert attached == [(1, 64)]


def test_megakernel_workspaces_are_bounded(monkeypatch):
    """At most MEGA_WORKSPACES_KEPT megakernel workspaces are kept, least recently used dropped
    first; a shape used again keeps its workspace (and so its counters and epoch)."""
    from tttj_2026_amd import optimized_transformer as OT

    cfg = TransformerConfig(1, 64, 256, 8, 1024, 4, True)
    mod = OT.OptimizedTransformer(build_model(cfg), plan=OT.PLAN_MEGAKERNEL)
    monkeypatch.setattr(mod, "_attach", lambda entry, b, s: None)
    detached = []
    monkeypatch.setattr(mod, "_detach", lambda entry, b, s: detached.append((b, s, entry[0])))
    monkeypatch.setattr(mod, "_new_status_word", lambda: torch.zeros(1, dtype=torch.int32))
    cpu = torch.device("cpu")
    first = mod._mega_entry(1, 64, 0, 16, cpu)[0]
    for s in (65, 66, 67):
        mod._mega_entry(1, s, 0, 16, cpu)
    evicted = mod._mega[(1, 65, 0)][0]
    assert mod._mega_entry(1, 64, 0, 16, cpu)[0] is first     # reused, now most recent
    mod._mega_entry(1, 68, 0, 16, cpu)                          # evicts (1, 65)
    assert list(mod._mega) == [(1, 66, 0), (1, 67, 0), (1, 64, 0), (1, 68, 0)]
    assert len(mod._mega) == OT.MEGA_WORKSPACES_KEPT
    # the evicted workspace's status word was detached before the entry was dropped
    assert len(detached) == 1 and detached[0][:2] == (1, 65) and detached[0][2] is evicted


def test_pinned_megakernel_workspace_is_never_evicted(monkeypatch):
    """A workspace a captured graph replays on (pinned) outlives any number of other shapes."""
    from tttj_2026_amd import optimized_transformer as OT

    cfg = TransformerConfig(1, 64, 256, 8, 1024, 4, True)
    mod = OT.OptimizedTransformer(build_model(cfg), plan=OT.PLAN_MEGAKERNEL)
    monkeypatch.setattr(mod, "_attach", lambda entry, b, s: None)
    detached = []
    monkeypatch.setattr(mod, "_detach", lambda entry, b, s: detached.append((b, s)))
    monkeypatch.setattr(mod, "_new_status_word", lambda: torch.zeros(1, dtype=torch.int32))
    cpu = torch.device("cpu")
    kept = mod._mega_entry(1, 64, 0, 16, cpu)
    assert mod.pin_workspace(1, 64, 0) is kept
    for s in range(65, 75):
        mod._mega_entry(1, s, 0, 16, cpu)
    assert (1, 64, 0) in mod._mega and mod._mega[(1, 64, 0)] is kept
    assert (1, 64) not in detached
    assert len(mod._mega) == OT.MEGA_WORKSPACES_KEPT
    assert mod.pin_workspace(1, 99, 0) is None   # no workspace of that shape (another plan)


def test_stage_offsets():
    """tt_stage_offsets: the layer-wise workspace order (x', context / LN output, Q|K|V^T, hidden)
    and which plans keep the attention context."""
    T, D, F, B, S = 8192, 1024, 4096, 2, 4096
    q, c, h = _lib.stage_offsets(B, S, D, 16, F, 12, _lib.PLAN_LAYERWISE)
    assert q == 2 * T * D * 2 and c == -1 and h == q + (2 * T * D + B * D * S) * 2
    q, c, h = _lib.stage_offsets(4, 128, 256, 4, 1024, 2, _lib.PLAN_LAYERWISE)  # folded LN
    assert c == 512 * 256 * 2 and q == 2 * c
    q, c, h = _lib.stage_offsets(2, 100, 128, 4, 512, 2, _lib.PLAN_FUSED_LN)
    assert c >= 0
    n = _lib.workspace_bytes(1, 64, 256, 8, 1024, 2, _lib.PLAN_MEGAKERNEL)
    q, c, h = _lib.stage_offsets(1, 64, 256, 8, 1024, 2, _lib.PLAN_MEGAKERNEL)
    assert len({q, c, h}) == 3 and max(q, c, h) < n
    with pytest.raises(ValueError):
        _lib.stage_offsets(1, 64, 240, 5, 1024, 1, _lib.PLAN_LAYERWISE)


def test_forward_packs_rows_rule():
    """Masked layer-wise forwards whose four projections run on MFMA tiles pack the valid tokens;
    the few-token (narrow-tile, folded-LayerNorm), fused-LN and megakernel plans do not."""
    assert _lib.forward_packs_rows(8, 512, 512, 8, 2048)          # C3
    assert _lib.forward_packs_rows(8, 1024, 1024, 16, 4096)       # C4
    assert _lib.forward_packs_rows(2, 4096, 1024, 16, 4096)       # C5 (only with a mask)
    assert not _lib.forward_packs_rows(4, 128, 256, 4, 1024)      # C1: narrow tiles, LN folded
    assert not _lib.forward_packs_rows(1, 64, 256, 8, 1024)       # C2: megakernel
    assert not _lib.forward_packs_rows(2, 100, 128, 4, 512)       # fused-LN plan
    assert not _lib.forward_packs_rows(8, 512, 512, 8, 2048, _lib.PLAN_MEGAKERNEL)
    assert _lib.forward_packs_rows(8, 512, 512, 8, 2048, _lib.PLAN_LAYERWISE)
    with pytest.raises(ValueError):
        _lib.forward_packs_rows(8, 512, 512, 8, 2048, 9)


def test_packed_row_tokens_layout():
    """Host restatement of the packed layout: right-padded sequences take min(l rounded up to 8,
    S) rows (the rows past l pad to 8, token -1), other masks their valid tokens in order."""
    S = 12
    mask = torch.zeros(4, S, dtype=torch.bool)
    mask[0, :5] = True                 # prefix of 5 -> 8 rows
    mask[2, :12] = True                # full -> 12 rows
    mask[3, [1, 4, 5]] = True          # not a prefix -> its 3 valid tokens
    rows = _lib.packed_row_tokens(mask, S)
    assert rows[:8] == [0, 1, 2, 3, 4, -1, -1, -1]
    assert rows[8:20] == list(range(24, 36))     # sequence 1 is empty
    assert rows[20:] == [37, 40, 41]
    assert len(rows) == 23
    mask2 = torch.zeros(1, 10, dtype=torch.bool)
    mask2[0, :9] = True                # 9 rounds up to 16, capped at S = 10
    assert _lib.packed_row_tokens(mask2, 10) == list(range(9)) + [-1]
