"""Public construction API: ``make_optimized_transformer(model)`` -> module with ``forward(x, mask)``.

Drop-in for ``optimized_transformer.make_optimized_transformer`` (optimized_transformer.py:69-93):
the same signature and the same ``forward(x, valid_token_mask=None)`` contract
(kernels/sequence_resident.py:227-233).  Instead of the reference's table of 14 fixed shapes
(optimized_transformer.py:22-66) any configuration with ``head_dim in {8, 16, 32, 64, 128, 256}``,
``d_model`` and ``ffn_dim`` multiples of 8 and ``d_model <= 8192`` is accepted, causal or not --
every shape of that table included (``SUPPORTED_HEAD_DIMS``); anything else raises
``ValueError`` before any work, as the reference does for unsupported shapes.

The module packs the parameter model's fp16 weights once (``prepare``) into the layout of
``tt_weight_layout`` and runs every forward as one call into the HIP library on the caller's
current stream: either the layer-wise plan (LN, four GEMMs with fused epilogues and attention per
layer) or, for small token counts, the persistent megakernel (one launch for the whole
stack, workgroups handing work to each other through dependency counters); ``plan`` forces one.
It returns a fresh output tensor per call; repeated calls on the same inputs are bit-identical.
A module instance owns one scratch workspace per device for the layer-wise plans (grown to the
largest shape seen and reused for smaller ones) and a few megakernel workspaces (the most recent
``MEGA_WORKSPACES_KEPT`` (batch, seq) shapes; each holds that shape's dependency counters and launch
epoch, so it is zero-filled once and then reused), and is not re-entrant across streams (the
reference's scheduler buffer has the same contract, kernels/sequence_resident.py:148-150).

The megakernel's dependency waits are bounded; a wait that gives up makes that launch write NaN
over its output and sets an error flag that the kernel mirrors into a pinned host word.  The next
``forward`` on that shape reads the word (host memory, no synchronisation) and raises
``MegakernelWaitError`` after re-arming the workspace, so one expiry never turns into silently
wrong results.
"""

from __future__ import annotations

import ctypes
from collections import OrderedDict
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn

from . import _lib
from .configs import REFERENCE_CASE_LAYERS, REFERENCE_CASES

PLAN_AUTO, PLAN_LAYERWISE, PLAN_MEGAKERNEL, PLAN_FUSED_LN = (
    _lib.PLAN_AUTO, _lib.PLAN_LAYERWISE, _lib.PLAN_MEGAKERNEL, _lib.PLAN_FUSED_LN)


SUPPORTED_HEAD_DIMS = (8, 16, 32, 64, 128, 256)

# Megakernel workspaces kept per module (least recently used ones are dropped beyond this).
MEGA_WORKSPACES_KEPT = 4


class MegakernelWaitError(RuntimeError):
    """A dependency wait of the persistent megakernel gave up (the device did not run all of its
    workgroups at once, e.g. because other kernels held CUs); that launch's output was NaN."""

# The reference's public case table under its own names (optimized_transformer.py:22-42); this
# build accepts those shapes and more (check_supported), the table is kept for callers that use it.
IMPLEMENTED_CASES = REFERENCE_CASES
IMPLEMENTED_CASE_LAYERS = REFERENCE_CASE_LAYERS


def case_number_for_model(parameter_model: nn.Module) -> int:
    """The reference case (optimized_transformer.py:45-66) whose shape ``parameter_model`` has:
    causal, ffn_dim == d_model, (batch, seq, d_model, heads) and the layer count of one table
    entry; ``ValueError`` otherwise, with the reference's message."""
    cfg = parameter_model.config
    shape = (cfg.batch_size, cfg.seq_len, cfg.d_model, cfg.num_heads)
    if cfg.ffn_dim == cfg.d_model and cfg.causal:
        for case, case_shape in IMPLEMENTED_CASES.items():
            if shape == case_shape and cfg.num_layers == IMPLEMENTED_CASE_LAYERS[case]:
                return case
    raise ValueError(f"no optimized transformer is implemented for shape={shape}, "
                     f"ffn_dim={cfg.ffn_dim}, layers={cfg.num_layers}, causal={cfg.causal}")


def check_supported(config) -> None:
    """Raise ValueError unless the HIP path implements ``config`` (a TransformerConfig-like)."""
    d, h, f = config.d_model, config.num_heads, config.ffn_dim
    problems = []
    if min(config.batch_size, config.seq_len, d, h, f, config.num_layers) <= 0:
        problems.append("all sizes must be positive")
    elif d % h != 0:
        problems.append(f"d_model {d} not divisible by num_heads {h}")
    else:
        if d // h not in SUPPORTED_HEAD_DIMS:
            problems.append(f"head_dim {d // h} not in {SUPPORTED_HEAD_DIMS}")
        if d % 8 or f % 8:
            problems.append("d_model and ffn_dim must be multiples of 8")
        if d > 8192:
            problems.append("d_model must be <= 8192")
    if problems:
        raise ValueError(
            "no optimized transformer is implemented for "
            f"shape={(config.batch_size, config.seq_len, d, h)}, ffn_dim={f}, "
            f"layers={config.num_layers}, causal={config.causal}: " + "; ".join(problems))


def pack_model_weights(model: nn.Module) -> torch.Tensor:
    """Pack ``model``'s parameters into one contiguous fp16 buffer in the C-ABI layout.

    Generalises kernels/sequence_resident.py:74-109 (F == D only) to any F; q, k and v weights and
    biases are concatenated into one [3D, D] projection.  Segment offsets come from the library
    (``tt_weight_layout``) so Python and C cannot disagree about the layout; the derived segments
    (LayerNorm gains and biases folded into the QKV and ffn_in weights) are computed on the device
    by ``tt_pack_derived``.
    """
    cfg = model.config
    d, f, n_layers = cfg.d_model, cfg.ffn_dim, cfg.num_layers
    offs, stride, final, total = _lib.weight_layout(d, f, n_layers)
    ref = model.final_norm.weight
    if ref.device.type != "cuda" or ref.dtype != torch.float16:
        raise ValueError("parameters must be CUDA float16 before prepare()")
    packed = torch.zeros(total, dtype=torch.float16, device=ref.device)

    def put(base: int, seg: int, *tensors: torch.Tensor) -> None:
        o = base + offs[seg]
        for t in tensors:
            t = t.detach()
            if t.dtype != torch.float16 or t.device != ref.device:
                raise ValueError("all parameters must be CUDA float16 on one device")
            packed[o:o + t.numel()].copy_(t.reshape(-1))
            o += t.numel()

    for i, layer in enumerate(model.layers):
        base = i * stride
        att = layer.attention
        for lin in (att.q_proj, att.k_proj, att.v_proj, att.out_proj, layer.ffn_in, layer.ffn_out):
            if lin.bias is None:
                raise ValueError("every projection must have a bias")
        put(base, 0, layer.norm1.weight)
        put(base, 1, layer.norm1.bias)
        put(base, 2, att.q_proj.weight, att.k_proj.weight, att.v_proj.weight)
        put(base, 3, att.q_proj.bias, att.k_proj.bias, att.v_proj.bias)
        put(base, 4, att.out_proj.weight)
        put(base, 5, att.out_proj.bias)
        put(base, 6, layer.norm2.weight)
        put(base, 7, layer.norm2.bias)
        put(base, 8, layer.ffn_in.weight)
        put(base, 9, layer.ffn_in.bias)
        put(base, 10, layer.ffn_out.weight)
        put(base, 11, layer.ffn_out.bias)
    dpad = (d + 63) // 64 * 64
    packed[final:final + d].copy_(model.final_norm.weight.detach().reshape(-1))
    packed[final + dpad:final + dpad + d].copy_(model.final_norm.bias.detach().reshape(-1))
    # segments 12-17: the LayerNorms folded into the projections that follow them
    lib = _lib.load()
    _lib.check(lib.tt_pack_derived(packed.data_ptr(), d, f, n_layers,
                                   torch.cuda.current_stream(packed.device).cuda_stream),
               "tt_pack_derived")
    return packed


class OptimizedTransformer(nn.Module):
    """Inference-only module running the pre-LN stack through the gfx950 HIP library."""

    def __init__(self, parameter_model: nn.Module, plan: int = PLAN_AUTO) -> None:
        super().__init__()
        if plan not in (PLAN_AUTO, PLAN_LAYERWISE, PLAN_MEGAKERNEL, PLAN_FUSED_LN):
            raise ValueError(f"unknown plan {plan}")
        self.parameter_model = parameter_model
        self.config = parameter_model.config
        self.plan = plan
        self.register_buffer("packed_weights", None, persistent=False)
        # layer-wise plans: one scratch buffer per device, grown to the largest shape seen
        self._scratch: Dict[int, torch.Tensor] = {}
        # megakernel plan: (batch, seq, device) -> (workspace, pinned host error word, its numpy
        # view)
        self._mega: "OrderedDict[Tuple[int, int, int], Tuple[torch.Tensor, torch.Tensor]]" = \
            OrderedDict()
        self._nbytes: Dict[Tuple[int, int, int], int] = {}
        self.last_workspace: Optional[torch.Tensor] = None
        self.last_mask: Optional[torch.Tensor] = None
        self._pinned = set()  # megakernel workspaces a captured graph holds

    def prepare(self) -> None:
        check_supported(self.config)
        lib = _lib.load()
        self.packed_weights = pack_model_weights(self.parameter_model)
        self._lib = lib

    def _workspace(self, batch: int, seq: int, plan: int, device: torch.device) -> torch.Tensor:
        cfg = self.config
        nbytes = self._nbytes.get((batch, seq, plan))
        if nbytes is None:
            nbytes = _lib.workspace_bytes(batch, seq, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
                                          cfg.num_layers, plan)
            if len(self._nbytes) >= 256:
                self._nbytes.clear()
            self._nbytes[(batch, seq, plan)] = nbytes
        dev = device.index if device.index is not None else 0
        if plan == PLAN_MEGAKERNEL:
            return self._mega_entry(batch, seq, dev, nbytes, device)[0]
        ws = self._scratch.get(dev)
        if ws is None or ws.numel() < nbytes:
            # the previous buffer is released here unless a captured graph still holds it
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            self._scratch[dev] = ws
        return ws

    def _mega_entry(self, batch, seq, dev, nbytes, device):
        key = (batch, seq, dev)
        entry = self._mega.pop(key, None)
        if entry is None:
            # zero-filled: the dependency counters and epoch must start at 0
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
            status = self._new_status_word()
            entry = (ws, status, status.numpy())  # the numpy view reads host memory cheaply
            self._attach(entry, batch, seq)
        self._mega[key] = entry  # most recently used last
        while len(self._mega) > MEGA_WORKSPACES_KEPT:
            # least recently used first; a workspace a captured graph replays on is never dropped
            victim = next((k for k in self._mega if k not in self._pinned), None)
            if victim is None:
                break
            self._detach(self._mega.pop(victim), victim[0], victim[1])
        return entry

    @staticmethod
    def _new_status_word() -> torch.Tensor:
        return torch.zeros(1, dtype=torch.int32, pin_memory=True)

    def _attach(self, entry, batch, seq) -> None:
        ws, status, _ = entry
        cfg = self.config
        _lib.check(self._lib.tt_megakernel_attach_status(
            ws.data_ptr(), ws.numel(), batch, seq, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
            cfg.num_layers, status.data_ptr(),
            torch.cuda.current_stream(ws.device).cuda_stream), "tt_megakernel_attach_status")

    def _detach(self, entry, batch, seq) -> None:
        """Before a workspace and its pinned status word are dropped: detach the word, ordered
        after the workspace's last launch (whose final workgroup writes through the attached
        address), and wait for that point, so the freed word is never written."""
        ws, _, _ = entry
        cfg = self.config
        stream = torch.cuda.current_stream(ws.device)
        _lib.check(self._lib.tt_megakernel_attach_status(
            ws.data_ptr(), ws.numel(), batch, seq, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
            cfg.num_layers, None, stream.cuda_stream), "tt_megakernel_attach_status")
        stream.synchronize()

    def pin_workspace(self, batch: int, seq: int, device_index: int):
        """Keep the megakernel workspace of (batch, seq) and its status word for good (a captured
        graph replays on them) and return that entry; None for other plans."""
        key = (batch, seq, device_index)
        entry = self._mega.get(key)
        if entry is not None:
            self._pinned.add(key)
        return entry

    def _check_mega_health(self, entry, batch, seq) -> None:
        """Raise MegakernelWaitError if an earlier launch on this workspace reported a wait that
        gave up (its output was NaN), after re-arming the workspace: synchronise, zero-fill,
        re-attach the host word and clear it."""
        ws, status, word = entry
        if word[0] == 0:
            return
        torch.cuda.current_stream(ws.device).synchronize()  # no launch may still write the word
        ws.zero_()
        status[0] = 0
        self._attach(entry, batch, seq)
        raise MegakernelWaitError(
            "megakernel: a dependency wait gave up in an earlier forward on this shape (its "
            "output was NaN); the workspace has been reset")

    def forward_traced(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None):
        """Megakernel forward that also returns its per-task trace: an int64 [tasks, 4] CPU
        tensor of (task | workgroup << 32, start, ready, end) on the GPU's 100 MHz clock, where
        `ready` is when the task's dependencies were satisfied (tracing of the persistent plan,
        after the reference's capture slots, kernels/fused_megakernel.py:20-26)."""
        if self.packed_weights is None:
            self.prepare()
        cfg = self.config
        x = x.contiguous()
        batch, seq, _ = x.shape
        mask = None if valid_token_mask is None else valid_token_mask.contiguous()
        ntask = self._lib.tt_megakernel_tasks(batch, seq, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
                                              cfg.num_layers)
        if ntask < 0:
            raise ValueError(f"tt_megakernel_tasks: {_lib.last_error()}")
        trace = torch.zeros(4 * ntask, dtype=torch.int64, device=x.device)
        ws = self._workspace(batch, seq, PLAN_MEGAKERNEL, x.device)
        y = torch.empty_like(x)
        rc = self._lib.tt_megakernel_trace_fwd(
            self.packed_weights.data_ptr(), x.data_ptr(), None if mask is None else mask.data_ptr(),
            y.data_ptr(), ws.data_ptr(), ws.numel(), batch, seq, cfg.d_model, cfg.num_heads,
            cfg.ffn_dim, cfg.num_layers, int(bool(cfg.causal)), trace.data_ptr(), trace.numel(),
            torch.cuda.current_stream(x.device).cuda_stream)
        _lib.check(rc, "tt_megakernel_trace_fwd")
        return y, trace.view(ntask, 4).cpu()

    def megakernel_status(self, batch: int, seq: int) -> int:
        """0 if every dependency wait of the megakernel workspace for (batch, seq) completed so
        far, 1 if one exceeded its bound (synchronises the current stream)."""
        cfg = self.config
        dev = self.packed_weights.device
        entry = self._mega.get((batch, seq, dev.index or 0))
        if entry is None:
            return 0
        status = ctypes.c_int(0)
        _lib.check(self._lib.tt_megakernel_status(
            entry[0].data_ptr(), batch, seq, cfg.d_model, cfg.ffn_dim, cfg.num_layers,
            ctypes.byref(status), torch.cuda.current_stream(dev).cuda_stream),
            "tt_megakernel_status")
        return status.value

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None):
        if self.packed_weights is None:
            self.prepare()
        cfg = self.config
        if x.dim() != 3 or x.shape[2] != cfg.d_model:
            raise ValueError(f"x must be [B, S, {cfg.d_model}], got {tuple(x.shape)}")
        if x.dtype != torch.float16 or x.device.type != "cuda":
            raise ValueError("x must be a CUDA float16 tensor")
        if self.packed_weights.device != x.device or self.packed_weights.dtype != torch.float16:
            raise ValueError("packed weights and input must be fp16 on the same device")
        batch, seq, _ = x.shape
        x = x.contiguous()
        mask_ptr = None
        if valid_token_mask is not None:
            if valid_token_mask.shape != (batch, seq) or valid_token_mask.dtype != torch.bool:
                raise ValueError("valid_token_mask must be a bool [B, S] tensor")
            if valid_token_mask.device != x.device:
                raise ValueError("valid_token_mask must be on the input's device")
            valid_token_mask = valid_token_mask.contiguous()
            mask_ptr = valid_token_mask.data_ptr()
        y = torch.empty_like(x)
        if batch * seq == 0:
            return y
        plan = _lib.resolve_plan(batch, seq, cfg.d_model, cfg.num_heads, cfg.ffn_dim, self.plan)
        ws = self._workspace(batch, seq, plan, x.device)
        if plan == PLAN_MEGAKERNEL:
            self._check_mega_health(self._mega[(batch, seq, x.device.index or 0)], batch, seq)
        self.last_workspace = ws
        self.last_mask = valid_token_mask
        stream = torch.cuda.current_stream(x.device).cuda_stream
        rc = self._lib.tt_transformer_fwd(
            self.packed_weights.data_ptr(), x.data_ptr(), mask_ptr, y.data_ptr(), ws.data_ptr(),
            ws.numel(), batch, seq, cfg.d_model, cfg.num_heads, cfg.ffn_dim, cfg.num_layers,
            int(bool(cfg.causal)), plan, stream)
        _lib.check(rc, "tt_transformer_fwd")
        return y


    def captured_stages(self, batch: int, seq: int) -> Dict[str, Optional[torch.Tensor]]:
        """Intermediates of the LAST layer of the most recent forward of shape (batch, seq), read
        back from its workspace (the fused plans never materialise them otherwise; the reference
        captures them from inside its fused kernels for its stage checks):
        ``q``, ``k``, ``v`` [B, H, S, hd] (q divided back by the softmax factor the projection
        applies), ``ctx`` [B, S, D] (None where the plan overwrites it) and ``hidden`` [B, S, F]
        (GELU output).  Valid until the next forward on this module."""
        cfg = self.config
        plan = _lib.resolve_plan(batch, seq, cfg.d_model, cfg.num_heads, cfg.ffn_dim, self.plan)
        ws = self.last_workspace
        if ws is None:
            raise RuntimeError("no forward has run on this module")
        oq, oc, oh = _lib.stage_offsets(batch, seq, cfg.d_model, cfg.num_heads, cfg.ffn_dim,
                                        cfg.num_layers, plan)
        d, h, f = cfg.d_model, cfg.num_heads, cfg.ffn_dim
        hd, t, sp = d // h, batch * seq, (seq + 63) // 64 * 64

        def view(off: int, n: int) -> torch.Tensor:
            return ws[off:off + 2 * n].view(torch.float16)

        plane = t * d
        qkv = view(oq, 2 * plane + batch * d * sp)
        scale = hd ** -0.5 * 1.4426950408889634
        q = (qkv[:plane].view(batch, h, seq, hd).float() / scale).half()
        k = qkv[plane:2 * plane].view(batch, h, seq, hd)
        v = qkv[2 * plane:].view(batch, h, hd, sp)[..., :seq].transpose(-1, -2)
        ctx = None if oc < 0 else view(oc, t * d).view(batch, seq, d)
        hidden = view(oh, t * f).view(t, f)
        mask = self.last_mask
        if mask is not None and plan != PLAN_MEGAKERNEL and _lib.forward_packs_rows(
                batch, seq, d, h, f, plan):
            # packed variable-length rows: scatter the valid tokens' rows back to [B, S, F]
            rows = torch.tensor(_lib.packed_row_tokens(mask.cpu(), seq), dtype=torch.long)
            keep = rows >= 0
            full = torch.zeros(t, f, dtype=hidden.dtype, device=hidden.device)
            full[rows[keep].to(hidden.device)] = hidden[:rows.numel()][keep.to(hidden.device)]
            hidden = full
        hidden = hidden.view(batch, seq, f)
        return {"q": q, "k": k, "v": v, "ctx": ctx, "hidden": hidden}


class GraphedOptimizedTransformer(nn.Module):
    """HIP-graph replay around an ``OptimizedTransformer`` (the reference's
    ``GraphedHybridTransformer``, kernels/layerwise_hybrid.py:364-446).

    The first call with a given (input allocation, mask allocation, shape) captures the whole
    forward -- the single ``tt_transformer_fwd`` call and the launches it makes -- into one graph,
    after warm-up calls on a side stream that create the workspace and run the library's one-time
    set-up outside the capture.  Later calls whose input and mask live at the captured addresses
    replay the graph: the graph reads those buffers at replay time, so new contents written into
    the same allocations are picked up.  A call with any other input or mask allocation runs the
    eager module instead (as the reference does for a different pointer, :440-441).

    Output aliasing is the reference's: replay returns the graph's **static** output tensor, which
    the next replay overwrites; callers that keep results across calls must ``.clone()`` them
    (benchmarks/regression.py:123).  Nothing inside the captured forward clears memory with a
    memset: the workspace is zero-filled once before capture, and the megakernel's launch epoch
    lives in device memory, so every replay advances it.
    """

    def __init__(self, module: OptimizedTransformer) -> None:
        super().__init__()
        self.module = module
        self.config = module.config
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._key = None
        self._static_input: Optional[torch.Tensor] = None
        self._static_mask: Optional[torch.Tensor] = None
        self._static_output: Optional[torch.Tensor] = None
        self._static_workspace: Optional[torch.Tensor] = None
        self._static_entry = None

    @staticmethod
    def _signature(x: torch.Tensor, mask: Optional[torch.Tensor]):
        return (x.data_ptr(), tuple(x.shape), x.device,
                None if mask is None else (mask.data_ptr(), tuple(mask.shape)))

    def capture(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> None:
        """Capture the forward on ``(x, valid_token_mask)`` (their allocations are what replay
        reads).  Both must be contiguous, as the eager forward requires for a zero-copy call."""
        if not x.is_contiguous() or (valid_token_mask is not None
                                     and not valid_token_mask.is_contiguous()):
            raise ValueError("graph capture needs a contiguous input and mask")
        dev = x.device
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(3):
                self.module(x, valid_token_mask)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph), torch.inference_mode():
            out = self.module(x, valid_token_mask)
        # the graph replays on this workspace: keep it alive even if the module later grows or
        # drops its own buffers; a megakernel workspace is pinned in the module together with
        # the status word its launches write (never evicted, never freed while replays run)
        self._static_workspace = self.module.last_workspace
        b, s = x.shape[:2]
        self._static_entry = self.module.pin_workspace(b, s, dev.index if dev.index is not None else 0)
        self._graph = graph
        self._key = self._signature(x, valid_token_mask)
        self._static_input, self._static_mask, self._static_output = x, valid_token_mask, out

    @property
    def captured(self) -> bool:
        return self._graph is not None

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None):
        contiguous = x.is_contiguous() and (valid_token_mask is None
                                            or valid_token_mask.is_contiguous())
        if not contiguous:
            return self.module(x, valid_token_mask)
        key = self._signature(x, valid_token_mask)
        if self._graph is None:
            self.module(x, valid_token_mask)  # validates arguments before any capture
            self.capture(x, valid_token_mask)
        elif key != self._key:
            return self.module(x, valid_token_mask)
        self._graph.replay()
        return self._static_output


def make_optimized_transformer(parameter_model: nn.Module, *, verbose_build: bool = False,
                               plan: int = PLAN_AUTO, graphed: bool = False) -> nn.Module:
    """Build and prepare the optimized module for ``parameter_model``.

    ``parameter_model`` supplies the weights and must already be on its ROCm device in fp16
    (the reference's contract, optimized_transformer.py:74-77).  ``verbose_build`` is accepted for
    signature compatibility; the library is prebuilt, so there is nothing to report.
    ``graphed=True`` wraps the module in ``GraphedOptimizedTransformer`` (HIP-graph replay with a
    static output tensor, as the reference's graphed production paths return).
    """
    del verbose_build
    check_supported(parameter_model.config)
    module = OptimizedTransformer(parameter_model, plan=plan)
    module.prepare()
    if graphed:
        return GraphedOptimizedTransformer(module)
    return module
