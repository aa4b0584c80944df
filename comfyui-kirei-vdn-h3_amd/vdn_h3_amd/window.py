"""Exact VDN-H3 local-window softmax attention on MI355X (one HIP backend).

Mirrors the public surface of ``vdn_h3/window.py``:

* geometry: ``window_bounds`` (``:141-153``), ``full_coverage`` (``:156-159``),
  ``window_group_count`` (``:273-274``), ``ANCHOR_FRAME_MODES`` (``:18``);
* the op: ``window_softmax_hip(query, key, value, video_start, video_end, num_frames,
  tokens_per_frame, bounds, scale, anchor_frames="none", cache=None)`` with the argument
  meaning and ``ValueError`` behaviour of ``window_softmax_grouped`` / ``_flex`` /
  ``_flash2`` / ``_decomposed`` (``:277-313``, ``:694-723``, ``:839-861``); those four names
  are kept as aliases of the one exact HIP kernel;
* ``window_softmax_normed``: the same op taking the raw q / k with the block's q_norm / k_norm
  (and RoPE) fused in (``vdn_h3/hybrid.py:271-302``);
* ``WindowAttentionCache`` (``:77-138``) holds the per-model tile plans;
* ``resolve_attention_backend`` (``:581-673``) resolves every request to ``"hip"``.

There is no CPU path: a CPU tensor raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
from collections import OrderedDict
from contextlib import nullcontext
from dataclasses import dataclass
from typing import Any

import torch

from . import _lib

ANCHOR_FRAME_MODES = ("none", "columns", "rows", "both")
ATTENTION_BACKENDS = ("auto", "hip", "grouped", "flex", "flash2", "decomposed", "reference", "compat")


def window_bounds(num_frames: int, radius: int, chunk: int = 0) -> list[tuple[int, int]]:
    """Per-frame window ``(lo, hi)``: frame +- radius, or the chunk +- radius chunks."""
    if isinstance(num_frames, bool) or not isinstance(num_frames, int) or num_frames < 0:
        raise ValueError("num_frames must be a non-negative integer")
    if isinstance(radius, bool) or not isinstance(radius, int) or radius < 0:
        raise ValueError("radius must be a non-negative integer")
    if isinstance(chunk, bool) or not isinstance(chunk, int):
        raise ValueError("chunk must be an integer")
    if chunk <= 0:
        return [(f - radius, f + radius) for f in range(num_frames)]
    out = []
    for f in range(num_frames):
        c = f // chunk
        out.append(((c - radius) * chunk, (c + radius + 1) * chunk - 1))
    return out


def full_coverage(bounds, num_frames: int) -> bool:
    """True when every frame's window spans all frames (the block then runs dense attention)."""
    if len(bounds) != num_frames:
        raise ValueError("bounds must contain exactly one entry per frame")
    return all(lo <= 0 and hi >= num_frames - 1 for lo, hi in bounds)


def window_group_count(num_frames, bounds, anchor_frames="none") -> int:
    """Number of runs of consecutive frames that share one key set."""
    anchor_rows = anchor_frames in ("rows", "both")
    anchor_cols = anchor_frames in ("columns", "both")
    last = num_frames - 1
    count, previous = 0, object()
    for f in range(num_frames):
        if anchor_rows and f in (0, last):
            sig = None
        else:
            frames = set(range(max(bounds[f][0], 0), min(bounds[f][1], last) + 1))
            if anchor_cols:
                frames |= {0, last}
            sig = tuple(sorted(frames))
        if f == 0 or sig != previous:
            count += 1
        previous = sig
    return count


@dataclass
class WindowPlan:
    """Device copy of a tile plan (see ``vdnh3_window_plan_build``)."""

    items: torch.Tensor     # int32 [n_items, 4]
    tiles: torch.Tensor     # int32 [n_tiles, 2]
    n_items: int
    n_tiles: int
    pairs_per_head: int     # allowed (query, key) pairs per head


def build_plan_host(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames):
    """Run the C++ planner on the host; returns ``(items[n,4], tiles[m,2], pairs)`` CPU int32 tensors."""
    if anchor_frames not in ANCHOR_FRAME_MODES:
        raise ValueError(f"anchor_frames={anchor_frames!r}; expected one of {ANCHOR_FRAME_MODES}")
    if len(bounds) != num_frames:
        raise ValueError("bounds must contain exactly one entry per frame")
    for frame, pair in enumerate(bounds):
        if len(pair) != 2:
            raise ValueError(f"bounds[{frame}] must be a (lo, hi) pair")
    lib = _lib.lib()
    flat = (ctypes.c_int32 * max(1, 2 * num_frames))(*[int(x) for pair in bounds for x in pair])
    bm, bn = lib.vdnh3_window_block_m(), lib.vdnh3_window_block_n()
    mode = _lib.ANCHOR_MODE_CODES[anchor_frames]
    n_items, n_tiles, pairs = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
    _lib.check(lib.vdnh3_window_plan_size(int(seq), int(video_start), int(video_end), int(num_frames),
                                          int(tokens_per_frame), flat, mode, bm, bn, ctypes.byref(n_items),
                                          ctypes.byref(n_tiles), ctypes.byref(pairs)), "window plan")
    items = torch.empty((n_items.value, 4), dtype=torch.int32)
    tiles = torch.empty((n_tiles.value, 2), dtype=torch.int32)
    _lib.check(lib.vdnh3_window_plan_build(
        int(seq), int(video_start), int(video_end), int(num_frames), int(tokens_per_frame), flat, mode, bm, bn,
        ctypes.cast(items.data_ptr(), ctypes.POINTER(ctypes.c_int32)), n_items.value,
        ctypes.cast(tiles.data_ptr(), ctypes.POINTER(ctypes.c_int32)), n_tiles.value), "window plan")
    return items, tiles, int(pairs.value)


class WindowAttentionCache:
    """Tile plans of one patched model, keyed by geometry and device (LRU, bounded)."""

    def __init__(self, limit: int = 16):
        if limit <= 0:
            raise ValueError("cache limit must be positive")
        self.limit = int(limit)
        self._plans: OrderedDict[tuple[Any, ...], WindowPlan] = OrderedDict()
        self.last_dispatch_reason: str | None = None

    def plan(self, seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames, device):
        key = (int(seq), int(video_start), int(video_end), int(num_frames), int(tokens_per_frame),
               tuple((int(a), int(b)) for a, b in bounds), str(anchor_frames), device.type, device.index)
        cached = self._plans.get(key)
        if cached is not None:
            self._plans.move_to_end(key)
            return cached
        plan = make_plan(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames, device)
        self._plans[key] = plan
        while len(self._plans) > self.limit:
            self._plans.popitem(last=False)
        return plan

    def clear(self):
        self._plans.clear()
        self.last_dispatch_reason = None

    release = clear

    def __len__(self):
        return len(self._plans)


def make_plan(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames, device):
    items, tiles, pairs = build_plan_host(seq, video_start, video_end, num_frames, tokens_per_frame, bounds,
                                          anchor_frames)
    return WindowPlan(items.to(device), tiles.to(device), items.shape[0], tiles.shape[0], pairs)


def dense_plan(seq, device):
    """Plan in which every row attends to every key (the full-cover dense path)."""
    return make_plan(seq, 0, seq, 1, seq, [(0, 0)], "none", device)


def _kernel_operand(t: torch.Tensor) -> torch.Tensor:
    """A view the kernel can read in place (16-byte aligned rows/heads), else a contiguous copy."""
    ok = (t.stride(2) == 1 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0 and t.data_ptr() % 16 == 0)
    return t if ok else t.contiguous()


def rope_table(rope_freqs: torch.Tensor, seq: int, head_dim: int, device) -> tuple[torch.Tensor, int, int]:
    """``(table, row_stride, rot_dim)`` of ``rope_freqs`` for the kernels' split-half RoPE.

    ``rope_freqs`` holds one 2x2 matrix per (row, pair): shape ``[..., rot_dim/2, 2, 2]`` whose
    leading dims hold one entry per row (``seq`` in total, e.g. ``[1, seq, 1, ...]``) or one entry
    shared by every row; ``rot_dim = 2 * rope_freqs.shape[-3]`` (``vdn_h3/hybrid.py:283``).
    """
    if rope_freqs.ndim < 3 or tuple(rope_freqs.shape[-2:]) != (2, 2):
        raise ValueError(f"rope_freqs must end in [rot_dim/2, 2, 2], got {tuple(rope_freqs.shape)}")
    half = int(rope_freqs.shape[-3])
    rot = 2 * half
    if rot % 16 or rot > head_dim:
        raise ValueError(f"rope rot_dim {rot} must be a multiple of 16 and at most head_dim {head_dim}")
    rows = rope_freqs.numel() // (4 * half)
    if rows not in (1, seq):
        raise ValueError(f"rope_freqs holds {rows} row entries; expected 1 or {seq}")
    table = rope_freqs.reshape(rows, half, 2, 2).to(device=device, dtype=torch.float32).contiguous()
    return table, (0 if rows == 1 else 4 * half), rot


def _attention_operands(shape, device, plan, cache, geometry, gate, out):
    """``(plan, gate, gate_row, out)`` for one call: the tile plan (cached or built), the gate as a
    bf16 ``[S, H]`` view with unit head stride, and the output buffer (new or checked)."""
    seq, heads, dim = shape
    if plan is None:
        plan = (cache.plan(*geometry, device) if cache is not None else make_plan(*geometry, device))
    if out is None:
        out = torch.empty((seq, heads, dim), dtype=torch.bfloat16, device=device)
    elif out.shape != (seq, heads, dim) or out.dtype != torch.bfloat16 or out.stride(2) != 1:
        raise ValueError("out must be a bf16 [S, H, D] tensor with a contiguous last dim")
    g_row = 0
    if gate is not None:
        gate = gate.reshape(seq, heads)
        if gate.dtype != torch.bfloat16:
            gate = gate.to(torch.bfloat16)
        if gate.stride(1) != 1:
            gate = gate.contiguous()
        g_row = gate.stride(0)
    return plan, gate, g_row, out


def _check_qkv(query, key, value, name):
    if query.ndim != 3 or query.shape != key.shape or query.shape != value.shape:
        raise ValueError("query, key and value must share shape [sequence, heads, dim]")
    if query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16:
        raise TypeError(f"{name} computes in bf16; got {query.dtype}/{key.dtype}/{value.dtype}")


KERNEL_HEAD_DIMS = (64, 128)


def padded_head_dim(dim: int) -> int:
    """The kernel head dim a ``dim``-channel head runs at: ``dim`` itself for 64 and 128, else the next of the
    two (zero channels added); above 128 there is none."""
    if dim <= 0 or dim > 128:
        raise ValueError(f"window attention supports head dims 1 to 128 (64 and 128 natively), got {dim}")
    return 64 if dim <= 64 else 128


def zero_pad_channels(t: torch.Tensor, width: int) -> torch.Tensor:
    """``[S, H, D]`` -> ``[S, H, width]`` bf16, the added channels zero."""
    out = torch.zeros((t.shape[0], t.shape[1], width), dtype=torch.bfloat16, device=t.device)
    out[..., :t.shape[2]] = t
    return out


def window_softmax_hip(query, key, value, video_start, video_end, num_frames, tokens_per_frame, bounds, scale,
                       anchor_frames="none", cache: WindowAttentionCache | None = None, *, gate=None,
                       out: torch.Tensor | None = None, plan: WindowPlan | None = None, diagnostics=None):
    """Exact window softmax attention on the GPU; returns a new ``[S, H, D]`` bf16 tensor.

    ``gate`` (optional, ``[S, H]`` or ``[S, H, 1]``) fuses the per-head softmax gate into the
    epilogue: the result is then ``bf16(bf16(O) * gate)``. Inputs are not modified.
    ``diagnostics`` (a ``DiagnosticsRecorder``) times the V^T pre-pass and the attention kernel
    as the stages ``attention.softmax.vt_prepass`` / ``attention.softmax.kernel``.
    Head dims other than 64 and 128 (up to 128; the reference's op is shape-generic,
    ``vdn_h3/window.py:277-313``) run at the next kernel head dim with zero channels added to q, k and v:
    a zero channel adds nothing to a score and yields a zero output channel, and ``scale`` is the caller's.
    """
    _check_qkv(query, key, value, "window_softmax_hip")
    _lib.forward_only("window_softmax_hip", query, key, value, gate)
    device = _lib.require_device(query, key, value, gate, out)
    seq, heads, dim = query.shape
    if dim not in KERNEL_HEAD_DIMS:
        width = padded_head_dim(dim)
        if out is not None and (out.shape != (seq, heads, dim) or out.dtype != torch.bfloat16):
            raise ValueError("out must be a bf16 [S, H, D] tensor")
        res = window_softmax_hip(zero_pad_channels(query, width), zero_pad_channels(key, width),
                                 zero_pad_channels(value, width), video_start, video_end, num_frames,
                                 tokens_per_frame, bounds, scale, anchor_frames, cache, gate=gate, plan=plan,
                                 diagnostics=diagnostics)
        if out is None:
            return res[..., :dim].contiguous()
        out.copy_(res[..., :dim])
        return out
    geometry = (seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames)
    plan, gate, g_row, out = _attention_operands(query.shape, device, plan, cache, geometry, gate, out)
    q, k, v = _kernel_operand(query), _kernel_operand(key), _kernel_operand(value)
    lib = _lib.lib()
    ws_bytes = lib.vdnh3_window_workspace_bytes(seq, heads, dim)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    sh = _lib.stream_handle(device)
    if diagnostics is None:
        rc = lib.vdnh3_window_attn_fwd(
            _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
            _lib.ptr(v), v.stride(0), v.stride(1), _lib.ptr(out), out.stride(0), out.stride(1),
            _lib.ptr(gate), g_row, seq, heads, dim, float(scale),
            _lib.ptr(plan.items), plan.n_items, _lib.ptr(plan.tiles), _lib.ptr(workspace), ws_bytes, sh)
        _lib.check(rc, "window_softmax_hip")
        return out
    with diagnostics.scope("attention.softmax.vt_prepass", device):
        rc = lib.vdnh3_window_vt_prepass(_lib.ptr(v), v.stride(0), v.stride(1), seq, heads, dim,
                                         _lib.ptr(workspace), ws_bytes, sh)
    _lib.check(rc, "window_softmax_hip")
    with diagnostics.scope("attention.softmax.kernel", device):
        rc = lib.vdnh3_window_attn_prepared(
            _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
            _lib.ptr(out), out.stride(0), out.stride(1), _lib.ptr(gate), g_row, seq, heads, dim, float(scale),
            _lib.ptr(plan.items), plan.n_items, _lib.ptr(plan.tiles), _lib.ptr(workspace), ws_bytes, sh)
    _lib.check(rc, "window_softmax_hip")
    return out


def window_softmax_normed(q_raw, k_raw, value, q_weight, k_weight, q_eps, k_eps, video_start, video_end,
                          num_frames, tokens_per_frame, bounds, scale, anchor_frames="none",
                          cache: WindowAttentionCache | None = None, *, rope_freqs=None, gate=None,
                          out: torch.Tensor | None = None, plan: WindowPlan | None = None, diagnostics=None):
    """``window_softmax_hip(q_norm(q_raw), k_norm(k_raw), value)`` with the block's q/k RMSNorm (and,
    with ``rope_freqs``, the split-half RoPE) fused into the attention (``vdn_h3/hybrid.py:271-302``).

    The keys are normalised (and rotated) once, by the pre-pass that also writes the V^T copy.
    Without RoPE each query row is normalised as the attention kernel loads it; with RoPE the
    pre-pass normalises and rotates the queries too (a rotation inside the attention kernel would
    re-read the table for every head and query block). Either way the result has the same bits as
    the separate q/k pass followed by ``window_softmax_hip``. ``q_eps`` / ``k_eps`` are the two
    norms' epsilons (with RoPE the reference takes ``q_eps`` for both: pass it as ``k_eps``).
    ``diagnostics`` times the stages ``attention.softmax.qkv_prepass`` / ``attention.softmax.kernel``.
    """
    _check_qkv(q_raw, k_raw, value, "window_softmax_normed")
    _lib.forward_only("window_softmax_normed", q_raw, k_raw, value, q_weight, k_weight, rope_freqs, gate)
    device = _lib.require_device(q_raw, k_raw, value, q_weight, k_weight, gate, out)
    seq, heads, dim = q_raw.shape
    wq = q_weight.to(torch.bfloat16).contiguous()
    wk = k_weight.to(torch.bfloat16).contiguous()
    if wq.numel() != dim or wk.numel() != dim:
        raise ValueError(f"q/k norm weights must have {dim} entries")
    table, f_row, rot = (None, 0, 0) if rope_freqs is None else rope_table(rope_freqs, seq, dim, device)
    geometry = (seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames)
    plan, gate, g_row, out = _attention_operands(q_raw.shape, device, plan, cache, geometry, gate, out)
    q, k, v = _kernel_operand(q_raw), _kernel_operand(k_raw), _kernel_operand(value)
    lib = _lib.lib()
    rotate = table is not None
    ws_bytes = lib.vdnh3_window_norm_workspace_bytes(seq, heads, dim, int(rotate))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    sh = _lib.stream_handle(device)
    with _maybe_scope(diagnostics, "attention.softmax.qkv_prepass", device):
        rc = lib.vdnh3_window_qkv_prepass(
            _lib.ptr(q) if rotate else None, q.stride(0), q.stride(1), _lib.ptr(wq), float(q_eps),
            _lib.ptr(k), k.stride(0), k.stride(1), _lib.ptr(wk), float(k_eps), _lib.ptr(v), v.stride(0), v.stride(1),
            _lib.ptr(table), f_row, rot, seq, heads, dim, _lib.ptr(workspace), ws_bytes, sh)
    _lib.check(rc, "window_softmax_normed")
    with _maybe_scope(diagnostics, "attention.softmax.kernel", device):
        if rotate:
            # regions 2 (queries) and 1 (keys) of the workspace, [heads][s_pad][dim]
            region = lib.vdnh3_window_workspace_bytes(seq, heads, dim)
            head_stride = region // (2 * heads)
            base = workspace.data_ptr()
            rc = lib.vdnh3_window_attn_prepared(
                ctypes.c_void_p(base + 2 * region), dim, head_stride, ctypes.c_void_p(base + region), dim,
                head_stride, _lib.ptr(out), out.stride(0), out.stride(1), _lib.ptr(gate), g_row, seq, heads, dim,
                float(scale), _lib.ptr(plan.items), plan.n_items, _lib.ptr(plan.tiles), _lib.ptr(workspace),
                ws_bytes, sh)
        else:
            rc = lib.vdnh3_window_attn_qnorm(
                _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(wq), float(q_eps),
                _lib.ptr(out), out.stride(0), out.stride(1), _lib.ptr(gate), g_row, seq, heads, dim, float(scale),
                _lib.ptr(plan.items), plan.n_items, _lib.ptr(plan.tiles), _lib.ptr(workspace), ws_bytes, sh)
    _lib.check(rc, "window_softmax_normed")
    return out


def _maybe_scope(diagnostics, name, device):
    return nullcontext() if diagnostics is None else diagnostics.scope(name, device)


# The reference's exact backends all resolve to the one HIP kernel on MI355X.
window_softmax_grouped = window_softmax_hip
window_softmax_flex = window_softmax_hip
window_softmax_flash2 = window_softmax_hip
window_softmax_decomposed = window_softmax_hip


def resolve_attention_backend(requested: str, query=None, num_frames=None, bounds=None, anchor_frames=None,
                              cache: WindowAttentionCache | None = None, **_unused) -> str:
    """Every exact backend name maps to ``"hip"`` (the only exact kernel on gfx950)."""
    if requested not in ATTENTION_BACKENDS:
        raise ValueError(f"unsupported attention backend {requested!r}")
    if cache is not None:
        cache.last_dispatch_reason = "hip" if requested in ("auto", "hip") else f"explicit: {requested} -> hip"
    return "hip"


def attention_flops(pairs_per_head: int, heads: int, head_dim: int) -> float:
    """Algorithmic FLOP of one call: ``4 * D * H * sum_i |A(i)|`` (QK^T and PV, no exp)."""
    return 4.0 * head_dim * heads * pairs_per_head


__all__ = ["ANCHOR_FRAME_MODES", "ATTENTION_BACKENDS", "WindowAttentionCache", "WindowPlan", "attention_flops",
           "build_plan_host", "dense_plan", "full_coverage", "make_plan", "resolve_attention_backend",
           "window_bounds", "window_group_count", "window_softmax_decomposed", "window_softmax_flash2",
           "window_softmax_flex", "window_softmax_grouped", "window_softmax_hip"]
