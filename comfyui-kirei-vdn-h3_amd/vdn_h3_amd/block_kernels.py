"""The MiniMax-H3 DiT block around the hybrid attention on MI355X: pointwise passes and MLP.

Interface of ``vdn_h3/block_kernels.py``: ``BlockPointwiseCache`` (``:25-82``, ``indices`` /
``clear`` / ``release``), ``make_fast_block_forward`` (``:149-240``) and
``install_block_fusions`` / ``release_block_fusions`` (``:243-260``), with the same call
signatures, fallbacks and exception types. Per block forward, on the caller's current stream:

  h   = rms_norm(x, norm1.w) * (1 + scale_msa[seg]) + shift_msa[seg]   one HIP pass
  x   = x + gate_msa[seg] * attn(h)                                      one HIP pass
  h   = rms_norm(x, norm2.w) * (1 + scale_mlp[seg]) + shift_mlp[seg]   one HIP pass
  x   = x + gate_mlp[seg] * fc2(silu(fc1(h)[:, :F]) * fc1(h)[:, F:])    SwiGLU fused into fc2's
                                                                          activation quantisation
                                                                          when fc2 is W8A8

``seg`` is the per-token row of the AdaLN modulation tables. The segment map
``[(start, stop, row), ...]`` becomes an int32 device index without any device-to-host copy:
integer rows are expanded on the host and copied over once (then cached), tensor rows are
copied into the index on the device. The index's value range is kept with it whenever the
host knows it (integer rows, CPU tensor rows) and checked against the table before launch
(``ValueError``, as ``index_select`` raises); indices with an unknown range are guarded inside
the kernels, which read no table memory for them and write NaN rows.

The block falls back to its original forward in the cases the reference does (an explicit
``attention`` argument, fusion disabled, gradients enabled, a CPU input, weights not resident
on the device); there is no CPU path for the fused ops themselves.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Any, NamedTuple

import torch

from . import _lib
from . import linear as _linear


class SegmentIndex(NamedTuple):
    """A per-token int32 device index and its value range (``None`` when only the device knows it)."""

    ids: torch.Tensor
    low: int | None
    high: int | None


def _segment_runs(segments, rows: int) -> list[tuple[int, int, Any]]:
    """``(start, stop, row)`` runs that tile ``[0, rows)`` in order; ``ValueError`` otherwise."""
    runs, edge = [], 0
    for entry in segments:
        start, stop, row = int(entry[0]), int(entry[1]), entry[2]
        if start != edge or not start <= stop <= rows:
            raise ValueError(f"modulation segments must tile the {rows} tokens in order; "
                             f"[{start}, {stop}) does not continue at token {edge}")
        runs.append((start, stop, row))
        edge = stop
    if edge != rows:
        raise ValueError(f"modulation segments end at token {edge} of {rows}")
    return runs


def _row_values(row: Any, count: int) -> torch.Tensor | int:
    """An integer row, or a tensor row as one value or ``count`` values (shape checked)."""
    if not isinstance(row, torch.Tensor):
        return int(row)
    flat = row.reshape(-1)
    if flat.numel() not in (1, count):
        raise ValueError(f"a tensor modulation row must hold 1 or {count} values, it holds {flat.numel()}")
    return flat


def build_segment_index(segments, rows: int, device: torch.device) -> SegmentIndex:
    """The ``SegmentIndex`` of a segment map (no device-to-host synchronisation)."""
    device = torch.device(device)
    runs = [(a, b, _row_values(r, b - a)) for a, b, r in _segment_runs(segments, rows)]
    if all(isinstance(v, int) for _, _, v in runs):
        counts = torch.tensor([b - a for a, b, _ in runs], dtype=torch.int64)
        values = torch.tensor([v for _, _, v in runs], dtype=torch.int32)
        ids = torch.repeat_interleave(values, counts).to(device, non_blocking=False)
        present = [v for a, b, v in runs if b > a]
        return SegmentIndex(ids, min(present, default=0), max(present, default=0))
    ids = torch.empty(rows, dtype=torch.int32, device=device)
    low = high = None
    known = True
    for a, b, v in runs:
        if b == a:
            continue
        if isinstance(v, int):
            ids[a:b].fill_(v)
            lo = hi = v
        else:
            ids[a:b].copy_(v.to(torch.int32).expand(b - a), non_blocking=True)
            if v.device.type != "cpu":
                known = False
                continue
            lo, hi = int(v.min()), int(v.max())
        low = lo if low is None else min(low, lo)
        high = hi if high is None else max(high, hi)
    return SegmentIndex(ids, low if known else None, high if known else None)


class BlockPointwiseCache:
    """Segment indices of the block's modulation map, cached (LRU) for maps of integer rows."""

    def __init__(self, limit: int = 16):
        self.limit = int(limit)
        self._cache: OrderedDict[tuple, SegmentIndex] = OrderedDict()

    def index(self, segments, rows: int, device) -> SegmentIndex:
        device = torch.device(device)
        if any(isinstance(entry[2], torch.Tensor) for entry in segments):
            return build_segment_index(segments, rows, device)
        key = (tuple((int(a), int(b), int(r)) for a, b, r in segments), int(rows), device.type, device.index)
        hit = self._cache.pop(key, None)
        if hit is None:
            hit = build_segment_index(key[0], rows, device)
        self._cache[key] = hit  # most recently used last
        while len(self._cache) > self.limit:
            self._cache.popitem(last=False)
        return hit

    def indices(self, segments, rows: int, device) -> torch.Tensor:
        """The per-token index tensor (int32 on ``device``)."""
        return self.index(segments, rows, device).ids

    def clear(self):
        self._cache.clear()

    release = clear


def _rows(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or (t.stride(0) * t.element_size()) % 16 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _table(mod: torch.Tensor, hidden: int) -> tuple[torch.Tensor, int]:
    """A modulation table ``[n, hidden]`` (fp32 or bf16) and its bf16 flag."""
    t = mod.reshape(-1, mod.shape[-1])
    if t.shape[-1] != hidden:
        raise ValueError(f"modulation width {t.shape[-1]} does not match hidden {hidden}")
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.float()
    return _rows(t), int(t.dtype == torch.bfloat16)


def _index_operand(indices, rows: int, table_rows: int) -> torch.Tensor:
    """The int32 index tensor of ``indices`` (a tensor or a ``SegmentIndex``), range-checked where the
    host knows the range (a CPU tensor, or a ``SegmentIndex`` with bounds)."""
    low = high = None
    if isinstance(indices, SegmentIndex):
        ids, low, high = indices
    else:
        ids = indices
        if ids.device.type == "cpu" and ids.numel():
            low, high = int(ids.min()), int(ids.max())
    if ids.numel() != rows:
        raise ValueError(f"one modulation index per row is required ({rows} rows, {ids.numel()} indices)")
    if low is not None and (low < 0 or high >= table_rows):
        raise ValueError(f"modulation index out of range: [{low}, {high}] for a table of {table_rows} rows")
    return ids.to(torch.int32).contiguous()


def rmsnorm_modulate(hidden: torch.Tensor, weight: torch.Tensor, eps: float, scale: torch.Tensor,
                     shift: torch.Tensor, indices) -> torch.Tensor:
    """``_pre_body``: ``rms_norm(hidden, weight, eps) * (1 + scale[idx]) + shift[idx]`` in bf16."""
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16:
        raise ValueError("rmsnorm_modulate expects bf16 [rows, hidden]")
    rows, width = hidden.shape
    sc, sc_bf16 = _table(scale, width)
    sh, _ = _table(shift.to(sc.dtype), width)
    if sh.shape != sc.shape:
        raise ValueError("scale and shift tables must match")
    idx = _index_operand(indices, rows, sc.shape[0])
    device = _lib.require_device(hidden, weight, sc, sh, idx)
    x = _rows(hidden)
    w = weight.to(torch.bfloat16).contiguous()
    out = torch.empty_like(x)
    rc = _lib.lib().vdnh3_rmsnorm_modulate(_lib.ptr(x), x.stride(0), _lib.ptr(w), float(eps), _lib.ptr(sc),
                                           _lib.ptr(sh), sc.stride(0), sc_bf16, _lib.ptr(idx), sc.shape[0],
                                           _lib.ptr(out), out.stride(0), rows, width, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_rmsnorm_modulate")
    return out


def gated_residual(residual: torch.Tensor, gate: torch.Tensor, indices, branch_out: torch.Tensor, *,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """``_post_body``: ``residual + gate[idx] * branch_out`` in bf16 (``out`` may be ``residual``)."""
    if residual.ndim != 2 or residual.dtype != torch.bfloat16 or branch_out.shape != residual.shape:
        raise ValueError("gated_residual expects bf16 [rows, hidden] residual and branch output")
    rows, width = residual.shape
    g, g_bf16 = _table(gate, width)
    idx = _index_operand(indices, rows, g.shape[0])
    device = _lib.require_device(residual, g, idx, branch_out, out)
    x, b = _rows(residual), _rows(branch_out.to(torch.bfloat16))
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != residual.shape or out.dtype != torch.bfloat16:
        raise ValueError("out must match the residual")
    rc = _lib.lib().vdnh3_gated_residual(_lib.ptr(x), x.stride(0), _lib.ptr(g), g.stride(0), g_bf16, _lib.ptr(idx),
                                         g.shape[0], _lib.ptr(b), b.stride(0), _lib.ptr(out), out.stride(0), rows,
                                         width, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_gated_residual")
    return out


def swiglu(hidden: torch.Tensor) -> torch.Tensor:
    """``_swiglu_body``: ``silu(gate) * up`` with ``gate, up = hidden.chunk(2, -1)``, bf16."""
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16 or hidden.shape[1] % 2:
        raise ValueError("swiglu expects bf16 [rows, 2 * ffn]")
    device = _lib.require_device(hidden)
    h = _rows(hidden)
    rows, ffn = h.shape[0], h.shape[1] // 2
    out = torch.empty((rows, ffn), dtype=torch.bfloat16, device=device)
    rc = _lib.lib().vdnh3_swiglu(_lib.ptr(h), h.stride(0), rows, ffn, _lib.ptr(out), out.stride(0),
                                 _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_swiglu")
    return out


def swiglu_quantize_rows(hidden: torch.Tensor, kind: int):
    """Row-wise int8 / fp8 codes and scales of ``swiglu(hidden)`` (the W8A8 fc2 input)."""
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16 or hidden.shape[1] % 2:
        raise ValueError("swiglu_quantize_rows expects bf16 [rows, 2 * ffn]")
    device = _lib.require_device(hidden)
    h = _rows(hidden)
    rows, ffn = h.shape[0], h.shape[1] // 2
    dtype = torch.int8 if kind == _linear.KIND_I8 else torch.float8_e4m3fn
    q = torch.empty((rows, ffn), dtype=dtype, device=device)
    scale = torch.empty((rows, 1), dtype=torch.float32, device=device)
    rc = _lib.lib().vdnh3_swiglu_quant_rows(kind, _lib.ptr(h), h.stride(0), rows, ffn, _lib.ptr(q), q.stride(0),
                                            _lib.ptr(scale), _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_swiglu_quant_rows")
    return q, scale


def _mlp_forward(block: Any, h: torch.Tensor) -> torch.Tensor:
    """The H3 MLP (``vdn_h3/block_kernels.py:119-146``): ``fc2(swiglu(fc1(h)))``.

    With W8A8 per-token ``HipLinear`` layers the SwiGLU is fused into fc2's activation
    quantisation; other MLPs (or one with an instance ``forward`` hook) run as they are.
    """
    mlp = block.mlp
    fc1, fc2 = getattr(mlp, "fc1", None), getattr(mlp, "fc2", None)
    if fc1 is None or fc2 is None or "forward" in mlp.__dict__:
        return mlp(h)
    hidden = fc1(h)
    if isinstance(fc2, _linear.HipLinear) and (fc2.precision == "int8"
                                               or (fc2.precision == "fp8" and not fc2.per_tensor)):
        kind = _linear.KIND_I8 if fc2.precision == "int8" else _linear.KIND_F8
        q, s = swiglu_quantize_rows(hidden, kind)
        return _linear.gemm_w8a8(q, s, fc2.weight, fc2.weight_scale)
    return fc2(swiglu(hidden))


# The six AdaLN tables block.adaln_proj(t_emb) returns, in order (vdn_h3/block_kernels.py:183).
_MODULATION = ("shift_msa", "scale_msa", "gate_msa", "shift_mlp", "scale_mlp", "gate_mlp")


class _FastBlockForward:
    """The patched ``DiTBlock.forward`` (``vdn_h3/block_kernels.py:149-240``) of one block."""

    def __init__(self, block: Any, state: Any, block_index: int):
        self.block, self.state = block, state
        self._vdn_h3_fast_block = True
        self._vdn_h3_block_index = int(block_index)
        self._vdn_h3_original = block.forward

    def _fused(self, x: torch.Tensor, attention) -> bool:
        """Whether this call takes the fused path (else the original forward runs)."""
        state, block = self.state, self.block
        if attention is not None or torch.is_grad_enabled() or not x.is_cuda:
            return False
        if not (getattr(state, "block_fusion", False) and getattr(state, "inference", False)):
            return False
        if getattr(state, "weight_mode", "") != "resident":
            return False
        return all(isinstance(getattr(n, "weight", None), torch.Tensor) and n.weight.device == x.device
                   for n in (block.norm1, block.norm2))

    def _segments(self, mod_segments, x: torch.Tensor) -> SegmentIndex:
        cache = getattr(self.state, "block_pointwise_cache", None)
        if cache is None:
            cache = self.state.block_pointwise_cache = BlockPointwiseCache()
        return cache.index(mod_segments, x.shape[0], x.device)

    def __call__(self, x, t_emb, mod_segments, rope_freqs, transformer_options=None, attention=None):
        options = transformer_options or {}
        if not self._fused(x, attention):
            return self._vdn_h3_original(x, t_emb, mod_segments, rope_freqs, transformer_options=options,
                                         attention=attention)
        block, scope = self.block, self.state.diagnostics.scope
        seg = self._segments(mod_segments, x)
        mod = dict(zip(_MODULATION, block.adaln_proj(t_emb)))
        # attention half: norm1 + (shift, scale)_msa in, gate_msa on the residual
        with scope("block.pre_attn", x.device):
            h = rmsnorm_modulate(x, block.norm1.weight, float(block.norm1.eps), mod["scale_msa"], mod["shift_msa"],
                                 seg)
        attended = block.attn(h, rope_freqs=rope_freqs, transformer_options=options)
        del h
        with scope("block.post_attn", x.device):
            x = gated_residual(x, mod["gate_msa"], seg, attended)
        del attended
        # MLP half: norm2 + (shift, scale)_mlp in, gate_mlp on the residual (in place: x is this call's)
        with scope("block.pre_mlp", x.device):
            h = rmsnorm_modulate(x, block.norm2.weight, float(block.norm2.eps), mod["scale_mlp"], mod["shift_mlp"],
                                 seg)
        with scope("block.mlp", x.device):
            mlp_out = _mlp_forward(block, h)
        with scope("block.post_mlp", x.device):
            return gated_residual(x, mod["gate_mlp"], seg, mlp_out, out=x)


def make_fast_block_forward(block: Any, state: Any, block_index: int):
    """Drop-in ``DiTBlock.forward`` with the fused pointwise passes (``vdn_h3/block_kernels.py:149-240``)."""
    return _FastBlockForward(block, state, block_index)


def install_block_fusions(model_patcher: Any, state: Any, blocks) -> int:
    """Patch ``diffusion_model.blocks.{i}.forward`` of every block when ``state.block_fusion`` is set
    (``vdn_h3/block_kernels.py:243-255``); ``RuntimeError`` before any patch if one path is taken."""
    if not getattr(state, "block_fusion", False):
        return 0
    blocks = list(blocks)
    paths = [f"diffusion_model.blocks.{i}.forward" for i in range(len(blocks))]
    taken = sorted(set(paths) & set(getattr(model_patcher, "object_patches", {})))
    if taken:
        raise RuntimeError(f"VDN-H3 fast block fusion: object patch {taken[0]} already exists "
                           f"({len(taken)} block forward(s) are patched by someone else)")
    for index, (path, block) in enumerate(zip(paths, blocks)):
        model_patcher.add_object_patch(path, make_fast_block_forward(block, state, index))
    return len(paths)


def release_block_fusions(state: Any) -> None:
    """Drop the cached segment indices of ``state``."""
    cache = getattr(state, "block_pointwise_cache", None)
    if cache is not None:
        cache.release()


__all__ = ["BlockPointwiseCache", "SegmentIndex", "build_segment_index", "gated_residual", "install_block_fusions",
           "make_fast_block_forward", "release_block_fusions", "rmsnorm_modulate", "swiglu", "swiglu_quantize_rows"]
