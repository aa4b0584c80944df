"""The MiniMax-H3 DiT block around the hybrid attention on MI355X: pointwise passes and MLP.

Mirrors ``vdn_h3/block_kernels.py``: ``BlockPointwiseCache`` (``:25-82``), the fused
``_pre_body`` / ``_post_body`` (``:85-93``), the SwiGLU MLP (``:113-146``),
``make_fast_block_forward`` (``:149-240``) and ``install_block_fusions`` /
``release_block_fusions`` (``:243-260``). Per block forward, on the caller's current stream:

  h   = rms_norm(x, norm1.w) * (1 + scale_msa[seg]) + shift_msa[seg]   one HIP pass
  x   = x + gate_msa[seg] * attn(h)                                      one HIP pass
  h   = rms_norm(x, norm2.w) * (1 + scale_mlp[seg]) + shift_mlp[seg]   one HIP pass
  x   = x + gate_mlp[seg] * fc2(silu(fc1(h)[:, :F]) * fc1(h)[:, F:])    SwiGLU fused into fc2's
                                                                          activation quantisation
                                                                          when fc2 is W8A8

The block falls back to its original forward in the cases the reference does (an explicit
``attention`` argument, fusion disabled, gradients enabled, weights not resident on the
device); there is no CPU path for the fused ops themselves.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Any

import torch

from . import _lib
from . import linear as _linear


class BlockPointwiseCache:
    """Per-token modulation-row index of a segment map ``[(start, stop, row), ...]``.

    ``row`` is an int or a tensor (one value, or one per token of the segment); the segments
    must cover the sequence contiguously (``vdn_h3/block_kernels.py:34-62``). Indices are int32
    device tensors (the fused kernels' operand); scalar-only maps are cached per device.
    """

    def __init__(self, limit: int = 16):
        self.limit = int(limit)
        self._indices: OrderedDict[tuple[Any, ...], torch.Tensor] = OrderedDict()

    @staticmethod
    def _fill_indices(segments, rows: int, device: torch.device) -> torch.Tensor:
        ids = torch.empty(rows, dtype=torch.int32)
        covered = 0
        for raw_start, raw_stop, row in segments:
            start, stop = int(raw_start), int(raw_stop)
            if start != covered or stop < start or stop > rows:
                raise ValueError("MiniMax-H3 modulation segments must cover the sequence contiguously")
            count = stop - start
            if isinstance(row, torch.Tensor):
                values = row.reshape(-1).to(device="cpu", dtype=torch.int32)
                if values.numel() == 1:
                    ids[start:stop] = values[0]
                elif values.numel() == count:
                    ids[start:stop] = values
                else:
                    raise ValueError(
                        f"modulation row tensor for [{start}:{stop}] has {values.numel()} values, expected {count}")
            else:
                ids[start:stop] = int(row)
            covered = stop
        if covered != rows:
            raise ValueError(f"MiniMax-H3 modulation segments cover {covered}/{rows} rows")
        return ids.to(device)

    def indices(self, segments, rows: int, device: torch.device) -> torch.Tensor:
        device = torch.device(device)
        if any(isinstance(row, torch.Tensor) for _, _, row in segments):
            return self._fill_indices(segments, rows, device)
        key = (tuple((int(a), int(b), int(r)) for a, b, r in segments), int(rows), device.type, device.index)
        cached = self._indices.get(key)
        if cached is not None:
            self._indices.move_to_end(key)
            return cached
        ids = self._fill_indices(key[0], rows, device)
        self._indices[key] = ids
        while len(self._indices) > self.limit:
            self._indices.popitem(last=False)
        return ids

    def clear(self):
        self._indices.clear()

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


def _segment_index(indices: torch.Tensor, table_rows: int) -> torch.Tensor:
    if indices.dtype != torch.int32:
        indices = indices.to(torch.int32)
    return indices.contiguous()


def rmsnorm_modulate(hidden: torch.Tensor, weight: torch.Tensor, eps: float, scale: torch.Tensor,
                     shift: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """``_pre_body``: ``rms_norm(hidden, weight, eps) * (1 + scale[idx]) + shift[idx]`` in bf16."""
    if hidden.ndim != 2 or hidden.dtype != torch.bfloat16:
        raise ValueError("rmsnorm_modulate expects bf16 [rows, hidden]")
    rows, width = hidden.shape
    device = _lib.require_device(hidden, weight, scale, shift, indices)
    x = _rows(hidden)
    w = weight.to(torch.bfloat16).contiguous()
    sc, sc_bf16 = _table(scale, width)
    sh, sh_bf16 = _table(shift.to(sc.dtype), width)
    if sh.shape != sc.shape:
        raise ValueError("scale and shift tables must match")
    idx = _segment_index(indices, sc.shape[0])
    if idx.numel() != rows:
        raise ValueError("one modulation index per row is required")
    out = torch.empty_like(x)
    rc = _lib.lib().vdnh3_rmsnorm_modulate(_lib.ptr(x), x.stride(0), _lib.ptr(w), float(eps), _lib.ptr(sc),
                                           _lib.ptr(sh), sc.stride(0), sc_bf16, _lib.ptr(idx), _lib.ptr(out),
                                           out.stride(0), rows, width, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_rmsnorm_modulate")
    return out


def gated_residual(residual: torch.Tensor, gate: torch.Tensor, indices: torch.Tensor, branch_out: torch.Tensor, *,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """``_post_body``: ``residual + gate[idx] * branch_out`` in bf16 (``out`` may be ``residual``)."""
    if residual.ndim != 2 or residual.dtype != torch.bfloat16 or branch_out.shape != residual.shape:
        raise ValueError("gated_residual expects bf16 [rows, hidden] residual and branch output")
    rows, width = residual.shape
    device = _lib.require_device(residual, gate, indices, branch_out, out)
    x, b = _rows(residual), _rows(branch_out.to(torch.bfloat16))
    g, g_bf16 = _table(gate, width)
    idx = _segment_index(indices, g.shape[0])
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != residual.shape or out.dtype != torch.bfloat16:
        raise ValueError("out must match the residual")
    rc = _lib.lib().vdnh3_gated_residual(_lib.ptr(x), x.stride(0), _lib.ptr(g), g.stride(0), g_bf16, _lib.ptr(idx),
                                         _lib.ptr(b), b.stride(0), _lib.ptr(out), out.stride(0), rows, width,
                                         _lib.stream_handle(device))
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


def _mlp_forward(block: Any, state: Any, h: torch.Tensor) -> torch.Tensor:
    """The H3 MLP (``vdn_h3/block_kernels.py:119-146``): ``fc2(swiglu(fc1(h)))``.

    With W8A8 per-token ``HipLinear`` layers the SwiGLU is fused into fc2's activation
    quantisation; other MLPs (or one with an instance ``forward`` hook) run as they are.
    """
    del state
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


def _weight_ready(norm, x: torch.Tensor) -> bool:
    weight = getattr(norm, "weight", None)
    return isinstance(weight, torch.Tensor) and weight.device == x.device


def make_fast_block_forward(block: Any, state: Any, block_index: int):
    """Drop-in ``DiTBlock.forward`` with the fused pointwise passes (``vdn_h3/block_kernels.py:149-240``)."""
    original_forward = block.forward

    def fallback(x, t_emb, mod_segments, rope_freqs, transformer_options, attention):
        return original_forward(x, t_emb, mod_segments, rope_freqs, transformer_options=transformer_options or {},
                                attention=attention)

    def forward(x, t_emb, mod_segments, rope_freqs, transformer_options=None, attention=None):
        if (attention is not None or not getattr(state, "block_fusion", False)
                or not getattr(state, "inference", False) or torch.is_grad_enabled() or not x.is_cuda
                or getattr(state, "weight_mode", "") != "resident"
                or not _weight_ready(block.norm1, x) or not _weight_ready(block.norm2, x)):
            return fallback(x, t_emb, mod_segments, rope_freqs, transformer_options, attention)
        cache = getattr(state, "block_pointwise_cache", None)
        if cache is None:
            cache = BlockPointwiseCache()
            state.block_pointwise_cache = cache
        indices = cache.indices(mod_segments, x.shape[0], x.device)
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = block.adaln_proj(t_emb)
        scope = state.diagnostics.scope
        with scope("block.pre_attn", x.device):
            h = rmsnorm_modulate(x, block.norm1.weight, float(block.norm1.eps), scale_msa, shift_msa, indices)
        attn_out = block.attn(h, rope_freqs=rope_freqs, transformer_options=transformer_options or {})
        with scope("block.post_attn", x.device):
            x = gated_residual(x, gate_msa, indices, attn_out)
        del h, attn_out
        with scope("block.pre_mlp", x.device):
            h = rmsnorm_modulate(x, block.norm2.weight, float(block.norm2.eps), scale_mlp, shift_mlp, indices)
        with scope("block.mlp", x.device):
            mlp_out = _mlp_forward(block, state, h)
        with scope("block.post_mlp", x.device):
            return gated_residual(x, gate_mlp, indices, mlp_out, out=x)

    forward._vdn_h3_fast_block = True
    forward._vdn_h3_block_index = int(block_index)
    forward._vdn_h3_original = original_forward
    return forward


def install_block_fusions(model_patcher: Any, state: Any, blocks) -> int:
    """Patch ``diffusion_model.blocks.{i}.forward`` when ``state.block_fusion`` (``:243-255``)."""
    if not getattr(state, "block_fusion", False):
        return 0
    existing = getattr(model_patcher, "object_patches", {})
    installed = 0
    for index, block in enumerate(blocks):
        path = f"diffusion_model.blocks.{index}.forward"
        if path in existing:
            raise RuntimeError(f"VDN-H3 fast block fusion collides with existing object patch {path}")
        model_patcher.add_object_patch(path, make_fast_block_forward(block, state, index))
        installed += 1
    return installed


def release_block_fusions(state: Any) -> None:
    cache = getattr(state, "block_pointwise_cache", None)
    if cache is not None:
        cache.release()


__all__ = ["BlockPointwiseCache", "gated_residual", "install_block_fusions", "make_fast_block_forward",
           "release_block_fusions", "rmsnorm_modulate", "swiglu", "swiglu_quantize_rows"]
