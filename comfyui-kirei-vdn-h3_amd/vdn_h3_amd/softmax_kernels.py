"""The per-head softmax gate of the hybrid block (``vdn_h3/softmax_kernels.py``).

``apply_softmax_gate(softmax_out, gate, state, *, inference)`` returns
``bf16(softmax_out * gate)`` flattened to ``[S, H*D]`` (``:8-9``, ``:12-37``) with one HIP
pass (``vdnh3_head_gate``). The block itself fuses the gate into the window attention
epilogue and does not call this; it is kept for callers of the reference op.
"""

from __future__ import annotations

import torch

from . import _lib


def apply_softmax_gate(softmax_out: torch.Tensor, gate: torch.Tensor, state=None, *, inference: bool = True):
    """``(softmax_out * gate).reshape(S, H*D)``; ``gate`` is ``[S, H]`` or ``[S, H, 1]``."""
    del state, inference
    if softmax_out.ndim != 3:
        raise ValueError("softmax_out must be [sequence, heads, dim]")
    seq, heads, dim = softmax_out.shape
    if gate.numel() != seq * heads:
        raise ValueError(f"gate must hold one value per (row, head): {seq}x{heads}, got {tuple(gate.shape)}")
    _lib.forward_only("apply_softmax_gate", softmax_out, gate)
    device = _lib.require_device(softmax_out, gate)
    o = softmax_out
    if o.dtype != torch.bfloat16:
        raise TypeError("apply_softmax_gate computes in bf16")
    if o.stride(2) != 1 or o.stride(0) % 8 or o.stride(1) % 8 or o.data_ptr() % 16:
        o = o.contiguous()
    g = gate.reshape(seq, heads).to(o.dtype)
    if g.stride(1) != 1:
        g = g.contiguous()
    out = torch.empty((seq, heads * dim), dtype=o.dtype, device=device)
    rc = _lib.lib().vdnh3_head_gate(_lib.ptr(o), o.stride(0), o.stride(1), _lib.ptr(g), g.stride(0), _lib.ptr(out),
                                    out.stride(0), seq, heads, dim, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_head_gate")
    return out


__all__ = ["apply_softmax_gate"]
