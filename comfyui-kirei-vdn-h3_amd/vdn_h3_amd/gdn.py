"""Token-level chunked Gated DeltaNet (chunk 64) on MI355X.

NOT part of hyukudan/ComfyUI-Kirei-VDN-H3: its Video Delta Attention solves the delta rule per
frame (``vdn_h3/branch.py:148-160``, ``vdn_h3_amd.runtime.OptimizedLinearBranch``). This module
is the published Gated DeltaNet recurrence in chunk (WY) form, the workload a token-level
"chunk 64" delta-rule benchmark names, per head with an fp32 state ``S`` (dv x dk)::

    S_t = a_t S_{t-1} (I - b_t k_t k_t^T) + b_t v_t k_t^T,   o_t = S_t q_t,   a_t = exp(g_t)

``chunk_gated_delta_rule`` keeps the argument names of the common Gated DeltaNet operator.
"""

from __future__ import annotations

import torch

from . import _lib


def chunk_gated_delta_rule(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                           g: torch.Tensor, *, initial_state: torch.Tensor | None = None,
                           output_final_state: bool = False, chunk_size: int = 64):
    """``(o [T, H, D] bf16, final state [H, D, D] fp32 or None)``.

    ``q``, ``k``, ``v``: ``[T, H, 128]`` bf16 (strided views are read in place); ``beta`` and ``g``
    (the log-decay, ``<= 0``): ``[T, H]``, computed in fp32; ``initial_state``: ``[H, D, D]``
    (dv rows, dk columns). Keys are used as given (the recurrence assumes unit-norm keys).
    """
    if chunk_size != 64:
        raise ValueError("the HIP kernel is built for chunk_size 64")
    if q.ndim != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k and v must share shape [tokens, heads, dim]")
    tokens, heads, dim = q.shape
    if dim != 128:
        raise ValueError(f"head_dim must be 128, got {dim}")
    if beta.shape != (tokens, heads) or g.shape != (tokens, heads):
        raise ValueError("beta and g must have shape [tokens, heads]")
    device = _lib.require_device(q, k, v, beta, g, initial_state)
    ops = []
    for t in (q, k, v):
        t = t if t.dtype == torch.bfloat16 else t.to(torch.bfloat16)
        if t.stride(-1) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or t.data_ptr() % 16:
            t = t.contiguous()
        ops.append(t)
    q, k, v = ops
    beta = beta.float().contiguous()
    g = g.float().contiguous()
    init = None
    if initial_state is not None:
        if initial_state.shape != (heads, dim, dim):
            raise ValueError(f"initial_state must have shape [{heads}, {dim}, {dim}]")
        init = initial_state.float().contiguous()
    final = torch.empty((heads, dim, dim), dtype=torch.float32, device=device) if output_final_state else None
    out = torch.empty((tokens, heads, dim), dtype=torch.bfloat16, device=device)
    lib = _lib.lib()
    ws_bytes = lib.vdnh3_gdn_workspace_bytes(tokens, heads, dim)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    rc = lib.vdnh3_gdn_chunk_fwd(_lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
                                 _lib.ptr(v), v.stride(0), v.stride(1), _lib.ptr(beta), beta.stride(0), _lib.ptr(g),
                                 g.stride(0), _lib.ptr(init), _lib.ptr(final), _lib.ptr(out), out.stride(0),
                                 out.stride(1), tokens, heads, dim, _lib.ptr(ws), ws_bytes,
                                 _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_gdn_chunk_fwd")
    return out, final


def gdn_flops(tokens: int, heads: int, dim: int = 128, chunk: int = 64) -> float:
    """Algorithmic work of the chunk form per call: per chunk and head K K^T and Q K^T (2 C^2 D each),
    the two triangular solves (C^2 D each), U = U~ - W S^T and Q S^T (2 C D^2 each), P U (2 C^2 D) and
    the state update (2 C D^2)."""
    chunks = -(-tokens // chunk)
    per = 2 * 2.0 * chunk * chunk * dim + 2 * chunk * chunk * dim + 3 * 2.0 * chunk * dim * dim \
        + 2.0 * chunk * chunk * dim
    return chunks * heads * per


__all__ = ["chunk_gated_delta_rule", "gdn_flops"]
