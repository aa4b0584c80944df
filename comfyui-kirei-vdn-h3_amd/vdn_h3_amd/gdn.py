"""Token-level chunked Gated DeltaNet (chunk 64) on MI355X.

NOT part of hyukudan/ComfyUI-Kirei-VDN-H3: its Video Delta Attention solves the delta rule per
frame (``vdn_h3/branch.py:148-160``, ``vdn_h3_amd.runtime.OptimizedLinearBranch``). This module
is the published Gated DeltaNet recurrence in chunk (WY) form, the workload a token-level
"chunk 64" delta-rule benchmark names, per head with an fp32 state ``S`` (dv x dk)::

    S_t = a_t S_{t-1} (I - b_t k_t k_t^T) + b_t v_t k_t^T,   o_t = S_t q_t,   a_t = exp(g_t)

``chunk_gated_delta_rule`` keeps the argument names of the common Gated DeltaNet operator.
"""

from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib


class _Pipe:
    """The second stream (default priority) and the events of the pipelined call on one device. Every call
    re-records the same events (a wait enqueued earlier keeps the state of the record before it), so calls on
    one device enqueue under ``lock``."""

    def __init__(self, device):
        self.side = torch.cuda.Stream(device=device)
        self.prep_done = [torch.cuda.Event(), torch.cuda.Event()]
        self.scan_done = [torch.cuda.Event(), torch.cuda.Event()]
        self.lock = threading.Lock()


_PIPES: dict = {}
_PIPES_LOCK = threading.Lock()


def _pipe(device: torch.device) -> _Pipe:
    """The pipe of ``device``, made on first use. While one thread captures a graph that holds a pipelined
    call, no other thread may make an eager pipelined call on the same device (its work would join that
    capture through the shared side stream)."""
    device = torch.device(device)
    with _PIPES_LOCK:
        pipe = _PIPES.get(device)
        if pipe is None:
            pipe = _PIPES[device] = _Pipe(device)
    return pipe


def side_stream(device: torch.device) -> torch.cuda.Stream:
    """The second stream of the pipelined call on ``device``."""
    return _pipe(device).side


def gdn_forward_into(q, k, v, beta, g, out, workspace, *, initial_state=None, final_state=None,
                     pipelined: bool = True) -> None:
    """Enqueue one chunk-64 Gated DeltaNet call on the current stream: ``out`` ``[T, H, 128]`` bf16 from ``q``,
    ``k``, ``v`` (bf16 views, 16-byte aligned, strides multiples of 8), fp32 ``beta`` / ``g`` ``[T, H]`` (row
    stride ``H``) and ``workspace`` (``vdnh3_gdn_workspace_bytes`` bytes); the final state into ``final_state``
    when given. A sequence of several segments runs with segment ``i + 1``'s prep on ``side_stream`` beside
    segment ``i``'s scan on the current stream (``pipelined``), each prep after the scan that last read its
    buffer, each scan after its prep; the current stream waits for every side-stream operation before its
    last scan, so the call is ordered on the current stream and can be captured in a graph."""
    tokens, heads, dim = q.shape
    device = q.device
    lib = _lib.lib()
    ws_bytes = workspace.numel() * workspace.element_size()
    segments = lib.vdnh3_gdn_segments(tokens, heads, dim)
    if segments <= 0:
        raise ValueError(f"gdn: no segment plan for tokens={tokens}, heads={heads}, head_dim={dim}")
    cur = torch.cuda.current_stream(device)

    def prep(i, stream):
        rc = lib.vdnh3_gdn_prep(_lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
                                _lib.ptr(v), v.stride(0), v.stride(1), _lib.ptr(beta), beta.stride(0), _lib.ptr(g),
                                g.stride(0), tokens, heads, dim, i, _lib.ptr(workspace), ws_bytes,
                                ctypes.c_void_p(stream.cuda_stream))
        _lib.check(rc, "vdnh3_gdn_prep")

    def scan(i):
        rc = lib.vdnh3_gdn_scan(_lib.ptr(initial_state), _lib.ptr(final_state), _lib.ptr(out), out.stride(0),
                                out.stride(1), tokens, heads, dim, i, _lib.ptr(workspace), ws_bytes,
                                ctypes.c_void_p(cur.cuda_stream))
        _lib.check(rc, "vdnh3_gdn_scan")

    if segments == 1 or not pipelined:
        for i in range(segments):
            prep(i, cur)
            scan(i)
        return
    pipe = _pipe(device)
    side = pipe.side
    with pipe.lock:
        prep(0, cur)
        # the fork follows prep 0: the side stream's first prep starts once segment 0 is prepared, so prep 0
        # runs alone and scan 0, the head of the critical chain, starts as early as it can
        side.wait_stream(cur)
        try:
            for i in range(segments):
                b = i & 1
                if i + 1 < segments:  # segment i + 1 fills buffer b ^ 1, last read by scan i - 1
                    if i >= 1:
                        side.wait_event(pipe.scan_done[b ^ 1])
                    prep(i + 1, side)
                    pipe.prep_done[b ^ 1].record(side)
                if i >= 1:
                    cur.wait_event(pipe.prep_done[b])
                scan(i)
                pipe.scan_done[b].record(cur)
        except BaseException:
            cur.wait_stream(side)  # no side-stream work outlives the call's ordering on the current stream
            raise


def chunk_gated_delta_rule(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
                           g: torch.Tensor, *, initial_state: torch.Tensor | None = None,
                           output_final_state: bool = False, chunk_size: int = 64, pipelined: bool = True):
    """``(o [T, H, D] bf16, final state [H, D, D] fp32 or None)``.

    ``q``, ``k``, ``v``: ``[T, H, D]`` bf16, D <= 128 (strided views are read in place; a head dim below 128
    runs at 128 with zero channels added, which leaves the result exact); ``beta`` and ``g``
    (the log-decay, ``<= 0``): ``[T, H]``, computed in fp32; ``initial_state``: ``[H, D, D]``
    (dv rows, dk columns). Keys are used as given (the recurrence assumes unit-norm keys).
    ``pipelined``: overlap the segments' preps and scans on two streams (``gdn_forward_into``).
    An empty sequence (``tokens == 0``) gives an empty output and the initial state (zeros without one).
    """
    if chunk_size != 64:
        raise ValueError("the HIP kernel is built for chunk_size 64")
    if q.ndim != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k and v must share shape [tokens, heads, dim]")
    tokens, heads, dim = q.shape
    if dim <= 0 or dim > 128:
        raise ValueError(f"head_dim must be 1 to 128 (128 natively), got {dim}")
    if beta.shape != (tokens, heads) or g.shape != (tokens, heads):
        raise ValueError("beta and g must have shape [tokens, heads]")
    _lib.forward_only("chunk_gated_delta_rule", q, k, v, beta, g, initial_state)
    device = _lib.require_device(q, k, v, beta, g, initial_state)
    if initial_state is not None and initial_state.shape != (heads, dim, dim):
        raise ValueError(f"initial_state must have shape [{heads}, {dim}, {dim}]")
    if tokens == 0:  # no token: no output row, and the state is the initial one
        final = None
        if output_final_state:
            final = (initial_state.float().clone() if initial_state is not None else
                     torch.zeros((heads, dim, dim), dtype=torch.float32, device=device))
        return torch.empty((0, heads, dim), dtype=torch.bfloat16, device=device), final
    if dim < 128:
        # zero channels are exact: k's zero entries leave the state's added rows and columns zero (S_t keeps
        # a_t S (I - b k k^T) there and b v k^T adds nothing), so the output's added channels are zero
        pad = lambda t: torch.nn.functional.pad(t.to(torch.bfloat16), (0, 128 - dim))  # noqa: E731
        init = None
        if initial_state is not None:
            init = torch.zeros((heads, 128, 128), dtype=torch.float32, device=device)
            init[:, :dim, :dim] = initial_state
        o, s = chunk_gated_delta_rule(pad(q), pad(k), pad(v), beta, g, initial_state=init,
                                      output_final_state=output_final_state, pipelined=pipelined)
        return o[..., :dim].contiguous(), None if s is None else s[:, :dim, :dim].contiguous()
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
        init = initial_state.float().contiguous()
    final = torch.empty((heads, dim, dim), dtype=torch.float32, device=device) if output_final_state else None
    out = torch.empty((tokens, heads, dim), dtype=torch.bfloat16, device=device)
    ws = torch.empty(_lib.lib().vdnh3_gdn_workspace_bytes(tokens, heads, dim), dtype=torch.uint8, device=device)
    gdn_forward_into(q, k, v, beta, g, out, ws, initial_state=init, final_state=final, pipelined=pipelined)
    return out, final


def gdn_flops(tokens: int, heads: int, dim: int = 128, chunk: int = 64) -> float:
    """Algorithmic work of the chunk form per call: per chunk and head K K^T and Q K^T (2 C^2 D each),
    the two triangular solves (C^2 D each), U = U~ - W S^T and Q S^T (2 C D^2 each), P U (2 C^2 D) and
    the state update (2 C D^2)."""
    chunks = -(-tokens // chunk)
    per = 2 * 2.0 * chunk * chunk * dim + 2 * chunk * chunk * dim + 3 * 2.0 * chunk * dim * dim \
        + 2.0 * chunk * chunk * dim
    return chunks * heads * per


__all__ = ["chunk_gated_delta_rule", "gdn_flops", "gdn_forward_into", "side_stream"]
