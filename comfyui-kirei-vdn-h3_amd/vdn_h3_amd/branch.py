"""Video Delta Attention (the VDN linear branch) on MI355X: functional ops.

Mirrors the inference pieces of ``vdn_h3/branch.py`` with HIP kernels behind each:

* ``cholesky_runtime_scope`` / deferred SPD validation (``:24-71``): factor statuses are
  collected on the device and checked once when the scope exits, raising
  ``torch.linalg.LinAlgError`` with the reference's message;
* ``frame_statistics_raw`` - ``frame_statistics`` (``:197-282``) with the feature map of
  ``vdn_h3/kernels.py:47-51`` fused into the loads;
* ``conv_features`` - the short convolutions (``:443-480``, ``vdn_h3/runtime.py:319-341``) as
  one kernel;
* ``VdnDelta`` / ``SanaDelta`` ``.factor_apply`` (``:144-180``);
* ``run_scans_inference`` (``:315-333``);
* ``alpha_gate`` (``:483-491``), ``frame_mean``;
* ``readout_epilogue`` - ``gather_linear_state`` + readout matmul + ``linear_epilogue``
  (``:372-396``, ``:494-530``, ``vdn_h3/runtime.py:406-419``) as one kernel.

Every op takes and returns device tensors; there is no CPU path.
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from typing import Any

import ctypes

import torch

from . import _lib

TEXT_STATE_SCALE = 0.5
_CHOLESKY_CHECKS: ContextVar[Any] = ContextVar("vdn_h3_amd_cholesky_checks", default=None)


class _CholeskyChecks:
    """Factor statuses of one forward, validated with a single host read."""

    def __init__(self):
        self.statuses: list[torch.Tensor] = []
        self.factor_calls = 0

    def validate(self):
        if not self.statuses:
            return
        info = torch.cat([s.reshape(-1) for s in self.statuses])
        bad = torch.nonzero(info != 0)
        if bad.numel():
            failed = int(bad[0, 0])
            for index, status in enumerate(self.statuses):
                if failed < status.numel():
                    minor = int(status.reshape(-1)[failed])
                    raise torch.linalg.LinAlgError(
                        f"VDN-H3 Cholesky factor {index}, batch {failed}: "
                        f"leading minor of order {minor} is not positive-definite")
                failed -= status.numel()


@contextmanager
def cholesky_runtime_scope(diagnostics=None):
    """Collect factor statuses inside the scope; validate them once on exit."""
    del diagnostics
    checks = _CholeskyChecks()
    token = _CHOLESKY_CHECKS.set(checks)
    try:
        yield checks
        checks.validate()
    finally:
        checks.statuses.clear()
        _CHOLESKY_CHECKS.reset(token)


def _record_status(info: torch.Tensor):
    checks = _CHOLESKY_CHECKS.get()
    if checks is None:
        scope = _CholeskyChecks()
        scope.statuses.append(info)
        scope.validate()
        return
    checks.statuses.append(info)
    checks.factor_calls += 1


def _dim(head_dim: int):
    if head_dim not in (64, 128):
        raise ValueError(f"the HIP delta-rule kernels support head_dim 64 or 128, got {head_dim}")


def _rows(t: torch.Tensor) -> torch.Tensor:
    """A ``[rows, heads, D]`` view whose D is contiguous and whose strides are 16-byte multiples."""
    if t.stride(-1) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def frame_statistics_raw(k_raw: torch.Tensor, v_raw: torch.Tensor, beta: torch.Tensor, num_frames: int,
                         tokens_per_frame: int, *, k_features: bool = False, v_features: bool = False,
                         a_fp32: bool = True, out=None):
    """``A, B`` ``[F, H, D, D]`` fp32 from ``k``/``v`` rows ``[F*T, H, D]`` and ``beta`` ``[F*T, H]``.

    ``k``/``v`` are raw projections (the feature map is applied on load) unless
    ``k_features``/``v_features`` say they already hold the features (short-convolution output).
    ``a_fp32=False`` forms ``A`` as the reference does for that flag (``vdn_h3/branch.py:238-240``):
    the bf16 product of ``bf16(k~ * beta)`` and ``k~``, rounded to bf16, then symmetrised.
    ``out=(A, B)``: contiguous fp32 ``[F, H, D, D]`` tensors (e.g. frame slices of larger ones) to write into.
    """
    if k_raw.shape != v_raw.shape or k_raw.ndim != 3:
        raise ValueError("key and value must share shape [rows, heads, dim]")
    rows, heads, dim = k_raw.shape
    if rows != num_frames * tokens_per_frame:
        raise ValueError("rows must equal num_frames * tokens_per_frame")
    if beta.shape != (rows, heads):
        raise ValueError("beta must have shape [rows, heads]")
    _dim(dim)
    device = _lib.require_device(k_raw, v_raw, beta)
    k_raw, v_raw = _rows(k_raw), _rows(v_raw)
    beta = beta.to(torch.bfloat16)
    if beta.stride(1) != 1:
        beta = beta.contiguous()
    if out is None:
        a = torch.empty((num_frames, heads, dim, dim), dtype=torch.float32, device=device)
        b = torch.empty_like(a)
    else:
        a, b = out
        for t in (a, b):
            if t.shape != (num_frames, heads, dim, dim) or t.dtype != torch.float32 or not t.is_contiguous():
                raise ValueError(f"out must hold two contiguous fp32 [{num_frames}, {heads}, {dim}, {dim}] tensors")
    flags = int(bool(k_features)) | (int(bool(v_features)) << 1) | (int(not a_fp32) << 2)
    rc = _lib.lib().vdnh3_frame_stats(_lib.ptr(k_raw), k_raw.stride(0), k_raw.stride(1), _lib.ptr(v_raw),
                                      v_raw.stride(0), v_raw.stride(1), flags, _lib.ptr(beta), beta.stride(0),
                                      num_frames, tokens_per_frame, heads, dim, _lib.ptr(a), _lib.ptr(b),
                                      _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_frame_stats")
    return a, b


class _ConvJob(ctypes.Structure):
    """``vdnh3_short_conv_job`` (include/vdnh3.h)."""
    _fields_ = [("x", ctypes.c_void_p), ("x_row", ctypes.c_int64), ("x_head", ctypes.c_int64),
                ("w_spatial", ctypes.c_void_p), ("w_temporal", ctypes.c_void_p), ("l2norm", ctypes.c_int),
                ("out", ctypes.c_void_p), ("out_row", ctypes.c_int64), ("out_head", ctypes.c_int64)]


def _conv_job(tokens, spatial_weight, temporal_weight, num_frames, frame_size, l2norm, out):
    if tokens.ndim != 3 or frame_size is None:
        raise ValueError("conv features need [rows, heads, dim] and frame_size")
    heads, head_dim = tokens.shape[-2:]
    gh, gw = (int(v) for v in frame_size)
    if gh <= 0 or gw <= 0:
        raise ValueError("frame_size dimensions must be positive")
    channels = heads * head_dim
    if tokens.shape[0] != num_frames * gh * gw:
        raise ValueError("token rows do not match num_frames * frame area")
    if spatial_weight.ndim != 4 or spatial_weight.shape[0] != channels or spatial_weight.shape[1] != 1:
        raise ValueError("spatial convolution must have one depthwise filter per channel")
    kh, kw = spatial_weight.shape[-2:]
    if kh % 2 == 0 or kw % 2 == 0:
        raise ValueError("spatial kernels must have odd dimensions")
    kt = temporal_weight.shape[-1]
    if temporal_weight.numel() != channels * kt or kt <= 0 or kt % 2 == 0:
        raise ValueError("temporal kernel must be positive, odd and symmetrically padded")
    _dim(head_dim)
    device = _lib.require_device(tokens, spatial_weight, temporal_weight, out)
    tokens = _rows(tokens)
    sp = spatial_weight.to(torch.bfloat16).reshape(channels, kh * kw).contiguous()
    tm = temporal_weight.to(torch.bfloat16).reshape(channels, kt).contiguous()
    if out is None:
        out = torch.empty((tokens.shape[0], heads, head_dim), dtype=torch.bfloat16, device=device)
    elif out.shape != tokens.shape or out.dtype != torch.bfloat16 or out.stride(-1) != 1:
        raise ValueError("out must be a bf16 [rows, heads, dim] view with contiguous dim")
    job = _ConvJob(_lib.ptr(tokens), tokens.stride(0), tokens.stride(1), _lib.ptr(sp), _lib.ptr(tm), int(bool(l2norm)),
                   _lib.ptr(out), out.stride(0), out.stride(1))
    return job, (kh, kw, kt, gh, gw, heads, head_dim), device, out, (tokens, sp, tm)


def conv_features(tokens: torch.Tensor, spatial_weight: torch.Tensor, temporal_weight: torch.Tensor,
                  num_frames: int, frame_size, l2norm: bool, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Short-convolution features ``[F*T, H, D]`` bf16 (``vdn_h3/branch.py:443-480``, ``vdn_h3/runtime.py:319-341``).

    Depthwise ``kh x kw`` spatial convolution per frame (rounded to bf16), depthwise temporal
    convolution over the ``num_frames`` frames (zero padded), SiLU, and with ``l2norm`` a unit
    L2 norm over each head's ``D`` channels, as one kernel.
    """
    job, (kh, kw, kt, gh, gw, heads, head_dim), device, out, held = _conv_job(
        tokens, spatial_weight, temporal_weight, num_frames, frame_size, l2norm, out)
    rc = _lib.lib().vdnh3_short_conv(job.x, job.x_row, job.x_head, job.w_spatial, kh, kw, job.w_temporal, kt,
                                     num_frames, gh, gw, heads, head_dim, job.l2norm, job.out, job.out_row,
                                     job.out_head, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_short_conv")
    del held
    return out


def conv_features_batch(items, num_frames: int, frame_size) -> list:
    """``conv_features`` of up to four ``(tokens, spatial_weight, temporal_weight, l2norm, out)`` over the
    same frame grid and kernel sizes in one launch (``vdnh3_short_conv_batch``); returns the outputs."""
    if not 1 <= len(items) <= 4:
        raise ValueError("conv_features_batch takes 1 to 4 tensors")
    jobs, shapes, outs, keep, device = [], set(), [], [], None
    for tokens, sw, tw, l2, out in items:
        job, shape, dev, out, held = _conv_job(tokens, sw, tw, num_frames, frame_size, l2, out)
        if device is not None and dev != device:
            raise ValueError("all tensors of a batch must be on one device")
        device = dev
        jobs.append(job)
        shapes.add(shape)
        outs.append(out)
        keep.append(held)
    if len(shapes) != 1:
        raise ValueError("a batch needs one frame grid, kernel size and head geometry")
    kh, kw, kt, gh, gw, heads, head_dim = shapes.pop()
    arr = (_ConvJob * len(jobs))(*jobs)
    rc = _lib.lib().vdnh3_short_conv_batch(ctypes.addressof(arr), len(jobs), kh, kw, kt, num_frames, gh, gw, heads,
                                           head_dim, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_short_conv_batch")
    del keep
    return outs


class VdnDelta:
    """``Phi = diag(alpha) (I + A)^-1``, ``J = B (I + A)^-1`` by Cholesky, with deferred SPD checks."""

    def __init__(self, tokens_per_frame: int | None = None):
        del tokens_per_frame

    def factor_apply(self, alpha, a_raw, b_raw, *, jay_scale: float = 1.0, need_phi: bool = True):
        if a_raw.shape != b_raw.shape or a_raw.shape[-1] != a_raw.shape[-2]:
            raise ValueError("A and B must share a square [..., D, D] shape")
        if alpha is not None and alpha.shape != a_raw.shape[:-1]:
            raise ValueError("alpha must have shape A.shape[:-1]")
        dim = a_raw.shape[-1]
        _dim(dim)
        device = _lib.require_device(a_raw, b_raw, alpha)
        a32, b32 = a_raw.float().contiguous(), b_raw.float().contiguous()
        n = a32.numel() // (dim * dim)
        phi = torch.empty_like(a32) if need_phi else None
        jay = torch.empty_like(a32)
        info = torch.empty(a32.shape[:-2], dtype=torch.int32, device=device)
        al = None if alpha is None else alpha.float().contiguous()
        rc = _lib.lib().vdnh3_delta_factor(_lib.ptr(a32), _lib.ptr(b32), _lib.ptr(al), _lib.ptr(phi), _lib.ptr(jay),
                                           float(jay_scale), _lib.ptr(info), n, dim, _lib.stream_handle(device))
        _lib.check(rc, "vdnh3_delta_factor")
        _record_status(info)
        return phi, jay


class SanaDelta:
    """``Phi = alpha (I - A/T)``, ``J = B / sqrt(T)``."""

    def __init__(self, tokens_per_frame: int):
        if tokens_per_frame <= 0:
            raise ValueError("tokens_per_frame must be positive")
        self.tokens = int(tokens_per_frame)

    def factor_apply(self, alpha, a_raw, b_raw, *, jay_scale: float = 1.0, need_phi: bool = True):
        """``(Phi, J)``; ``alpha=None`` means ones. ``jay_scale`` multiplies ``J`` after its own rounding (the
        text state's exact 1/2); with ``need_phi=False`` no ``Phi`` is written and ``None`` is returned for it."""
        if a_raw.shape != b_raw.shape or a_raw.shape[-1] != a_raw.shape[-2]:
            raise ValueError("A and B must share a square [..., D, D] shape")
        if alpha is not None and alpha.shape != a_raw.shape[:-1]:
            raise ValueError("alpha must have shape A.shape[:-1]")
        dim = a_raw.shape[-1]
        device = _lib.require_device(a_raw, b_raw, alpha)
        a32, b32 = a_raw.float().contiguous(), b_raw.float().contiguous()
        phi = torch.empty_like(a32) if need_phi else None
        jay = torch.empty_like(a32)
        al = None if alpha is None else alpha.float().contiguous()
        rc = _lib.lib().vdnh3_sana_factor(_lib.ptr(a32), _lib.ptr(b32), _lib.ptr(al), _lib.ptr(phi), _lib.ptr(jay),
                                          float(jay_scale), self.tokens, a32.numel() // (dim * dim), dim,
                                          _lib.stream_handle(device))
        _lib.check(rc, "vdnh3_sana_factor")
        return phi, jay


DELTA_BACKENDS = {"vdn_solve": VdnDelta, "sana_scaled": SanaDelta}


def run_scans_from_factors(transitions, injections, initial=None):
    """Prefix / suffix scans from already factored ``Phi``/``J`` ``[F, H, D, D]``."""
    frames, heads, dim, _ = transitions.shape
    _dim(dim)
    device = _lib.require_device(transitions, injections, initial)
    transitions, injections = transitions.contiguous(), injections.contiguous()
    if initial is not None:
        if initial.shape != (heads, dim, dim):
            raise ValueError("text_state must have shape [heads, D, D]")
        initial = initial.float().contiguous()
    prefix = torch.empty_like(transitions)
    suffix = torch.empty_like(transitions)
    rc = _lib.lib().vdnh3_delta_scan(_lib.ptr(transitions), _lib.ptr(injections), _lib.ptr(initial),
                                     _lib.ptr(prefix), _lib.ptr(suffix), frames, heads, dim,
                                     _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_delta_scan")
    return prefix, suffix


def run_scans_inference(backend, alpha, a_raw, b_raw, text_state=None):
    """Factor all frames, then the bidirectional recurrence (``vdn_h3/branch.py:315-333``)."""
    if a_raw.ndim != 4 or a_raw.shape != b_raw.shape or a_raw.shape[0] == 0:
        raise ValueError("A and B must share non-empty [frames, heads, D, D] shape")
    phi, jay = backend.factor_apply(alpha, a_raw, b_raw)
    return run_scans_from_factors(phi, jay, text_state)


def frame_mean(xv: torch.Tensor, num_frames: int, tokens_per_frame: int) -> torch.Tensor:
    """``xv.reshape(F, T, -1).mean(1, dtype=float32)``."""
    device = _lib.require_device(xv)
    if xv.stride(1) != 1:
        xv = xv.contiguous()
    out = torch.empty((num_frames, xv.shape[1]), dtype=torch.float32, device=device)
    rc = _lib.lib().vdnh3_frame_mean(_lib.ptr(xv), xv.stride(0), num_frames, tokens_per_frame, xv.shape[1],
                                     _lib.ptr(out), _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_frame_mean")
    return out


def linear_f32(x: torch.Tensor, weight: torch.Tensor, bias=None) -> torch.Tensor:
    """fp32 ``F.linear(x, weight.float(), bias)`` (small projections)."""
    device = _lib.require_device(x, weight, bias)
    x = x.float().contiguous()
    if weight.dtype == torch.bfloat16:
        w, w_bf16 = weight.contiguous(), 1
    else:
        w, w_bf16 = weight.float().contiguous(), 0
    b = None if bias is None else bias.float().contiguous()
    m, k = x.shape
    n = w.shape[0]
    out = torch.empty((m, n), dtype=torch.float32, device=device)
    rc = _lib.lib().vdnh3_linear_f32(_lib.ptr(x), x.stride(0), _lib.ptr(w), w_bf16, w.stride(0), _lib.ptr(b),
                                     _lib.ptr(out), out.stride(0), m, n, k, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_linear_f32")
    return out


def alpha_gate(frame_mean_f32, weight_down, weight_up, dt_bias, a_log, num_heads, head_dim):
    """``exp(-exp(A_log) * softplus(W_up W_down m + dt_bias))`` as ``[F, H, D]`` fp32."""
    d1 = linear_f32(frame_mean_f32, weight_down)
    d2 = linear_f32(d1, weight_up, dt_bias)
    if d2.shape[-1] != num_heads * head_dim or a_log.numel() != num_heads:
        raise ValueError("alpha weights are incompatible with head geometry")
    device = d2.device
    alpha = torch.empty((d2.shape[0], num_heads, head_dim), dtype=torch.float32, device=device)
    a_log = a_log.float().contiguous()
    rc = _lib.lib().vdnh3_alpha_decay(_lib.ptr(d2), _lib.ptr(a_log), _lib.ptr(alpha), d2.shape[0], num_heads,
                                      head_dim, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_alpha_decay")
    return alpha


_BOUNDS_CACHE: dict[tuple, torch.Tensor] = {}


def _device_bounds(bounds, device) -> torch.Tensor:
    """The ``(lo, hi)`` pairs as a device int32 tensor, copied once per geometry and device."""
    key = (tuple((int(lo), int(hi)) for lo, hi in bounds), device.type, device.index)
    cached = _BOUNDS_CACHE.get(key)
    if cached is None:
        if len(_BOUNDS_CACHE) > 64:
            _BOUNDS_CACHE.clear()
        cached = torch.tensor([x for pair in key[0] for x in pair], dtype=torch.int32).to(device)
        _BOUNDS_CACHE[key] = cached
    return cached


def readout_epilogue(q_raw, prefix, suffix, alpha, bounds, norm_weight, gate, *, text_state=None,
                     bridge="alpha", num_frames, tokens_per_frame, out=None, q_features=False, gate_hidden=None,
                     gate_up_weight=None, gate_up_bias=None, frame_range=None):
    """Gather, readout and RMSNorm/gate epilogue: ``[F*T, H*D]`` bf16.

    ``q_raw`` is the raw query (``L2(SiLU(q))`` is applied on load) unless ``q_features`` says it
    already holds the query features (short-convolution output). With ``gate=None`` the output
    gate ``sigmoid(gate_hidden @ gate_up_weight.T + gate_up_bias)`` (``vdn_h3/branch.py:754-758``,
    ``gate_hidden`` = the down-projection ``[F*T, D]``) is computed inside the readout kernel.
    ``frame_range=(start, stop)`` reads out only frames ``start .. stop - 1`` of the ``num_frames``
    that ``prefix``, ``suffix``, ``alpha`` and ``bounds`` describe (the reference's frame-tiled gather,
    ``_gather_range``, ``vdn_h3/runtime.py:513-517``): ``q_raw``, ``gate`` / ``gate_hidden`` and the
    ``[(stop - start)*T, H*D]`` result then hold that range's rows only.
    """
    if bridge not in ("alpha", "none"):
        raise ValueError("bridge must be 'alpha' or 'none'")
    rows, heads, dim = q_raw.shape
    _dim(dim)
    if len(bounds) != num_frames:
        raise ValueError("bounds must contain one entry per frame")
    for frame, (lo, hi) in enumerate(bounds):
        if lo > frame or hi < frame or lo > hi:
            raise ValueError(f"bounds[{frame}] does not contain its query frame")
    start, stop = (0, num_frames) if frame_range is None else (int(frame_range[0]), int(frame_range[1]))
    if not 0 <= start < stop <= num_frames:
        raise ValueError(f"frame_range ({start}, {stop}) is not a non-empty range of the {num_frames} frames")
    frames_state = (num_frames, heads, dim, dim)
    for name, t in (("prefix", prefix), ("suffix", suffix)):
        if t.dtype != torch.float32 or tuple(t.shape) != frames_state:
            raise ValueError(f"{name} must be fp32 {list(frames_state)}, got {t.dtype} {list(t.shape)}")
    if bridge == "alpha" and (alpha is None or tuple(alpha.shape) != frames_state[:3]):
        raise ValueError(f"alpha must be [{num_frames}, {heads}, {dim}]")
    if text_state is not None and tuple(text_state.shape) != (heads, dim, dim):
        raise ValueError(f"text_state must be [{heads}, {dim}, {dim}]")
    if rows != (stop - start) * tokens_per_frame:
        raise ValueError(f"q holds {rows} rows, not the range's frames * tokens_per_frame = "
                         f"{(stop - start) * tokens_per_frame}")
    fused = gate is None
    if fused:
        if gate_hidden is None or gate_up_weight is None:
            raise ValueError("readout needs the gate or gate_hidden and gate_up_weight")
        if gate_hidden.shape != (rows, dim) or gate_up_weight.shape != (heads * dim, dim):
            raise ValueError(f"gate_hidden must be [{rows}, {dim}] and gate_up_weight [{heads * dim}, {dim}]")
        if gate_up_bias is not None and gate_up_bias.shape != (heads * dim,):
            raise ValueError(f"gate_up_bias must be [{heads * dim}]")
    device = _lib.require_device(q_raw, prefix, suffix, alpha, gate, text_state, out, gate_hidden, gate_up_weight,
                                 gate_up_bias)
    q_raw = _rows(q_raw)
    bounds_t = _device_bounds(bounds, device)
    norm_w = norm_weight.to(torch.bfloat16).contiguous()
    if fused:
        gate_hidden = gate_hidden.to(torch.bfloat16)
        if gate_hidden.stride(1) != 1 or gate_hidden.stride(0) % 8 or gate_hidden.data_ptr() % 16:
            gate_hidden = gate_hidden.contiguous()
        gate_up_weight = gate_up_weight.to(torch.bfloat16).contiguous()
        if gate_up_bias is not None:
            gate_up_bias = gate_up_bias.to(torch.bfloat16).contiguous()
        gate = gate_hidden  # alignment checks below are for the gate path only
    else:
        gate = gate.to(torch.bfloat16)
        if gate.stride(1) != 1:
            gate = gate.contiguous()
    text = None if text_state is None else text_state.float().contiguous()
    if out is None:
        out = torch.empty((rows, heads * dim), dtype=torch.bfloat16, device=device)
    if out.stride(-1) != 1 or out.stride(0) % 8 or out.data_ptr() % 16:
        raise ValueError("out must have contiguous, 16-byte aligned rows")
    if not fused and (gate.stride(0) % 8 or gate.data_ptr() % 16):
        gate = gate.contiguous()
    logsum = None
    if bridge == "alpha":
        alpha = alpha.float().contiguous()
        logsum = torch.empty((num_frames + 1, heads, dim), dtype=torch.float32, device=device)
        rc = _lib.lib().vdnh3_alpha_logsum(_lib.ptr(alpha), num_frames, heads, dim, _lib.ptr(logsum),
                                           _lib.stream_handle(device))
        _lib.check(rc, "vdnh3_alpha_logsum")
    # the operands stay bound to locals until the launch has been enqueued (a temporary copy freed
    # earlier could hand its memory to the next copy)
    prefix, suffix = prefix.contiguous(), suffix.contiguous()
    common = (_lib.ptr(q_raw), q_raw.stride(0), q_raw.stride(1), int(bool(q_features)), _lib.ptr(prefix),
              _lib.ptr(suffix), _lib.ptr(logsum), _lib.ptr(text), _lib.ptr(bounds_t),
              int(bridge == "alpha"), _lib.ptr(norm_w))
    tail = (_lib.ptr(out), out.stride(0), num_frames, start, stop - start, tokens_per_frame, heads, dim,
            _lib.stream_handle(device))
    if fused:
        rc = _lib.lib().vdnh3_readout_fused_gate(*common, _lib.ptr(gate_hidden), gate_hidden.stride(0),
                                                 _lib.ptr(gate_up_weight), _lib.ptr(gate_up_bias), *tail)
        _lib.check(rc, "vdnh3_readout_fused_gate")
    else:
        rc = _lib.lib().vdnh3_readout(*common, _lib.ptr(gate), gate.stride(0), *tail)
        _lib.check(rc, "vdnh3_readout")
    return out


def fill_rows(t: torch.Tensor, value: float = 0.0):
    """Fill a bf16 ``[rows, cols]`` view (contiguous rows) with ``value`` on the device."""
    if t.numel() == 0:
        return t
    device = _lib.require_device(t)
    rc = _lib.lib().vdnh3_fill_rows_bf16(_lib.ptr(t), t.stride(0), t.shape[0], t.shape[1], float(value),
                                         _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_fill_rows_bf16")
    return t


__all__ = ["DELTA_BACKENDS", "SanaDelta", "TEXT_STATE_SCALE", "VdnDelta", "alpha_gate", "cholesky_runtime_scope",
           "conv_features", "fill_rows", "frame_mean", "frame_statistics_raw", "linear_f32", "readout_epilogue",
           "run_scans_from_factors", "run_scans_inference"]
