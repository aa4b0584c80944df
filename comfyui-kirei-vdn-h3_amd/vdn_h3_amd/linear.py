"""Projections on MI355X MFMA through ``vdnh3_gemm`` (bf16, W8A8 int8 and fp8 e4m3fn).

``linear(x, weight, bias)`` is ``F.linear`` in bf16 (fp32 accumulation, one rounding);
``sigmoid_linear`` is ``torch.sigmoid(F.linear(...))`` with the reference's intermediate bf16
rounding (``vdn_h3/branch.py:736``, ``:754-758``, ``vdn_h3/hybrid.py:520-522``);
``gemm_w8a8`` multiplies pre-quantised operands with per-row and per-column scales fused into
the epilogue; ``quantize_rows`` / ``quantize_tensor_fp8`` are the matching quantisation passes.
"""

from __future__ import annotations

import torch

from . import _lib

KIND_BF16, KIND_I8, KIND_F8 = 0, 1, 2
OUT_BF16, OUT_F32, OUT_I32 = 0, 1, 2
_OUT_CODES = {torch.bfloat16: OUT_BF16, torch.float32: OUT_F32, torch.int32: OUT_I32}


def _operand(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or (t.stride(0) * t.element_size()) % 16 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def gemm(kind: int, a: torch.Tensor, b: torch.Tensor, *, a_scale=None, b_scale=None, alpha: float = 1.0,
         bias=None, act: str | None = None, out_dtype=torch.bfloat16, out: torch.Tensor | None = None,
         accumulate: bool = False, round_linear: bool = True, act_cols: int = 0) -> torch.Tensor:
    """``C = act(A B^T * scales + bias)``; ``a``: ``[M, K]``, ``b``: ``[N, K]`` (nn.Linear weight layout).

    ``act_cols`` > 0 limits the activation to the first ``act_cols`` output columns (the rest are the
    plain linear result), so two projections of the same rows run as one GEMM.
    """
    if a.ndim != 2 or b.ndim != 2 or a.shape[1] != b.shape[1]:
        raise ValueError(f"gemm operands must be [M, K] and [N, K]; got {tuple(a.shape)} and {tuple(b.shape)}")
    _lib.forward_only("gemm", a, b, a_scale, b_scale, bias)
    device = _lib.require_device(a, b, a_scale, b_scale, bias, out)
    m, k = a.shape
    n = b.shape[0]
    a, b = _operand(a), _operand(b)
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs an existing output tensor")
        out = torch.empty((m, n), dtype=out_dtype, device=device)
    if out.shape != (m, n) or out.stride(1) != 1:
        raise ValueError(f"out must be [{m}, {n}] with a contiguous last dim")
    if out.dtype not in _OUT_CODES:
        raise TypeError(f"unsupported output dtype {out.dtype}")
    if a_scale is not None:
        a_scale = a_scale.reshape(-1).float().contiguous()
    if b_scale is not None:
        b_scale = b_scale.reshape(-1).float().contiguous()
    bias_bf16 = 0
    if bias is not None:
        bias = bias.reshape(-1).contiguous()
        if bias.dtype == torch.bfloat16:
            bias_bf16 = 1
        elif bias.dtype != torch.float32:
            bias = bias.float()
    act_code = {None: 0, "sigmoid": 1}[act]
    if act_cols:
        if act_code == 0 or not 0 < act_cols <= n:
            raise ValueError(f"act_cols must lie in (0, {n}] and needs an activation")
        act_code |= int(act_cols) << 1
    rc = _lib.lib().vdnh3_gemm(
        kind, _lib.ptr(a), a.stride(0), _lib.ptr(b), b.stride(0), _lib.ptr(out), out.stride(0), m, n, k,
        _lib.ptr(a_scale), 0 if a_scale is None else a_scale.numel(), _lib.ptr(b_scale),
        0 if b_scale is None else b_scale.numel(), float(alpha), _lib.ptr(bias), bias_bf16, act_code,
        _OUT_CODES[out.dtype], int(accumulate), int(round_linear), _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_gemm")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias=None, *, out=None, accumulate=False) -> torch.Tensor:
    """bf16 ``F.linear(x, weight, bias)`` for 2-D ``x`` (fp32 accumulation, rounded once)."""
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("linear computes in bf16")
    return gemm(KIND_BF16, x, weight, bias=bias, out=out, accumulate=accumulate)


def sigmoid_linear_split(x: torch.Tensor, weight: torch.Tensor, act_cols: int) -> torch.Tensor:
    """``F.linear(x, weight)`` in bf16 with ``sigmoid`` on the first ``act_cols`` columns (the linear
    value rounded to bf16 first there, as ``sigmoid_linear``); the remaining columns equal ``linear``."""
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("sigmoid_linear_split computes in bf16")
    return gemm(KIND_BF16, x, weight, act="sigmoid", round_linear=True, act_cols=act_cols)


def sigmoid_linear(x: torch.Tensor, weight: torch.Tensor, bias=None, *, out=None) -> torch.Tensor:
    """``torch.sigmoid(F.linear(x, weight, bias))`` in bf16, rounding the linear result first."""
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("sigmoid_linear computes in bf16")
    return gemm(KIND_BF16, x, weight, bias=bias, act="sigmoid", out=out, round_linear=True)


def quantize_rows(x: torch.Tensor, kind: int):
    """Row-wise symmetric quantisation of bf16 ``[M, K]``: ``(codes, scale[M, 1] fp32)``."""
    if x.ndim != 2 or x.dtype != torch.bfloat16:
        raise ValueError("quantize_rows expects a bf16 [rows, channels] matrix")
    device = _lib.require_device(x)
    x = _operand(x)
    m, k = x.shape
    dtype = torch.int8 if kind == KIND_I8 else torch.float8_e4m3fn
    q = torch.empty((m, k), dtype=dtype, device=device)
    scale = torch.empty((m, 1), dtype=torch.float32, device=device)
    rc = _lib.lib().vdnh3_quant_rows(kind, _lib.ptr(x), x.stride(0), m, k, _lib.ptr(q), q.stride(0),
                                     _lib.ptr(scale), _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_quant_rows")
    return q, scale


def quantize_tensor_fp8(x: torch.Tensor):
    """Per-tensor e4m3fn quantisation of a bf16 tensor: ``(codes, scale[1, 1] fp32)``."""
    if x.dtype != torch.bfloat16:
        raise ValueError("quantize_tensor_fp8 expects bf16")
    device = _lib.require_device(x)
    x = x.contiguous()
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=device)
    scale = torch.empty((1, 1), dtype=torch.float32, device=device)
    amax = torch.empty(1, dtype=torch.float32, device=device)
    rc = _lib.lib().vdnh3_quant_tensor_f8(_lib.ptr(x), x.numel(), _lib.ptr(q), _lib.ptr(scale), _lib.ptr(amax),
                                          _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_quant_tensor_f8")
    return q, scale


def quantize_tensor_fp8_into(x: torch.Tensor, q: torch.Tensor, scale: torch.Tensor):
    """``quantize_tensor_fp8`` into caller-owned ``q`` (e4m3fn, ``x``'s shape) and ``scale`` (fp32, 1 value),
    with nothing allocated on the device (``vdnh3_quant_tensor_f8_noalloc``): usable inside a HIP graph
    capture. ``x`` must be contiguous bf16 with at most ``vdnh3_quant_tensor_f8_noalloc_max_elements()``
    values. Calls that overlap on one GPU share the library's scratch and race."""
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("quantize_tensor_fp8_into expects a contiguous bf16 tensor")
    if q.dtype != torch.float8_e4m3fn or q.shape != x.shape or not q.is_contiguous():
        raise ValueError("q must be a contiguous float8_e4m3fn tensor of x's shape")
    if scale.dtype != torch.float32 or scale.numel() != 1:
        raise ValueError("scale must be one fp32 value")
    device = _lib.require_device(x, q, scale)
    rc = _lib.lib().vdnh3_quant_tensor_f8_noalloc(_lib.ptr(x), x.numel(), _lib.ptr(q), _lib.ptr(scale),
                                                  _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_quant_tensor_f8_noalloc")
    return q, scale


def gemm_w8a8(a_q, a_scale, b_q, b_scale, *, out_dtype=torch.bfloat16, bias=None, out=None, accumulate=False):
    """``(a_q b_q^T) * a_scale[m] * b_scale[n] (+ bias)`` for int8 or fp8 e4m3fn operands."""
    if a_q.dtype == torch.int8 and b_q.dtype == torch.int8:
        kind = KIND_I8
    elif a_q.dtype == torch.float8_e4m3fn and b_q.dtype == torch.float8_e4m3fn:
        kind = KIND_F8
    else:
        raise TypeError(f"W8A8 operands must both be int8 or both float8_e4m3fn, got {a_q.dtype}/{b_q.dtype}")
    return gemm(kind, a_q.view(torch.uint8) if kind == KIND_F8 else a_q,
                b_q.view(torch.uint8) if kind == KIND_F8 else b_q,
                a_scale=a_scale, b_scale=b_scale, bias=bias, out_dtype=out_dtype, out=out, accumulate=accumulate)


def int8_accumulators(a_q: torch.Tensor, b_q: torch.Tensor) -> torch.Tensor:
    """Raw int32 accumulators ``a_q b_q^T`` of two int8 matrices."""
    return gemm(KIND_I8, a_q, b_q, out_dtype=torch.int32)


LINEAR_PRECISIONS = ("bf16", "int8", "fp8")


class HipLinear(torch.nn.Module):
    """``nn.Linear`` (no bias) on MI355X MFMA with bf16, W8A8 int8 or fp8 e4m3fn weights.

    The host model's ``attn.qkv_proj`` / ``attn.out_proj`` (``vdn_h3/hybrid.py:263``, ``:535``)
    and the VDN ``to_out_linear`` run through it. ``int8`` stores symmetric per-output-channel
    codes and quantises activations per token at call time (int32 accumulation, both scales in
    the epilogue); ``fp8`` stores e4m3fn codes with a per-tensor or per-channel scale and
    quantises activations the same way (per tensor / per token). Output is bf16.
    """

    def __init__(self, weight: torch.Tensor, precision: str = "bf16", *, per_tensor: bool = False):
        super().__init__()
        if precision not in LINEAR_PRECISIONS:
            raise ValueError(f"unknown precision {precision!r}; expected one of {LINEAR_PRECISIONS}")
        if weight.ndim != 2:
            raise ValueError("weight must be [out_features, in_features]")
        _lib.require_device(weight)
        self.precision = precision
        self.per_tensor = bool(per_tensor)
        self.out_features, self.in_features = int(weight.shape[0]), int(weight.shape[1])
        w = weight.detach().to(torch.bfloat16).contiguous()  # a constant of the forward-only op
        if precision == "bf16":
            self.register_buffer("weight", w)
            self.register_buffer("weight_scale", None)
        elif precision == "int8":
            q, s = quantize_rows(w, KIND_I8)
            self.register_buffer("weight", q)
            self.register_buffer("weight_scale", s.reshape(1, -1))
        else:
            q, s = quantize_tensor_fp8(w) if per_tensor else quantize_rows(w, KIND_F8)
            self.register_buffer("weight", q)
            self.register_buffer("weight_scale", s.reshape(1, -1))

    def forward(self, x: torch.Tensor, *, out: torch.Tensor | None = None, accumulate: bool = False):
        if x.ndim != 2 or x.shape[1] != self.in_features:
            raise ValueError(f"expected [rows, {self.in_features}] input, got {tuple(x.shape)}")
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        if self.precision == "bf16":
            return linear(x, self.weight, out=out, accumulate=accumulate)
        if self.precision == "int8":
            xq, xs = quantize_rows(x, KIND_I8)
        elif self.per_tensor:
            xq, xs = quantize_tensor_fp8(x)
        else:
            xq, xs = quantize_rows(x, KIND_F8)
        return gemm_w8a8(xq, xs, self.weight, self.weight_scale, out=out, accumulate=accumulate)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, precision={self.precision}"
