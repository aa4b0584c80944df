"""FP8 (OCP e4m3fn) execution of the VDN ``to_out_linear`` projection on MI355X.

Mirrors ``vdn_h3/fp8.py``: the storage keys (``:31-33``), ``quantize_activation`` (``:108-133``),
weight quantisation (``:88-96``), ``prepare_projection_maps`` with bf16 edge blocks
(``:168-222``) and ``project`` (``:239-266``). The activation quantisation and the scaled GEMM
are HIP kernels (``vdnh3_quant_rows`` / ``vdnh3_quant_tensor_f8`` / ``vdnh3_gemm``). gfx950's
fp8 MFMA runs both scale layouts; rowwise activation scales with per-output-channel weight
scales are the default, per-tensor scales are kept for checkpoints quantised that way.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping, Sequence

import torch

from . import linear as _linear

FP8_DTYPE = torch.float8_e4m3fn
FP8_MAX = 448.0
FP8_WEIGHT_KEY = "to_out_linear.weight_fp8"
FP8_SCALE_KEY = "to_out_linear.weight_scale"
BF16_WEIGHT_KEY = "to_out_linear.weight"
PROJECTION_PRECISIONS = ("bf16", "fp8")
DEFAULT_SKIP_END_BLOCKS = 4


@dataclass(frozen=True)
class FP8ProjectionInfo:
    per_tensor: bool
    original_bytes: int
    quantized_bytes: int
    quantized_blocks: int
    bf16_blocks: int
    skip_end_blocks: int


def quantize_activation(rows: torch.Tensor, *, per_tensor: bool):
    """``(codes e4m3fn [M, K], scale)``: scale ``[M, 1]`` rowwise or ``[1, 1]`` per tensor."""
    if rows.ndim != 2 or not rows.is_cuda:
        raise ValueError("FP8 projection activation must be a GPU [rows, channels] tensor")
    if rows.dtype != torch.bfloat16:
        rows = rows.to(torch.bfloat16)
    if per_tensor:
        return _linear.quantize_tensor_fp8(rows)
    return _linear.quantize_rows(rows, _linear.KIND_F8)


def quantize_weight(weight: torch.Tensor, *, per_tensor: bool):
    """Weight codes and scales (``[1, 1]`` per tensor or ``[1, N]`` per output channel)."""
    w = weight.to(dtype=torch.bfloat16)
    if per_tensor:
        return _linear.quantize_tensor_fp8(w)
    q, s = _linear.quantize_rows(w, _linear.KIND_F8)
    return q, s.reshape(1, -1)


def fp8_supported(device) -> bool:
    device = torch.device(device)
    return device.type == "cuda" and torch.cuda.is_available()


def prepare_projection_maps(branch_maps: Sequence[Mapping[str, torch.Tensor]], device, *,
                            skip_end_blocks: int = DEFAULT_SKIP_END_BLOCKS, per_tensor: bool = False):
    """BF16 edge blocks and FP8 interior blocks, as the reference's accuracy policy."""
    device = torch.device(device)
    if not fp8_supported(device):
        raise RuntimeError(f"FP8 VDN projection needs a ROCm GPU; {device} is not one")
    if isinstance(skip_end_blocks, bool) or not isinstance(skip_end_blocks, int) or skip_end_blocks < 0:
        raise ValueError("skip_end_blocks must be a non-negative integer")
    count = len(branch_maps)
    if count == 0:
        raise ValueError("branch_maps cannot be empty")
    if skip_end_blocks * 2 >= count:
        raise ValueError(f"skip_end_blocks={skip_end_blocks} leaves no FP8 interior blocks for {count} branches")
    out, orig, quant, nq, nb = [], 0, 0, 0, 0
    for index, block in enumerate(branch_maps):
        if BF16_WEIGHT_KEY not in block:
            raise KeyError(f"VDN block {index} has no {BF16_WEIGHT_KEY!r}")
        weight = block[BF16_WEIGHT_KEY]
        orig += weight.numel() * weight.element_size()
        copied = dict(block)
        if index < skip_end_blocks or index >= count - skip_end_blocks:
            quant += weight.numel() * weight.element_size()
            nb += 1
        else:
            q, s = quantize_weight(weight.to(device), per_tensor=per_tensor)
            copied.pop(BF16_WEIGHT_KEY)
            copied[FP8_WEIGHT_KEY], copied[FP8_SCALE_KEY] = q, s
            quant += q.numel() + s.numel() * 4
            nq += 1
        out.append(copied)
    return tuple(out), FP8ProjectionInfo(per_tensor, orig, quant, nq, nb, skip_end_blocks)


def project(rows: torch.Tensor, weights: Mapping[str, torch.Tensor], *, out=None, accumulate=False):
    """BF16 or FP8 ``to_out_linear`` by stored dtype; the result is bf16 ``[M, N]``."""
    if BF16_WEIGHT_KEY in weights:
        return _linear.linear(rows, weights[BF16_WEIGHT_KEY], out=out, accumulate=accumulate)
    w_q, w_s = weights[FP8_WEIGHT_KEY], weights[FP8_SCALE_KEY]
    x_q, x_s = quantize_activation(rows, per_tensor=w_s.numel() == 1)
    return _linear.gemm_w8a8(x_q, x_s, w_q, w_s, out=out, accumulate=accumulate)


__all__ = ["BF16_WEIGHT_KEY", "DEFAULT_SKIP_END_BLOCKS", "FP8ProjectionInfo", "FP8_DTYPE", "FP8_MAX", "FP8_SCALE_KEY",
           "FP8_WEIGHT_KEY", "PROJECTION_PRECISIONS", "fp8_supported", "prepare_projection_maps", "project",
           "quantize_activation", "quantize_weight"]
