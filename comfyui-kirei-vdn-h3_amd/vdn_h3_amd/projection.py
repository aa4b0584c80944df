"""Precision-dispatched ``to_out_linear`` (bf16 / fp8 / int8) on MI355X.

Mirrors ``vdn_h3/projection.py``: one storage slot for quantised weights (``:41-47``), dispatch
on the stored dtype in ``project`` (``:259-268``) and ``prepare_projection_maps`` (``:209-232``).
INT8 here is W8A8 with per-token activation and per-output-channel weight scales on the int8
MFMA; the reference's comfy-kitchen ``ck.int8_linear`` additionally applies a ConvRot
rotation, which is not reproduced (that library is not available to check against).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping, Sequence

import torch

from . import fp8 as _fp8
from . import linear as _linear
from .fp8 import BF16_WEIGHT_KEY, DEFAULT_SKIP_END_BLOCKS, FP8_SCALE_KEY, FP8_WEIGHT_KEY

INT8_WEIGHT_KEY = FP8_WEIGHT_KEY
INT8_SCALE_KEY = FP8_SCALE_KEY
PROJECTION_PRECISIONS = ("bf16", "fp8", "int8")


@dataclass(frozen=True)
class INT8ProjectionInfo:
    original_bytes: int
    quantized_bytes: int
    quantized_blocks: int
    bf16_blocks: int
    skip_end_blocks: int
    per_channel: bool = True


def quantize_int8_weight(weight: torch.Tensor):
    """Per-output-channel symmetric int8 codes and ``[1, N]`` scales."""
    q, s = _linear.quantize_rows(weight.to(torch.bfloat16), _linear.KIND_I8)
    return q, s.reshape(1, -1)


def prepare_int8_projection_maps(branch_maps: Sequence[Mapping[str, torch.Tensor]], device, *,
                                 skip_end_blocks: int = 0):
    device = torch.device(device)
    if isinstance(skip_end_blocks, bool) or not isinstance(skip_end_blocks, int) or skip_end_blocks < 0:
        raise ValueError("skip_end_blocks must be a non-negative integer")
    count = len(branch_maps)
    if count == 0:
        raise ValueError("branch_maps cannot be empty")
    if skip_end_blocks and skip_end_blocks * 2 >= count:
        raise ValueError(f"skip_end_blocks={skip_end_blocks} leaves no INT8 interior blocks for {count} branches")
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
            q, s = quantize_int8_weight(weight.to(device))
            copied.pop(BF16_WEIGHT_KEY)
            copied[INT8_WEIGHT_KEY], copied[INT8_SCALE_KEY] = q, s
            quant += q.numel() + 4 * s.numel()
            nq += 1
        out.append(copied)
    return tuple(out), INT8ProjectionInfo(orig, quant, nq, nb, skip_end_blocks)


def prepare_projection_maps(branch_maps, device, precision: str, *, skip_end_blocks: int | None = None):
    if precision not in PROJECTION_PRECISIONS:
        raise ValueError(f"unknown VDN projection precision {precision!r}")
    if precision == "bf16":
        return tuple(dict(block) for block in branch_maps), None
    if precision == "fp8":
        return _fp8.prepare_projection_maps(
            branch_maps, device, skip_end_blocks=DEFAULT_SKIP_END_BLOCKS if skip_end_blocks is None
            else int(skip_end_blocks))
    return prepare_int8_projection_maps(branch_maps, device,
                                        skip_end_blocks=0 if skip_end_blocks is None else int(skip_end_blocks))


def projection_out_features(weights: Mapping[str, torch.Tensor]) -> int:
    if BF16_WEIGHT_KEY in weights:
        return int(weights[BF16_WEIGHT_KEY].shape[0])
    if FP8_WEIGHT_KEY in weights:
        return int(weights[FP8_WEIGHT_KEY].shape[0])
    raise KeyError("VDN branch has no projection weight")


def project(rows: torch.Tensor, weights: Mapping[str, torch.Tensor], *, out=None, accumulate=False):
    """Dispatch on the stored weight: bf16, int8 (W8A8 per-token x per-channel) or fp8."""
    if BF16_WEIGHT_KEY in weights:
        return _linear.linear(rows, weights[BF16_WEIGHT_KEY], out=out, accumulate=accumulate)
    if FP8_WEIGHT_KEY not in weights:
        raise KeyError("VDN projection state has no supported weight representation")
    quantized, scale = weights[FP8_WEIGHT_KEY], weights[FP8_SCALE_KEY]
    if quantized.dtype == torch.int8:
        x_q, x_s = _linear.quantize_rows(rows.to(torch.bfloat16), _linear.KIND_I8)
        return _linear.gemm_w8a8(x_q, x_s, quantized, scale, out=out, accumulate=accumulate)
    return _fp8.project(rows, weights, out=out, accumulate=accumulate)


__all__ = ["BF16_WEIGHT_KEY", "FP8_SCALE_KEY", "FP8_WEIGHT_KEY", "INT8ProjectionInfo", "INT8_SCALE_KEY",
           "INT8_WEIGHT_KEY", "PROJECTION_PRECISIONS", "prepare_int8_projection_maps", "prepare_projection_maps",
           "project", "projection_out_features", "quantize_int8_weight"]
