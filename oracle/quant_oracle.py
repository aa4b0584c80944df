"""Oracle: W8A8 quantisation and quantised GEMMs (CPU; integer products exact in int64).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``fp8_quantize_rows`` / ``fp8_quantize_tensor`` -> ``vdn_h3/fp8.py:29-30``, ``:88-105``
  (``scale = max(amax / 448, 1e-12)``, ``q = clamp(x / scale, +-448) -> float8_e4m3fn``).
* ``fp8_linear``    -> ``vdn_h3/fp8.py:239-262`` (``_scaled_mm(x_q, W_q^T, s_x, s_w)``, bf16 out),
  computed as the dequantised product accumulated in float64.
* ``int8_quantize_rows`` / ``int8_linear`` -> the W8A8 INT8 projection of the hybrid block's
  q/k/v and out GEMMs (``vdn_h3/hybrid.py:263``, ``:535``: ComfyUI-native
  ``qkv_proj``/``out_proj``; the reference's own INT8 path is comfy-kitchen
  ``ck.int8_linear`` with ConvRot, ``vdn_h3/projection.py:243-256``, a library absent here).
  Symmetric per-row scale ``amax / 127``, round half to even, clamp to +-127, int32
  accumulation, ``acc * s_row * s_col`` epilogue.

Pinning (``tests/test_oracle_quant.py``):

* ``int8_linear`` accumulators: brute-force pure-Python dot products on a small case, and
  exact identities (``A @ I`` returns the codes, sign flips, int32 range at K=5120).
* ``fp8`` codes: every one of the 256 e4m3fn codes round-trips through ``float8_e4m3fn``;
  the saturation at 448, the ``1e-12`` scale floor and round-to-nearest-even ties are
  checked on hand-picked values.
* ConvRot INT8 (comfy-kitchen): parity unpinned (library absent; no fixture exists).
"""

from __future__ import annotations

import numpy as np
import torch

FP8_MAX = 448.0      # torch.finfo(torch.float8_e4m3fn).max, vdn_h3/fp8.py:30
INT8_MAX = 127.0


def fp8_quantize_rows(x):
    """Rowwise e4m3fn quantisation (``vdn_h3/fp8.py:99-105``, ``per_tensor=False``)."""
    v = x.float()
    scale = (v.abs().amax(dim=1, keepdim=True) / FP8_MAX).clamp_min(1e-12)
    return (v / scale).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn), scale


def fp8_quantize_tensor(x):
    """Per-tensor e4m3fn quantisation (``vdn_h3/fp8.py:99-105``, ``per_tensor=True``)."""
    v = x.float()
    scale = (v.abs().amax() / FP8_MAX).clamp_min(1e-12).reshape(1, 1)
    return (v / scale).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn), scale


def fp8_quantize_weight(weight, per_tensor):
    """Weight quantisation (``vdn_h3/fp8.py:88-96``); per-channel scales come back as ``[1, N]``."""
    if per_tensor:
        return fp8_quantize_tensor(weight)
    q, s = fp8_quantize_rows(weight)
    return q, s.reshape(1, -1)


def fp8_linear(x_q, x_scale, w_q, w_scale, out_dtype=torch.bfloat16):
    """Dequantised fp8 GEMM ``(x_q s_x) (w_q s_w)^T`` accumulated in float64 (``vdn_h3/fp8.py:254-262``)."""
    acc = x_q.double() @ w_q.double().t()
    out = acc * x_scale.double().reshape(-1, 1) * w_scale.double().reshape(1, -1)
    return out.to(out_dtype)


def int8_quantize_rows(x):
    """Symmetric per-row int8: ``s = amax/127`` (fp32), ``q = rne(x / s)`` clamped to +-127.

    A zero row gets scale 1e-12 (the fp8 path's floor) and all-zero codes.
    """
    v = x.float()
    scale = (v.abs().amax(dim=1, keepdim=True) / INT8_MAX).clamp_min(1e-12)
    q = torch.round(v / scale).clamp(-INT8_MAX, INT8_MAX).to(torch.int8)   # torch.round = half to even
    return q, scale


def int8_accumulate(a_q, b_q):
    """Exact int32 accumulators ``A_q B_q^T`` (``[M,K] x [N,K] -> [M,N]``) via int64 numpy."""
    a = np.asarray(a_q.numpy(), dtype=np.int64)
    b = np.asarray(b_q.numpy(), dtype=np.int64)
    acc = a @ b.T
    if acc.size and (acc.max() > np.iinfo(np.int32).max or acc.min() < np.iinfo(np.int32).min):
        raise OverflowError("int32 accumulator overflow")
    return torch.from_numpy(acc.astype(np.int32))


def int8_linear(a_q, a_scale, b_q, b_scale, out_dtype=torch.bfloat16):
    """``acc * s_a[m] * s_b[n]`` in fp32, one rounding to ``out_dtype``."""
    acc = int8_accumulate(a_q, b_q).float()
    return (acc * a_scale.float().reshape(-1, 1) * b_scale.float().reshape(1, -1)).to(out_dtype)
