"""The VDN linear branch the hybrid block calls: ``OptimizedLinearBranch.projected_delta``.

Mirrors ``vdn_h3/runtime.py`` (``OptimizedLinearBranch`` ``:237-607``, ``projected_delta``
``:545-607``) and ``LinearBranch.readout`` (``vdn_h3/branch.py:672-722``): same arguments, the
same anchor-frame handling (``skip_ends`` slices frames 0 and F-1 off before any branch work
and leaves their rows zero), the text state (``vdn_h3/branch.py:649-670``) and the projector
hook. The inference spelling only: the device path runs under ``torch.no_grad()``.

Per call, on the caller's current stream:
  beta (GEMM + sigmoid) -> [short convolutions of the short_conv targets] -> frame statistics
  (features fused) -> frame means -> alpha
  -> text state (statistics + factor, J scaled by 1/2) -> factor of every frame
  -> bidirectional scans -> output gate (two GEMMs + sigmoid)
  -> gather + readout + RMSNorm epilogue -> projector (bf16 / fp8 / int8 GEMM).
"""

from __future__ import annotations

from typing import Mapping

import torch

from . import branch as _b
from . import linear as _linear
from . import projection as _projection


def _row_span(first: torch.Tensor | None, second: torch.Tensor):
    """``(view, gap)``: the rows from ``first[0]`` through ``second[-1]`` as one view, with ``second``
    starting ``gap`` rows in, when both are row slices of one row-major matrix and the rows between
    them add at most a quarter to the total; otherwise ``None``."""
    if first is None or first.ndim != 2 or second.ndim != 2 or first.shape[1] != second.shape[1]:
        return None
    if first.stride() != second.stride() or first.stride(1) != 1 or first.dtype != second.dtype:
        return None
    if first.untyped_storage().data_ptr() != second.untyped_storage().data_ptr():
        return None
    row = first.stride(0)
    off = second.storage_offset() - first.storage_offset()
    if row <= 0 or off % row or off // row < first.shape[0]:
        return None
    gap = off // row
    total = gap + second.shape[0]
    if total * 4 > 5 * (first.shape[0] + second.shape[0]):
        return None
    return first.as_strided((total, first.shape[1]), first.stride()), gap


class OptimizedLinearBranch:
    """One block's VDN branch (weights are passed per call, as in the reference)."""

    def __init__(self, weights: Mapping[str, torch.Tensor] | None, num_heads: int, head_dim: int,
                 delta_rule: str = "vdn_solve", bridge: str = "alpha", a_fp32: bool = True, short_conv=(),
                 enable_text_state: bool = True, **_runtime):
        if delta_rule not in _b.DELTA_BACKENDS:
            raise ValueError(f"unknown delta rule: {delta_rule!r}")
        if bridge not in ("alpha", "none"):
            raise ValueError("bridge must be 'alpha' or 'none'")
        targets = tuple(short_conv)
        if len(set(targets)) != len(targets) or any(t not in ("q", "k", "v") for t in targets):
            raise ValueError("short_conv must be a distinct subset of ('q', 'k', 'v')")
        self.w = weights
        self.num_heads = int(num_heads)
        self.head_dim = int(head_dim)
        self.delta_rule = delta_rule
        self.bridge = bridge
        self.a_fp32 = bool(a_fp32)
        self.short_conv = targets
        self.enable_text_state = bool(enable_text_state)

    def _backend(self, tokens):
        return _b.DELTA_BACKENDS[self.delta_rule](tokens)

    def _text_state(self, weights, text_x, text_k_raw, text_v_raw, beta=None):
        if not self.enable_text_state or text_x is None:
            return None
        if text_k_raw is None or text_v_raw is None:
            raise ValueError("text state needs both raw text key and value")
        length = text_x.shape[0]
        if length <= 0 or text_k_raw.shape[0] != length or text_v_raw.shape[0] != length:
            raise ValueError("text tensors must share a positive sequence length")
        if beta is None:
            beta = _linear.sigmoid_linear(text_x, weights["beta_proj.weight"])
        a, b = _b.frame_statistics_raw(text_k_raw, text_v_raw, beta, 1, length, a_fp32=self.a_fp32)
        _, jay = self._backend(length).factor_apply(None, a, b, jay_scale=_b.TEXT_STATE_SCALE, need_phi=False)
        return jay[0]

    def _beta_down_weight(self, weights):
        """``[W_beta; W_down]`` (``[heads + rank, hidden]`` bf16), rebuilt when either weight changes."""
        wb, wd = weights["beta_proj.weight"], weights["output_gate.down.weight"]
        key = (wb.data_ptr(), wb._version, tuple(wb.shape), wd.data_ptr(), wd._version, tuple(wd.shape))
        cached = getattr(self, "_beta_down", None)
        if cached is None or cached[0] != key:
            cached = (key, torch.cat([wb, wd], dim=0).contiguous())
            self._beta_down = cached
        return cached[1]

    def _features(self, weights, name, raw, num_frames, frame_size):
        """Short-convolution features of ``q``/``k``/``v`` (``vdn_h3/runtime.py:311-341``), or the raw
        rows when ``name`` has no short convolution (its feature map is fused into the consumer)."""
        if name not in self.short_conv:
            return raw, False
        if frame_size is None:
            raise ValueError("short convolution requires frame_size")
        feats = _b.conv_features(raw, weights[f"short_conv.{name}_sp.weight"], weights[f"short_conv.{name}_tm.weight"],
                                 num_frames, frame_size, name != "v")
        return feats, True

    def _readout_flat(self, weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds, text_x,
                      text_k_raw, text_v_raw, frame_size=None, out=None, proj_rows=None, text_proj_rows=None):
        heads, dim = self.num_heads, self.head_dim
        # beta = sigmoid(x W_beta^T) and the output-gate down-projection x W_down^T read the same rows:
        # one GEMM over [W_beta; W_down] with the sigmoid on the first `heads` columns (or rows the
        # caller computed with a wider GEMM over the same x)
        span = _row_span(text_x, xv) if self.enable_text_state and proj_rows is None else None
        if proj_rows is not None:
            both = proj_rows
            text_beta = None if text_proj_rows is None else text_proj_rows[:, :heads]
        elif span is None:
            both = _linear.sigmoid_linear_split(xv, self._beta_down_weight(weights), heads)
            text_beta = None
        else:  # text rows and video rows are row slices of one matrix: one launch covers both
            rows_view, gap = span
            both = _linear.sigmoid_linear_split(rows_view, self._beta_down_weight(weights), heads)
            text_beta = both[:text_x.shape[0], :heads]
            both = both[gap:]
        beta, gate_hidden = both[:, :heads], both[:, heads:]
        if "k" in self.short_conv and "v" in self.short_conv and frame_size is not None:
            # both convolutions in one launch (their workgroups share the launch's rounds)
            k_in, v_in = _b.conv_features_batch(
                [(k_raw, weights["short_conv.k_sp.weight"], weights["short_conv.k_tm.weight"], True, None),
                 (v_raw, weights["short_conv.v_sp.weight"], weights["short_conv.v_tm.weight"], False, None)],
                num_frames, frame_size)
            k_feat = v_feat = True
        else:
            k_in, k_feat = self._features(weights, "k", k_raw, num_frames, frame_size)
            v_in, v_feat = self._features(weights, "v", v_raw, num_frames, frame_size)
        a, b = _b.frame_statistics_raw(k_in, v_in, beta, num_frames, tokens_per_frame, k_features=k_feat,
                                       v_features=v_feat, a_fp32=self.a_fp32)
        del k_in, v_in
        mean = _b.frame_mean(xv, num_frames, tokens_per_frame)
        alpha = _b.alpha_gate(mean, weights["alpha.down.weight"], weights["alpha.up.weight"],
                              weights["alpha.dt_bias"], weights["alpha.A_log"], heads, dim)
        text_state = self._text_state(weights, text_x, text_k_raw, text_v_raw, text_beta)
        prefix, suffix = _b.run_scans_inference(self._backend(tokens_per_frame), alpha, a, b, text_state)
        del a, b
        q_in, q_feat = self._features(weights, "q", q_raw, num_frames, frame_size)
        # the output gate's up-projection and sigmoid run inside the readout kernel
        return _b.readout_epilogue(q_in, prefix, suffix, alpha, bounds, weights["norm.weight"], None,
                                   text_state=text_state, bridge=self.bridge, num_frames=num_frames,
                                   tokens_per_frame=tokens_per_frame, out=out, q_features=q_feat,
                                   gate_hidden=gate_hidden, gate_up_weight=weights["output_gate.up.weight"],
                                   gate_up_bias=weights.get("output_gate.up.bias"))

    def _check(self, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds):
        if torch.is_grad_enabled():
            raise RuntimeError("VDN-H3 inference linear branch requires no_grad/inference_mode")
        rows = num_frames * tokens_per_frame
        if xv.ndim != 2 or xv.shape[0] != rows:
            raise ValueError("xv rows must equal num_frames * tokens_per_frame")
        expected = (rows, self.num_heads, self.head_dim)
        if q_raw.shape != expected or k_raw.shape != expected or v_raw.shape != expected:
            raise ValueError("raw q/k/v have incompatible video row/head geometry")
        if len(bounds) != num_frames:
            raise ValueError("bounds must contain one entry per frame")

    def readout(self, weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds, frame_size=None,
                text_x=None, text_k_raw=None, text_v_raw=None, skip_ends=False, *, inference=True):
        """Branch readout before ``to_out_linear``: ``[F*T, H*D]`` bf16, anchor rows zero with ``skip_ends``."""
        del inference
        self._check(xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds)
        rows = num_frames * tokens_per_frame
        if not skip_ends:
            return self._readout_flat(weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds,
                                      text_x, text_k_raw, text_v_raw, frame_size)
        out = torch.empty((rows, self.num_heads * self.head_dim), dtype=torch.bfloat16, device=xv.device)
        if num_frames <= 2:
            return _b.fill_rows(out)
        t = tokens_per_frame
        inner = slice(t, (num_frames - 1) * t)
        _b.fill_rows(out[:t])
        _b.fill_rows(out[(num_frames - 1) * t:])
        self._readout_flat(weights, xv[inner], q_raw[inner], k_raw[inner], v_raw[inner], num_frames - 2, t,
                           [(lo - 1, hi - 1) for lo, hi in bounds[1:-1]], text_x, text_k_raw, text_v_raw,
                           frame_size, out=out[inner])
        return out

    def projected_delta(self, weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds, *,
                        frame_size=None, text_x=None, text_k_raw=None, text_v_raw=None, skip_ends=False,
                        inference=True, projector=None, tile_frames=None, out=None, accumulate=False,
                        proj_rows=None, text_proj_rows=None):
        """Branch output after ``to_out_linear``, ``[F*T, hidden]`` bf16, anchor rows zero.

        ``out``/``accumulate``: write (or add, ``out += delta``) straight into an existing
        ``[F*T, hidden]`` bf16 view, e.g. the video rows of the block output; with
        ``accumulate`` the anchor rows of ``out`` are left untouched (their delta is zero).
        ``projector(rows, out=..., accumulate=...)`` defaults to ``projection.project``.
        ``proj_rows`` / ``text_proj_rows`` (optional, ``[rows, heads + rank]`` bf16): ``[beta | x W_down^T]``
        of the rows of ``xv`` / ``text_x``, already computed by the caller (the block computes them in the
        softmax gate's GEMM); without them the branch computes them itself.
        """
        del inference, tile_frames
        self._check(xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds)
        proj = projector or (lambda rows, **kw: _projection.project(rows, weights, **kw))
        hidden = _projection.projection_out_features(weights)
        original_rows = num_frames * tokens_per_frame
        if out is None:
            if accumulate:
                raise ValueError("accumulate needs an existing output")
            out = torch.empty((original_rows, hidden), dtype=torch.bfloat16, device=xv.device)
        elif out.shape != (original_rows, hidden):
            raise ValueError(f"out must be [{original_rows}, {hidden}]")
        flat, rows = self.branch_rows(weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds,
                                      frame_size=frame_size, text_x=text_x, text_k_raw=text_k_raw,
                                      text_v_raw=text_v_raw, skip_ends=skip_ends, proj_rows=proj_rows,
                                      text_proj_rows=text_proj_rows)
        if flat is None:
            return out if accumulate else _b.fill_rows(out)
        if not accumulate and rows != slice(0, original_rows):
            _b.fill_rows(out[:rows.start])
            _b.fill_rows(out[rows.stop:])
        proj(flat, out=out[rows], accumulate=accumulate)
        return out

    def branch_rows(self, weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds, *,
                    frame_size=None, text_x=None, text_k_raw=None, text_v_raw=None, skip_ends=False,
                    proj_rows=None, text_proj_rows=None):
        """``(rows, sl)``: the branch's gated readout ``[n, heads * head_dim]`` bf16, the input of
        ``to_out_linear``, and the slice of ``xv``'s rows it belongs to; ``(None, None)`` when no row
        carries a delta (``skip_ends`` with at most two frames). ``projected_delta`` is
        ``to_out_linear`` of these rows, with zero rows elsewhere; the block's parallel branch execution
        computes them on a second stream and projects them after the attention."""
        self._check(xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds)
        t = tokens_per_frame
        if skip_ends:
            if num_frames <= 2:
                return None, None
            inner = slice(t, (num_frames - 1) * t)
            flat = self._readout_flat(weights, xv[inner], q_raw[inner], k_raw[inner], v_raw[inner],
                                      num_frames - 2, t, [(lo - 1, hi - 1) for lo, hi in bounds[1:-1]], text_x,
                                      text_k_raw, text_v_raw, frame_size,
                                      proj_rows=None if proj_rows is None else proj_rows[inner],
                                      text_proj_rows=text_proj_rows)
            return flat, inner
        flat = self._readout_flat(weights, xv, q_raw, k_raw, v_raw, num_frames, t, bounds, text_x, text_k_raw,
                                  text_v_raw, frame_size, proj_rows=proj_rows, text_proj_rows=text_proj_rows)
        return flat, slice(0, num_frames * t)


__all__ = ["OptimizedLinearBranch"]
