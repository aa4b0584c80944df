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
        self.tile_frames = 0

    def set_runtime(self, *, tile_frames: int = 0, **_ignored):
        """Runtime options a ``VDNState`` hands its branches (``vdn_h3/hybrid.py:136-148``): ``tile_frames``
        > 0 runs ``projected_delta`` in frame tiles of that many frames (the reference picks 5 on GPUs of at
        most 32 GB, ``vdn_h3/nodes.py:193-202``)."""
        if isinstance(tile_frames, bool) or int(tile_frames) < 0:
            raise ValueError("tile_frames must be a non-negative integer")
        self.tile_frames = int(tile_frames)

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

    def _gate_rows(self, weights, xv, text_x, proj_rows, text_proj_rows):
        """``(beta [rows, heads], gate_hidden [rows, rank], text_beta or None)`` of the video rows."""
        heads = self.num_heads
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
        return both[:, :heads], both[:, heads:], text_beta

    def _readout_flat(self, weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds, text_x,
                      text_k_raw, text_v_raw, frame_size=None, out=None, proj_rows=None, text_proj_rows=None):
        heads, dim = self.num_heads, self.head_dim
        beta, gate_hidden, text_beta = self._gate_rows(weights, xv, text_x, proj_rows, text_proj_rows)
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

    def _tile_features(self, weights, raws, start, stop, num_frames, tokens_per_frame, frame_size):
        """``{name: (rows, is_features)}`` for frames ``[start, stop)`` of each raw ``[F*T, H, D]`` tensor in
        ``raws``: names without a short convolution give their raw rows (the feature map is fused into the
        consumer); the others run the short convolution over the tile plus a halo of ``kt // 2`` frames on
        each side, the frames its temporal taps read, so the tile's rows are those of the untiled call
        (``vdn_h3/runtime.py:421-440``). Tensors with the same halo share one launch."""
        t = tokens_per_frame
        out = {n: (raw[start * t:stop * t], False) for n, raw in raws.items() if n not in self.short_conv}
        conv = [n for n in raws if n in self.short_conv]
        if not conv:
            return out
        if frame_size is None:
            raise ValueError("short convolution requires frame_size")
        groups = {}
        for n in conv:
            pad = int(weights[f"short_conv.{n}_tm.weight"].shape[-1]) // 2
            groups.setdefault((max(0, start - pad), min(num_frames, stop + pad)), []).append(n)
        for (hs, he), names in groups.items():
            items = [(raws[n][hs * t:he * t], weights[f"short_conv.{n}_sp.weight"],
                      weights[f"short_conv.{n}_tm.weight"], n != "v", None) for n in names]
            feats = _b.conv_features_batch(items, he - hs, frame_size)
            for n, f in zip(names, feats):
                out[n] = (f[(start - hs) * t:(stop - hs) * t], True)
        return out

    def _projected_tiled(self, weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds, text_x,
                         text_k_raw, text_v_raw, frame_size, tile, out, accumulate, proj, proj_rows=None,
                         text_proj_rows=None):
        """``to_out_linear`` of the branch readout into ``out`` (``[F*T, hidden]``), in frame tiles of ``tile``
        frames (``vdn_h3/runtime.py:442-543``): the k / v features and frame statistics one tile at a time,
        the recurrence over every frame, then the query features, gated readout and projection one tile at a
        time, so the feature and readout buffers hold one tile. Each frame's statistics and readout and each
        row's projection depend on that frame or row alone, so the result is the untiled one, bit for bit."""
        heads, dim, t = self.num_heads, self.head_dim, tokens_per_frame
        beta, gate_hidden, text_beta = self._gate_rows(weights, xv, text_x, proj_rows, text_proj_rows)
        a = torch.empty((num_frames, heads, dim, dim), dtype=torch.float32, device=xv.device)
        b = torch.empty_like(a)
        for start in range(0, num_frames, tile):
            stop = min(num_frames, start + tile)
            rows = slice(start * t, stop * t)
            feats = self._tile_features(weights, {"k": k_raw, "v": v_raw}, start, stop, num_frames, t, frame_size)
            (k_in, k_feat), (v_in, v_feat) = feats["k"], feats["v"]
            _b.frame_statistics_raw(k_in, v_in, beta[rows], stop - start, t, k_features=k_feat, v_features=v_feat,
                                    a_fp32=self.a_fp32, out=(a[start:stop], b[start:stop]))
            del feats, k_in, v_in
        mean = _b.frame_mean(xv, num_frames, t)
        alpha = _b.alpha_gate(mean, weights["alpha.down.weight"], weights["alpha.up.weight"],
                              weights["alpha.dt_bias"], weights["alpha.A_log"], heads, dim)
        text_state = self._text_state(weights, text_x, text_k_raw, text_v_raw, text_beta)
        prefix, suffix = _b.run_scans_inference(self._backend(t), alpha, a, b, text_state)
        del a, b
        for start in range(0, num_frames, tile):
            stop = min(num_frames, start + tile)
            rows = slice(start * t, stop * t)
            q_in, q_feat = self._tile_features(weights, {"q": q_raw}, start, stop, num_frames, t, frame_size)["q"]
            flat = _b.readout_epilogue(q_in, prefix, suffix, alpha, bounds, weights["norm.weight"], None,
                                       text_state=text_state, bridge=self.bridge, num_frames=num_frames,
                                       tokens_per_frame=t, q_features=q_feat, gate_hidden=gate_hidden[rows],
                                       gate_up_weight=weights["output_gate.up.weight"],
                                       gate_up_bias=weights.get("output_gate.up.bias"), frame_range=(start, stop))
            proj(flat, out=out[rows], accumulate=accumulate)
            del q_in, flat

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
        ``tile_frames`` (default: the branch's runtime option, 0 = untiled) > 0 runs the branch in frame tiles
        when ``inference`` (``vdn_h3/runtime.py:588-595``), with the same result.
        """
        tile = self.tile_frames if tile_frames is None else tile_frames
        if isinstance(tile, bool) or int(tile) < 0:
            raise ValueError("tile_frames must be a non-negative integer")
        tile = int(tile) if inference else 0
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
        if tile > 0:
            t = tokens_per_frame
            if skip_ends and num_frames <= 2:
                return out if accumulate else _b.fill_rows(out)
            rows = slice(t, (num_frames - 1) * t) if skip_ends else slice(0, original_rows)
            frames = num_frames - 2 if skip_ends else num_frames
            inner_bounds = [(lo - 1, hi - 1) for lo, hi in bounds[1:-1]] if skip_ends else list(bounds)
            if not accumulate and skip_ends:
                _b.fill_rows(out[:rows.start])
                _b.fill_rows(out[rows.stop:])
            self._projected_tiled(weights, xv[rows], q_raw[rows], k_raw[rows], v_raw[rows], frames, t, inner_bounds,
                                  text_x, text_k_raw, text_v_raw, frame_size, min(tile, frames), out[rows],
                                  accumulate, proj, None if proj_rows is None else proj_rows[rows], text_proj_rows)
            return out
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
