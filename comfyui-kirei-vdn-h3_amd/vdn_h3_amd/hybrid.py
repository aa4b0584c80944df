"""The VDN-H3 hybrid attention block on MI355X: the patched ``attn.forward``.

Mirrors ``vdn_h3/hybrid.py``: ``VDNState`` (``:33-213``), ``make_vdn_forward``
(``:409-579``) and ``apply_vdn`` (``:606-641``), with the same call signature
``vdn_forward(x, rope_freqs=None, transformer_options=None) -> [S, hidden]``, the same
layout contract (the request-local ``VDNLayout``; without one the original forward runs)
and the same exception types. Per call, on the caller's current stream:

  qkv = attn.qkv_proj(x)                         raw q / k / v views [S, H, D]
  g = sigmoid(x W_g^T + b_g)                     [S, H], GEMM with a sigmoid epilogue
  k' = k_norm(k_raw) [+ RoPE], V^T copy          one HIP pre-pass into the attention workspace
       [with RoPE also q' = q_norm(q_raw) + RoPE]
  flat = bf16(window_attention(q', k', v) * g)   one HIP kernel, the gate in its epilogue; without
                                                 RoPE it normalises q_raw as it loads it
  out = attn.out_proj(flat)
  out[video] += to_out_linear(branch(x, q_raw, k_raw, v))   GEMM epilogue accumulates into out

The branch runs after ``out_proj`` here (the reference computes it first and adds it last):
the sum is the same bf16 addition, ``bf16(out + bf16(delta))``. A full-cover layout runs
dense attention and no branch (``:422``, ``:495-499``). The path is forward-only: with
gradient mode on (the reference's deferred-branch case, ``:424``, ``:481-495``) a call whose input,
rotary table and block weights need no gradient runs the same forward under ``torch.no_grad``, and
one where any of them requires grad is a ``RuntimeError``. With ``rope_freqs`` the q/k pass also applies the
split-half rotary embedding (``vdn_h3/hybrid.py:274-292``; ``rope_table`` gives the layout),
with the q_norm epsilon for both, as the reference does. ``normalise_qk`` is the same q/k pass as a
standalone op (the fused path gives the same bits).
"""

from __future__ import annotations

import logging
from collections.abc import Mapping, Sequence
from contextlib import contextmanager
from typing import Any

import torch

from . import _lib
from . import linear as _linear
from . import projection as _projection
from . import window as _window
from .branch import cholesky_runtime_scope
from .diagnostics import DiagnosticsRecorder
from .layout import current_layout, publish_layout
from .window import rope_table

_LOG = logging.getLogger("vdn_h3_amd")
_STATE_PATCH = "diffusion_model._vdn_h3_state"


def _branch_weights(index: int, branch: Any) -> Mapping:
    """The weight mapping a branch carries: the branch itself when it is a mapping, else its ``.w``."""
    if branch is None:
        raise ValueError(f"block {index} has no branch (None)")
    source = branch if isinstance(branch, Mapping) else getattr(branch, "w", None)
    if isinstance(source, Mapping):
        return source
    raise TypeError(f"the branch of block {index} ({type(branch).__name__}) carries no weight mapping in .w")


def _block_weight_maps(branches: Sequence[Any], weight_maps) -> list:
    """One weight mapping per block: the given ``weight_maps`` (one per branch), or each branch's own."""
    if weight_maps is None:
        return [_branch_weights(i, b) for i, b in enumerate(branches)]
    maps = list(weight_maps)
    if len(maps) == len(branches):
        return maps
    raise ValueError(f"{len(maps)} weight maps were given for {len(branches)} branches")


# How the VDN branch runs beside the window attention (vdn_h3/nodes.py:26): "serial" on the caller's
# stream after the attention, "parallel" on a second stream of the same device from the qkv projection
# on, joined at the to_out_linear accumulation.
BRANCH_EXECUTION_MODES = ("serial", "parallel")


class VDNState:
    """Runtime state of one patched model: config, per-block branches and weights, plan cache."""

    def __init__(self, name: str, config: Mapping[str, Any], branches: Sequence[Any], num_heads: int,
                 head_dim: int, *, attention_backend: str = "hip", weight_maps=None, inference: bool = True,
                 projection_precision: str = "bf16", projection_info: Any = None, diagnostics: bool = False,
                 block_fusion: bool = False, branch_execution: str = "serial", tile_frames: int = 0, **_runtime):
        if attention_backend not in _window.ATTENTION_BACKENDS:
            raise ValueError(f"unsupported attention backend {attention_backend!r}")
        if projection_precision not in _projection.PROJECTION_PRECISIONS:
            raise ValueError(f"unsupported projection precision {projection_precision!r}")
        if branch_execution not in BRANCH_EXECUTION_MODES:
            raise ValueError(f"unknown branch execution mode {branch_execution!r}")
        self.name = str(name)
        self.config = dict(config)
        self.cfg = self.config
        self.num_heads = int(num_heads)
        self.head_dim = int(head_dim)
        self.attention_backend = attention_backend
        self.inference = bool(inference)
        self.projection_precision = projection_precision
        self.projection_info = projection_info
        self.branches = list(branches)
        self.window_cache = _window.WindowAttentionCache(limit=24)
        self.forwards = 0
        self.last_attention_backend = None
        self.last_layout = None
        self.branch_execution = branch_execution
        self._branch_streams: dict[Any, torch.cuda.Stream] = {}
        self.diagnostics = DiagnosticsRecorder(diagnostics)
        self.block_fusion = bool(block_fusion)
        self._maps = _block_weight_maps(self.branches, weight_maps)
        self._resident: dict[tuple[int, Any], dict[str, torch.Tensor]] = {}
        # frame tiling of the branch (vdn_h3/hybrid.py:86, :136-148): handed to every branch that takes it
        if isinstance(tile_frames, bool) or int(tile_frames) < 0:
            raise ValueError("tile_frames must be a non-negative integer")
        self.tile_frames = int(tile_frames)
        for branch in self.branches:
            set_runtime = getattr(branch, "set_runtime", None)
            if set_runtime is not None:
                set_runtime(tile_frames=self.tile_frames)

    # Weights are resident in HBM (a block's branch weights are ~55 MB at hidden 5120; all
    # 50 blocks fit many times over in 288 GB), so prefetch / consume are bookkeeping only.
    def prefetch_weights(self, index, device, dtype, keys=None):
        del keys
        self.weights_on(index, device, dtype)

    def weights_on(self, index, device, dtype, keys=None):
        device = torch.device(device)
        key = (int(index), device)
        cached = self._resident.get(key)
        if cached is None:
            cached = {}
            for name, value in self._maps[index].items():
                if not isinstance(value, torch.Tensor):
                    cached[name] = value
                    continue
                keep_fp32 = name in ("alpha.A_log", "alpha.dt_bias") or value.dtype in (
                    torch.int8, torch.float8_e4m3fn) or name.endswith("weight_scale")
                cached[name] = value.to(device=device, dtype=value.dtype if keep_fp32 else dtype)
            self._resident[key] = cached
        if keys is None:
            return cached
        return {k: cached[k] for k in keys if k in cached}

    @property
    def weight_mode(self):
        return "resident"

    def mark_weights_consumed(self, index, device, dtype):
        del index, device, dtype

    def projection_view(self, weights):
        """Branch-visible weights plus the ``to_out_linear`` projector (``vdn_h3/hybrid.py:168-181``)."""
        if _projection.BF16_WEIGHT_KEY not in weights and _projection.FP8_WEIGHT_KEY not in weights:
            raise RuntimeError("VDN projection state contains neither BF16 nor quantized weight")
        return weights, lambda rows, **kw: _projection.project(rows, weights, **kw)

    def branch_stream(self, device) -> torch.cuda.Stream:
        """The stream of the parallel branch execution on ``device`` (default priority), one per device."""
        device = torch.device(device)
        stream = self._branch_streams.get(device)
        if stream is None:
            stream = self._branch_streams[device] = torch.cuda.Stream(device=device)
        return stream

    def release(self):
        for stream in self._branch_streams.values():
            stream.synchronize()
        self._branch_streams.clear()
        self._resident.clear()
        self.__dict__.pop("_gate_branch_cache", None)
        self.window_cache.release()
        if self.block_fusion:
            from .block_kernels import release_block_fusions

            release_block_fusions(self)
        return self

    close = release


def normalise_qk(q_raw: torch.Tensor, k_raw: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                 eps: float = 1e-6, rope_freqs: torch.Tensor | None = None,
                 k_eps: float | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``attn.q_norm(q), attn.k_norm(k)`` (RMSNorm over the head dim) into one new ``[S, 2, H, D]`` buffer.

    ``eps`` is q_norm's epsilon and ``k_eps`` k_norm's (``eps`` when ``None``). With ``rope_freqs``
    the normalised vectors are also rotated (split-half RoPE, the fused op of
    ``vdn_h3/hybrid.py:274-292``, which takes q_norm's epsilon for both), before their one rounding
    to bf16.
    """
    if q_raw.shape != k_raw.shape or q_raw.ndim != 3:
        raise ValueError("q and k must share shape [sequence, heads, dim]")
    _lib.forward_only("normalise_qk", q_raw, k_raw, q_weight, k_weight, rope_freqs)
    device = _lib.require_device(q_raw, k_raw, q_weight, k_weight)
    seq, heads, dim = q_raw.shape
    q_raw, k_raw = _window._kernel_operand(q_raw), _window._kernel_operand(k_raw)
    wq = q_weight.to(torch.bfloat16).contiguous()
    wk = k_weight.to(torch.bfloat16).contiguous()
    if wq.numel() != dim or wk.numel() != dim:
        raise ValueError(f"q/k norm weights must have {dim} entries")
    buf = torch.empty((seq, 2, heads, dim), dtype=torch.bfloat16, device=device)
    qn, kn = buf[:, 0], buf[:, 1]
    if rope_freqs is not None:
        table, row_stride, rot = rope_table(rope_freqs, seq, dim, device)
        rc = _lib.lib().vdnh3_qk_rmsnorm_rope(
            _lib.ptr(q_raw), q_raw.stride(0), q_raw.stride(1), _lib.ptr(k_raw), k_raw.stride(0), k_raw.stride(1),
            _lib.ptr(wq), _lib.ptr(wk), float(eps), _lib.ptr(table), row_stride, rot, _lib.ptr(qn), qn.stride(0),
            qn.stride(1), _lib.ptr(kn), kn.stride(0), kn.stride(1), seq, heads, dim, _lib.stream_handle(device))
        _lib.check(rc, "vdnh3_qk_rmsnorm_rope")
        return qn, kn
    rc = _lib.lib().vdnh3_qk_rmsnorm(_lib.ptr(q_raw), q_raw.stride(0), q_raw.stride(1), _lib.ptr(k_raw),
                                     k_raw.stride(0), k_raw.stride(1), _lib.ptr(wq), _lib.ptr(wk), float(eps),
                                     float(eps if k_eps is None else k_eps), _lib.ptr(qn), qn.stride(0), qn.stride(1), _lib.ptr(kn), kn.stride(0),
                                     kn.stride(1), seq, heads, dim, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_qk_rmsnorm")
    return qn, kn


def _norm_weight_eps(module, dim, device):
    weight = getattr(module, "weight", None)
    if weight is None:
        weight = torch.ones(dim, dtype=torch.bfloat16)
    eps = getattr(module, "eps", None)
    return weight.to(device), 1e-6 if eps is None else float(eps)


def _split_qkv(projected: torch.Tensor, heads: int, head_dim: int):
    """The raw q / k / v of a fused ``[S, 3*H*D]`` projection as ``[S, H, D]`` views (row stride
    ``3*H*D``, no copy); ``RuntimeError`` when the width is not ``3*H*D`` (``vdn_h3/hybrid.py:260-268``)."""
    width = int(projected.shape[-1])
    if width != 3 * heads * head_dim:
        raise RuntimeError(f"qkv_proj produced {width} features per token; this block needs "
                           f"3 x {heads} heads x {head_dim} = {3 * heads * head_dim}")
    return projected.unflatten(-1, (3, heads, head_dim)).unbind(-3)


def _needs_grad(x, rope_freqs, attn, weight_map: Mapping) -> bool:
    """Whether any tensor a block call reads requires grad: ``x``, the rotary table, the attention
    module's parameters (or, for a plain object, the weights of its projections and norms) and the
    block's branch / gate weights."""
    tensors = [x, rope_freqs, *weight_map.values()]
    params = getattr(attn, "parameters", None)
    if callable(params):
        tensors.extend(params())
    else:
        for name in ("qkv_proj", "out_proj", "q_norm", "k_norm"):
            tensors.append(getattr(getattr(attn, name, None), "weight", None))
    return any(isinstance(t, torch.Tensor) and t.requires_grad for t in tensors)


class _VDNBlockForward:
    """The patched ``attn.forward`` of one block (``vdn_h3/hybrid.py:409-579``).

    Same call signature and contract as the reference's ``vdn_forward``: without a published
    layout the original forward runs; a layout whose length differs from ``x`` is a
    ``RuntimeError``; the path is forward-only (a call in gradient mode runs under ``no_grad``
    when nothing it reads requires grad, else it is a ``RuntimeError``).
    """

    def __init__(self, attn: Any, state: VDNState, block_index: int):
        self.attn, self.state, self.index = attn, state, int(block_index)
        self.heads, self.head_dim = int(attn.heads), int(attn.head_dim)
        self.branch = state.branches[block_index]
        self._vdn_h3_forward = True
        self._vdn_h3_original = attn.forward

    def __call__(self, x, rope_freqs=None, transformer_options=None):
        layout = current_layout(required=False)
        if layout is None:
            return self._vdn_h3_original(x, rope_freqs=rope_freqs, transformer_options=transformer_options or {})
        rows = int(x.shape[0])
        if rows != layout.seq_len:
            raise RuntimeError(f"attention got {rows} rows but the published VDN layout has {layout.seq_len}")
        if torch.is_grad_enabled():
            if _needs_grad(x, rope_freqs, self.attn, self.state._maps[self.index]):
                raise RuntimeError("the MI355X VDN-H3 block is forward-only (no backward), and a tensor it reads "
                                   "requires grad; run it under torch.no_grad() or inference_mode()")
            with torch.no_grad():
                out = self._forward(x, layout, rope_freqs)
        else:
            out = self._forward(x, layout, rope_freqs)
        self.state.forwards += 1
        self.state.last_layout = layout
        return out

    def _gate(self, x, weights, with_branch: bool):
        """``(g, proj_rows)``: the softmax gate ``sigmoid(x W_g^T + b_g)`` ``[S, H]`` and, when the branch
        runs, ``[beta | x W_down^T]`` from the same GEMM over ``x``; ``(None, None)`` with the gate off."""
        if not bool(self.state.config.get("enable_softmax_gate", True)):
            return None, None
        try:
            fused = _gate_branch_weights(self.state, self.index, weights, self.branch) if with_branch else None
            if fused is None:
                gate = _linear.sigmoid_linear(x, weights["softmax_gate.up.weight"],
                                              weights.get("softmax_gate.up.bias"))
                return gate, None
        except KeyError as exc:
            raise RuntimeError(f"VDN branch block {self.index} is missing softmax gate tensor "
                               f"{exc.args[0]!r}") from exc
        # [softmax gate | branch beta] (sigmoid) and the output-gate down-projection: x is read once
        w_all, b_all = fused
        rows = _linear.gemm(_linear.KIND_BF16, x, w_all, bias=b_all, act="sigmoid", round_linear=True,
                            act_cols=2 * self.heads)
        return rows[:, :self.heads], rows[:, self.heads:]

    def _plan(self, layout, device):
        cache = self.state.window_cache
        if layout.full_cover:
            self.state.last_attention_backend = "dense_exact"
            return cache.plan(layout.seq_len, 0, layout.seq_len, 1, layout.seq_len, [(0, 0)], "none", device)
        self.state.last_attention_backend = _window.resolve_attention_backend(self.state.attention_backend,
                                                                              cache=cache)
        return cache.plan(layout.seq_len, layout.video_start, layout.video_end, layout.num_frames,
                          layout.tokens_per_frame, layout.bounds, layout.anchor_frames, device)

    def _forward(self, x, layout, rope_freqs):
        state, attn, heads, head_dim = self.state, self.attn, self.heads, self.head_dim
        device, scope = x.device, state.diagnostics.scope
        with_branch = bool(state.config.get("linear_enabled", True)) and not layout.full_cover
        weights = state.weights_on(self.index, device, x.dtype)
        with scope("attention.qkv", device):
            q_raw, k_raw, value = _split_qkv(attn.qkv_proj(x), heads, head_dim)
        (qw, q_eps), (kw, k_eps) = (_norm_weight_eps(m, head_dim, device) for m in (attn.q_norm, attn.k_norm))
        if rope_freqs is not None:
            k_eps = q_eps  # split-half RoPE takes q_norm's epsilon for both (vdn_h3/hybrid.py:284-291)
        with scope("attention.gate", device):
            gate, proj_rows = self._gate(x, weights, with_branch)
        plan = self._plan(layout, device)
        pending = None
        if (with_branch and state.branch_execution == "parallel" and hasattr(self.branch, "branch_rows")
                and not getattr(self.branch, "tile_frames", 0)):
            # the branch reads only x, the raw q / k / v and its projections, none of which the attention
            # below writes: it runs on a second stream and joins at the to_out_linear accumulation (a
            # frame-tiled branch, whose point is to hold one tile of rows, runs in order after out_proj)
            pending = self._start_branch(x, q_raw, k_raw, value, layout, weights, proj_rows)
        with scope("attention.softmax", device):
            # q_norm / k_norm (+ RoPE) run inside the attention: the keys in its pre-pass, each query
            # row as the kernel loads it; the branch reads the raw q / k
            attended = _window.window_softmax_normed(
                q_raw, k_raw, value, qw, kw, q_eps, k_eps, layout.video_start, layout.video_end,
                layout.num_frames, layout.tokens_per_frame, layout.bounds, head_dim ** -0.5, layout.anchor_frames,
                rope_freqs=rope_freqs, gate=gate, plan=plan,
                diagnostics=state.diagnostics if state.diagnostics.enabled else None)
        with scope("attention.out_proj", device):
            out = attn.out_proj(attended.view(layout.seq_len, heads * head_dim))
        del attended
        if pending is not None:
            self._finish_branch(out, layout, *pending)
        elif with_branch:
            self._add_branch(out, x, q_raw, k_raw, value, layout, weights, proj_rows)
        return out

    def _branch_args(self, x, q_raw, k_raw, value, layout, weights, proj_rows):
        video = slice(layout.video_start, layout.video_end)
        text = slice(layout.text_start, layout.text_start + layout.text_len)
        use_text = bool(getattr(self.branch, "enable_text_state",
                                self.state.config.get("enable_text_state", False)))
        branch_weights, projector = self.state.projection_view(weights)
        kwargs = dict(frame_size=layout.frame_size, text_x=x[text] if use_text else None,
                      text_k_raw=k_raw[text] if use_text else None, text_v_raw=value[text] if use_text else None,
                      skip_ends=(layout.anchor_frames == "both"))
        if proj_rows is not None:
            kwargs.update(proj_rows=proj_rows[video], text_proj_rows=proj_rows[text] if use_text else None)
        args = (branch_weights, x[video], q_raw[video], k_raw[video], value[video], layout.num_frames,
                layout.tokens_per_frame, layout.bounds)
        return args, kwargs, projector

    def _start_branch(self, x, q_raw, k_raw, value, layout, weights, proj_rows):
        """The branch up to its gated readout rows, on the state's branch stream (the reference's
        ``branch_execution="parallel"``, ``vdn_h3/parallel.py:79-247``). Returns what the join needs."""
        main = torch.cuda.current_stream(x.device)
        side = self.state.branch_stream(x.device)
        side.wait_stream(main)  # qkv, the gate GEMM's beta / down-projection rows
        args, kwargs, projector = self._branch_args(x, q_raw, k_raw, value, layout, weights, proj_rows)
        with torch.cuda.stream(side):
            with self.state.diagnostics.scope("attention.linear_branch", x.device):
                rows, sl = self.branch.branch_rows(*args, **kwargs)
            done = torch.cuda.Event()
            done.record(side)
        return rows, sl, projector, done

    def _finish_branch(self, out, layout, rows, sl, projector, done):
        """``out[video][sl] += to_out_linear(rows)`` on the caller's stream once the branch stream is done."""
        main = torch.cuda.current_stream(out.device)
        main.wait_event(done)
        if rows is None:
            return
        rows.record_stream(main)  # allocated on the branch stream, read here
        video = out[layout.video_start:layout.video_end]
        with self.state.diagnostics.scope("attention.branch_projection", out.device):
            projector(rows, out=video[sl], accumulate=True)

    def _add_branch(self, out, x, q_raw, k_raw, value, layout, weights, proj_rows):
        """``out[video] += to_out_linear(branch)``, accumulated by the projection GEMM's epilogue."""
        args, kwargs, projector = self._branch_args(x, q_raw, k_raw, value, layout, weights, proj_rows)
        with self.state.diagnostics.scope("attention.linear_branch", x.device):
            self.branch.projected_delta(*args, inference=True, projector=projector,
                                        out=out[layout.video_start:layout.video_end], accumulate=True, **kwargs)


def make_vdn_forward(attn: Any, state: VDNState, block_index: int):
    """The patched ``attn.forward`` of block ``block_index``."""
    return _VDNBlockForward(attn, state, block_index)


def _gate_branch_weights(state, block_index, weights, branch):
    """``([W_softmax_gate; W_beta; W_down], bias)`` for one GEMM over the block input, or ``None`` when the
    branch is not this library's ``OptimizedLinearBranch`` or a weight is missing. Cached per block and
    rebuilt when a weight changes."""
    from .runtime import OptimizedLinearBranch

    if not isinstance(branch, OptimizedLinearBranch):
        return None
    try:
        ws, wb, wd = (weights["softmax_gate.up.weight"], weights["beta_proj.weight"],
                      weights["output_gate.down.weight"])
    except KeyError:
        return None
    bs = weights.get("softmax_gate.up.bias")
    parts = [t for t in (ws, wb, wd, bs) if t is not None]
    if ws.dtype != torch.bfloat16 or wb.dtype != torch.bfloat16 or wd.dtype != torch.bfloat16:
        return None
    key = tuple((t.data_ptr(), t._version, tuple(t.shape)) for t in parts)
    cache = state.__dict__.setdefault("_gate_branch_cache", {})
    hit = cache.get(block_index)
    if hit is None or hit[0] != key:
        w_all = torch.cat([ws, wb, wd], dim=0).contiguous()
        b_all = torch.zeros(w_all.shape[0], dtype=torch.float32, device=ws.device)
        if bs is not None:
            b_all[:ws.shape[0]] = bs.float()
        hit = (key, (w_all, b_all))
        cache[block_index] = hit
    return hit[1]


@contextmanager
def forward_scope(layout):
    """What the reference's DIFFUSION_MODEL wrapper does per model call (``vdn_h3/hybrid.py:216-241``):
    publish the layout and validate every Cholesky status of the call once at its end."""
    with publish_layout(layout), cholesky_runtime_scope():
        yield layout


def apply_vdn(model_patcher: Any, state: VDNState):
    """Install ``make_vdn_forward`` on every block (``vdn_h3/hybrid.py:606-641``, object patches only).

    ``model_patcher`` needs ``get_model_object`` and ``add_object_patch``; the caller publishes
    the layout around each model call with ``forward_scope`` (the reference installs a ComfyUI
    DIFFUSION_MODEL wrapper for that).
    """
    dm = model_patcher.get_model_object("diffusion_model")
    blocks = dm.blocks
    if len(blocks) != len(state.branches):
        raise RuntimeError(f"VDN state has {len(state.branches)} blocks but the model has {len(blocks)}")
    model_patcher.add_object_patch(_STATE_PATCH, state)
    for index, block in enumerate(blocks):
        model_patcher.add_object_patch(f"diffusion_model.blocks.{index}.attn.forward",
                                       make_vdn_forward(block.attn, state, index))
    from .block_kernels import install_block_fusions

    install_block_fusions(model_patcher, state, blocks)
    return model_patcher


__all__ = ["VDNState", "apply_vdn", "forward_scope", "make_vdn_forward", "normalise_qk"]
