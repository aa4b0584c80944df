"""Seeded synthetic inputs for the VDN-H3 hot-path workloads.

Every tensor k of a workload comes from its own ``torch.Generator`` seeded with
``SEED_BASE + k`` (a fixed, documented order), is drawn in fp32 and then cast, so the
device path and the CPU oracle see bit-identical operands (the oracle receives a host
copy of the same cast tensor).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from .layout import VDNLayout, text_first_layout

SEED_BASE = 20261201


def generator(k: int, device="cpu") -> torch.Generator:
    return torch.Generator(device=device).manual_seed(SEED_BASE + int(k))


def randn(shape, k: int, device="cpu", dtype=torch.float32, scale: float = 1.0) -> torch.Tensor:
    """``N(0, scale^2)`` drawn in fp32 from generator ``k`` on ``device``, then cast to ``dtype``."""
    x = torch.randn(shape, generator=generator(k, device), device=device, dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    return x.to(dtype)


@dataclass(frozen=True)
class WindowWorkload:
    """Local-window attention at a packed layout (text rows first, then video frames)."""

    name: str
    heads: int
    head_dim: int
    text_len: int
    num_frames: int
    frame_size: tuple[int, int]
    radius: int = 1
    chunk: int = 5
    anchor_frames: str = "both"

    @property
    def layout(self) -> VDNLayout:
        return text_first_layout(self.text_len, self.num_frames, self.frame_size, radius=self.radius,
                                 chunk=self.chunk, anchor_frames=self.anchor_frames)

    @property
    def scale(self) -> float:
        return self.head_dim ** -0.5


# Full-shape local-window attention: 40 heads x 128, 31 frames of 48x27 tokens + 512 text rows.
WINDOW_FULL = WindowWorkload("window_s40688_h40_d128", 40, 128, 512, 31, (48, 27))
# CPU-plumbing shape (full cover: every frame sees every frame) and its 13-frame variant.
WINDOW_SMALL = WindowWorkload("window_s464_h2_d64", 2, 64, 16, 7, (8, 8))
WINDOW_SMALL_13F = WindowWorkload("window_s848_h2_d64_13f", 2, 64, 16, 13, (8, 8))


def fused_qkv(seq: int, heads: int, head_dim: int, device="cpu", seed: int = 0, scale: float = 1.0) -> torch.Tensor:
    """``[S, 3*H*D]`` bf16 ~ N(0, scale^2): the layout of the block's fused q/k/v projection."""
    return randn((seq, 3 * heads * head_dim), seed, device=device, dtype=torch.bfloat16, scale=scale)


def split_qkv(qkv: torch.Tensor, heads: int, head_dim: int):
    """Strided ``[S, H, D]`` views of a fused ``[S, 3*H*D]`` buffer (row stride ``3*H*D``)."""
    inner = heads * head_dim
    seq = qkv.shape[0]
    q, k, v = qkv.split(inner, dim=-1)
    return q.view(seq, heads, head_dim), k.view(seq, heads, head_dim), v.view(seq, heads, head_dim)


def window_inputs(w: WindowWorkload, device="cpu", input_scale: float | None = None):
    """(qkv buffer, q, k, v views, layout, scale) for a window workload: q, k, v ~ N(0, 1) scaled by
    ``input_scale`` (default ``1/sqrt(head_dim)``, the window-attention benchmark's inputs)."""
    lay = w.layout
    scale = w.scale if input_scale is None else input_scale
    qkv = fused_qkv(lay.seq_len, w.heads, w.head_dim, device=device, seed=0, scale=scale)
    q, k, v = split_qkv(qkv, w.heads, w.head_dim)
    return qkv, q, k, v, lay, w.scale


def sigmoid_gate(seq: int, heads: int, device="cpu", seed: int = 10) -> torch.Tensor:
    """Per-head gate ``sigmoid(N(0,1))`` as bf16 ``[S, H]``."""
    return torch.sigmoid(randn((seq, heads), seed, device=device)).to(torch.bfloat16)


def softmax_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


def branch_weights(heads: int, head_dim: int, hidden: int, device="cpu", seed: int = 42,
                   short_conv=()) -> dict:
    """Random-init VDN branch weights of one block (shapes of ``vdn_h3/spec.py:471-486``).

    Matrices ~ N(0, 0.02); ``alpha.dt_bias`` / ``alpha.A_log`` ~ N(0, 0.5^2) kept in fp32 (the
    reference stores them in fp32); ``norm.weight`` = 1 + 0.1 N(0, 1); gate biases N(0, 0.5^2);
    for each ``short_conv`` target a depthwise 5x5 spatial filter ~ N(0, 0.2^2) and a 5-tap
    temporal filter ~ N(0, 0.4^2) per channel.
    """
    bf = torch.bfloat16
    conv = {}
    for i, name in enumerate(short_conv):
        conv[f"short_conv.{name}_sp.weight"] = randn((heads * head_dim, 1, 5, 5), seed + 12 + 2 * i, device, bf, 0.2)
        conv[f"short_conv.{name}_tm.weight"] = randn((heads * head_dim, 1, 5), seed + 13 + 2 * i, device, bf, 0.4)
    return {
        **conv,
        "beta_proj.weight": randn((heads, hidden), seed, device, bf, 0.02),
        "alpha.down.weight": randn((head_dim, hidden), seed + 1, device, bf, 0.02),
        "alpha.up.weight": randn((heads * head_dim, head_dim), seed + 2, device, bf, 0.02),
        "alpha.dt_bias": randn((heads * head_dim,), seed + 3, device, scale=0.5),
        "alpha.A_log": randn((heads,), seed + 4, device, scale=0.5),
        "output_gate.down.weight": randn((head_dim, hidden), seed + 5, device, bf, 0.02),
        "output_gate.up.weight": randn((heads * head_dim, head_dim), seed + 6, device, bf, 0.02),
        "output_gate.up.bias": randn((heads * head_dim,), seed + 7, device, bf, 0.5),
        "norm.weight": (1 + 0.1 * randn((head_dim,), seed + 8, device)).to(bf),
        "to_out_linear.weight": randn((hidden, heads * head_dim), seed + 9, device, bf, 0.02),
        "softmax_gate.up.weight": randn((heads, hidden), seed + 10, device, bf, 0.02),
        "softmax_gate.up.bias": randn((heads,), seed + 11, device, bf, 0.5),
    }


def attention_module(heads: int, head_dim: int, hidden: int, device, seed: int, precision: str = "int8"):
    """A random-init MiniMax-H3 attention stand-in with the attributes the patched forward reads
    (``heads``, ``head_dim``, ``qkv_proj``, ``out_proj``, ``q_norm``, ``k_norm``): W ~ N(0, 0.02) as
    ``HipLinear`` layers of ``precision``, RMSNorm weights 1 + 0.1 N(0, 1), eps 1e-6."""
    from types import SimpleNamespace

    from .linear import HipLinear

    bf = torch.bfloat16
    return SimpleNamespace(
        heads=heads, head_dim=head_dim, forward=None,
        qkv_proj=HipLinear(randn((3 * heads * head_dim, hidden), seed + 1, device, bf, 0.02), precision),
        out_proj=HipLinear(randn((hidden, heads * head_dim), seed + 2, device, bf, 0.02), precision),
        q_norm=SimpleNamespace(weight=(1 + 0.1 * randn((head_dim,), seed + 3, device)).to(bf), eps=1e-6),
        k_norm=SimpleNamespace(weight=(1 + 0.1 * randn((head_dim,), seed + 4, device)).to(bf), eps=1e-6))


def hybrid_stack(blocks: int, heads: int, head_dim: int, hidden: int, device, *, short_conv=("k", "v"),
                 precision: str = "int8", config=None, first_seed: int = 1000, branch_execution: str = "serial"):
    """``(state, forwards)``: ``blocks`` random-init VDN-H3 hybrid attention blocks (block i seeded from
    ``first_seed * (i + 1)``), branch and projections prepared for ``precision``, one ``VDNState``
    (``branch_execution`` "serial" or "parallel", the VDN branch on a second stream)."""
    from . import projection
    from .hybrid import VDNState, make_vdn_forward
    from .runtime import OptimizedLinearBranch

    attns, maps = [], []
    for i in range(blocks):
        seed = first_seed * (i + 1)
        attns.append(attention_module(heads, head_dim, hidden, device, seed, precision))
        (bw,), _ = projection.prepare_projection_maps(
            [branch_weights(heads, head_dim, hidden, device=device, seed=seed + 42, short_conv=short_conv)], device,
            precision)
        maps.append(bw)
    branches = [OptimizedLinearBranch(bw, heads, head_dim, short_conv=short_conv) for bw in maps]
    cfg = {"enable_softmax_gate": True, "linear_enabled": True, "enable_text_state": True}
    cfg.update(config or {})
    state = VDNState("hybrid-stack", cfg, branches, heads, head_dim, projection_precision=precision,
                     branch_execution=branch_execution)
    return state, [make_vdn_forward(attn, state, i) for i, attn in enumerate(attns)]


def rope_freqs(seq: int, head_dim: int, device="cpu", base: float = 10000.0) -> torch.Tensor:
    """Split-half RoPE matrices ``[1, seq, 1, head_dim / 2, 2, 2]`` (fp32) for row positions 0..seq-1:
    pair i of row r rotates by ``r * base^(-2i / head_dim)``, ``[[cos, -sin], [sin, cos]]`` -- the
    per-row table a DiT hands each block as ``rope_freqs`` (rot_dim = head_dim)."""
    half = head_dim // 2
    inv = base ** (-torch.arange(half, dtype=torch.float64) * 2.0 / head_dim)
    theta = torch.arange(seq, dtype=torch.float64)[:, None] * inv[None, :]
    c, s = torch.cos(theta), torch.sin(theta)
    m = torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2).to(torch.float32)
    return m.reshape(1, seq, 1, half, 2, 2).to(device)


def denoise_pass(forwards, x: torch.Tensor, steps: int, on_block=None, rope_freqs=None) -> torch.Tensor:
    """``steps`` passes of ``x <- x + block(rms_norm(x))`` over every block (a pre-norm residual, as H3's
    blocks normalise their input: random-init blocks fed the raw stream would grow it per block).
    ``on_block(step, index, block_input, block_output)`` sees every block call; ``rope_freqs`` is handed
    to every block."""
    hidden = x.shape[-1]
    for step in range(steps):
        for index, forward in enumerate(forwards):
            h = torch.nn.functional.rms_norm(x, (hidden,), eps=1e-6)
            y = forward(h, rope_freqs=rope_freqs)
            if on_block is not None:
                on_block(step, index, h, y)
            x = x + y
    return x
