"""Oracle: one VDN-H3 hybrid attention block (the patched ``attn.forward``) on the CPU.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates the inference spelling of ``make_vdn_forward.vdn_forward``
(``vdn_h3/hybrid.py:409-579``):

* ``qkv``             -> ``_qkv`` (``vdn_h3/hybrid.py:260-268``): one projection, split into
  ``[S, H, D]`` views of the raw q / k / v;
* ``rms_norm_bf16``   -> ``attn.q_norm`` / ``attn.k_norm`` (``vdn_h3/hybrid.py:271-273``): an
  ``F.rms_norm`` over the head dim, fp32 statistics, ``x * rsqrt(mean x^2 + eps) * w`` rounded once;
* ``rms_rope_split_half`` -> the same with RoPE (``vdn_h3/hybrid.py:274-292``) when ``rope_freqs``
  is given (parity unpinned: the comfy-kitchen op is absent);
* the branch          -> ``oracle.branch_oracle.projected_delta`` on the *raw* video rows, with
  ``skip_ends = (anchor_frames == "both")`` and the text rows as text state (``:443-477``);
* attention           -> ``oracle.window_oracle.window_attention_grouped`` on the normalised
  q / k (``:494-505``); a full-cover layout runs dense attention and skips the branch
  (``:422``, ``:495-499``);
* softmax gate        -> ``sigmoid(F.linear(x, W_g, b_g))`` per head, ``bf16(O * g)``
  (``:518-529``, ``vdn_h3/softmax_kernels.py:8-9``);
* ``out = out_proj(flat)``; ``out[video] += delta`` in bf16 (``:534-540``).

``project`` is any callable ``rows -> rows @ W^T`` (bf16 ``F.linear`` by default, or the
W8A8 oracle of ``oracle.quant_oracle``).

Pinning (``tests/test_oracle_hybrid.py``): the composite against the golden vector
``tests/golden/hybrid_13f.safetensors`` written by the reference's own ``make_vdn_forward``
(13 frames of 8x8, 16 text rows, 2 heads x 64, anchors both, text state, gate on);
``rms_norm_bf16`` against ``torch.nn.functional.rms_norm``; the full-cover branch skip and
the gate = 0 halving against closed forms (``tests/test_hybrid.py:107-189``).
"""

from __future__ import annotations

import torch

from . import branch_oracle as bo
from . import window_oracle as wo


def rms_norm_bf16(x, weight, eps=1e-6):
    """``F.rms_norm`` over the last dim of a bf16 tensor: fp32 statistics, one rounding."""
    xf = x.float()
    r = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (xf * r * weight.float()).to(x.dtype)


def rms_rope_split_half(x, weight, eps, freqs, rot_dim, rounded=True):
    """RMSNorm + split-half rotary embedding (``vdn_h3/hybrid.py:274-292``, the fused comfy-kitchen op).

    ``y = x * rsqrt(mean x^2 + eps) * w`` in fp32; for ``i < rot_dim / 2`` the pair
    ``(y_i, y_{i + rot_dim/2})`` becomes ``F (y_i, y_{i + rot_dim/2})`` with ``F = freqs[row, i]``
    (``[rows or 1, rot_dim/2, 2, 2]``); channels ``>= rot_dim`` pass; one bf16 rounding unless
    ``rounded`` is false. PARITY UNPINNED against comfy-kitchen (absent, version unpinned): pinned
    by closed forms only (identity, quarter turn, inverse rotation, per-pair norm).
    """
    xf = x.float()
    y = xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps) * weight.float()
    half = rot_dim // 2
    f = freqs.float().reshape(-1, 1, half, 2, 2)                  # [rows or 1, 1 (heads), half, 2, 2]
    a, b = y[..., :half], y[..., half:rot_dim]
    out = y.clone()
    out[..., :half] = f[..., 0, 0] * a + f[..., 0, 1] * b
    out[..., half:rot_dim] = f[..., 1, 0] * a + f[..., 1, 1] * b
    return out.to(x.dtype) if rounded else out


def qkv(x, weight, heads, head_dim, project=None):
    """``_qkv``: the fused projection split into three ``[S, H, D]`` tensors."""
    projected = project(x) if project is not None else bo.linear_bf16(x, weight)
    inner = heads * head_dim
    seq = x.shape[0]
    q, k, v = projected.split(inner, dim=-1)
    return q.reshape(seq, heads, head_dim), k.reshape(seq, heads, head_dim), v.reshape(seq, heads, head_dim)


def vdn_forward(x, layout, attn_weights, branch_weights, heads, head_dim, *, eps=1e-6, gate_enabled=True,
                linear_enabled=True, text_state=True, project_qkv=None, project_out=None, branch_projector=None,
                return_parts=False, rope_freqs=None, short_conv=()):
    """Block output ``[S, hidden]`` bf16 for ``x`` ``[S, hidden]`` bf16 and a ``VDNLayout``-like ``layout``.

    ``attn_weights``: ``qkv_proj.weight``, ``out_proj.weight``, ``q_norm.weight``, ``k_norm.weight``.
    """
    q_raw, k_raw, v_raw = qkv(x, attn_weights["qkv_proj.weight"], heads, head_dim, project_qkv)
    linear_active = linear_enabled and not layout.full_cover
    va, vb = layout.video_start, layout.video_end
    ta, tb = layout.text_start, layout.text_start + layout.text_len
    delta = None
    if linear_active:
        kw = {}
        if text_state:
            kw = dict(text_x=x[ta:tb], text_k_raw=k_raw[ta:tb], text_v_raw=v_raw[ta:tb])
        delta = bo.projected_delta(branch_weights, x[va:vb], q_raw[va:vb], k_raw[va:vb], v_raw[va:vb],
                                   layout.num_frames, layout.tokens_per_frame, list(layout.bounds),
                                   frame_size=layout.frame_size, skip_ends=layout.anchor_frames == "both",
                                   projector=branch_projector, short_conv=short_conv, fused_conv=True, **kw)
    if rope_freqs is None:
        query = rms_norm_bf16(q_raw, attn_weights["q_norm.weight"], eps)
        key = rms_norm_bf16(k_raw, attn_weights["k_norm.weight"], eps)
    else:
        rot = 2 * int(rope_freqs.shape[-3])
        query = rms_rope_split_half(q_raw, attn_weights["q_norm.weight"], eps, rope_freqs, rot)
        key = rms_rope_split_half(k_raw, attn_weights["k_norm.weight"], eps, rope_freqs, rot)
    scale = head_dim ** -0.5
    if layout.full_cover:
        soft = wo.window_attention_grouped(query, key, v_raw, 0, x.shape[0], 1, x.shape[0], [(0, 0)], scale, "none")
    else:
        soft = wo.window_attention_grouped(query, key, v_raw, va, vb, layout.num_frames, layout.tokens_per_frame,
                                           list(layout.bounds), scale, layout.anchor_frames)
    soft = soft.to(x.dtype)
    seq = x.shape[0]
    if gate_enabled:
        gate = torch.sigmoid(bo.linear_bf16(x, branch_weights["softmax_gate.up.weight"],
                                            branch_weights.get("softmax_gate.up.bias")))
        flat = (soft * gate.reshape(seq, heads, 1).to(soft.dtype)).reshape(seq, heads * head_dim)
    else:
        gate = None
        flat = soft.reshape(seq, heads * head_dim)
    out = project_out(flat) if project_out is not None else bo.linear_bf16(flat, attn_weights["out_proj.weight"])
    if delta is not None:
        out[va:vb] = out[va:vb] + delta
    if return_parts:
        return out, dict(q_raw=q_raw, k_raw=k_raw, v_raw=v_raw, query=query, key=key, softmax=soft, gate=gate,
                         flat=flat, delta=delta)
    return out
