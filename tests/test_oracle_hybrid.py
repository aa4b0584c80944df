"""Pinning of the hybrid-block oracle (CPU): the reference's own ``make_vdn_forward`` output,
``F.rms_norm``, and the closed forms of ``tests/test_hybrid.py:107-189`` (full-cover layouts
skip the branch; a gate of zero removes the softmax path)."""

from __future__ import annotations

from pathlib import Path

import pytest
import torch
import torch.nn.functional as F
from safetensors import safe_open

from oracle import branch_oracle as bo
from oracle import hybrid_oracle as ho

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with safe_open(str(GOLDEN / name), "pt") as f:
        return {k: f.get_tensor(k) for k in f.keys()}, f.metadata()


def _golden_case():
    from vdn_h3_amd.layout import text_first_layout

    t, meta = _load("hybrid_13f.safetensors")
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    grid = tuple(map(int, meta["grid"].split("x")))
    layout = text_first_layout(text, frames, grid, radius=int(meta["radius"]), chunk=int(meta["chunk"]),
                               anchor_frames=meta["anchor_frames"])
    bw = {k[2:]: v for k, v in t.items() if k.startswith("w.")}
    aw = {k[5:]: v for k, v in t.items() if k.startswith("attn.")}
    return t, layout, aw, bw, heads, dim


def _parity(got, want, atol=2e-2, min_cos=0.9995):
    got, want = got.float().flatten(), want.float().flatten()
    err = (got - want).abs().max().item()
    cos = F.cosine_similarity(got.double(), want.double(), dim=0).item()
    assert err <= atol and cos >= min_cos, f"max abs {err:.3e}, cosine {cos:.7f}"
    return err, cos


def test_rms_norm_matches_torch():
    g = torch.Generator().manual_seed(0)
    x = (3 * torch.randn(500, 4, 128, generator=g)).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16)
    assert torch.equal(ho.rms_norm_bf16(x, w), F.rms_norm(x, (128,), w, 1e-6))


def test_block_matches_reference_golden():
    t, layout, aw, bw, heads, dim = _golden_case()
    assert not layout.full_cover
    torch.set_num_threads(4)
    out = ho.vdn_forward(t["x"], layout, aw, bw, heads, dim)
    err, _ = _parity(out, t["out"])
    # the golden ran bf16 attention (grouped SDPA); the oracle computes attention in fp32
    assert err <= 8e-3


def test_planted_mistake_fails_the_golden():
    """A dropped branch, a wrong gate sign or skipped q/k norms each break the golden match."""
    t, layout, aw, bw, heads, dim = _golden_case()
    variants = {
        "no branch": dict(linear_enabled=False),
        "no gate": dict(gate_enabled=False),
    }
    for name, kw in variants.items():
        out = ho.vdn_forward(t["x"], layout, aw, bw, heads, dim, **kw)
        with pytest.raises(AssertionError):
            _parity(out, t["out"])
    flipped = dict(bw)
    flipped["softmax_gate.up.bias"] = -bw["softmax_gate.up.bias"]
    with pytest.raises(AssertionError):
        _parity(ho.vdn_forward(t["x"], layout, aw, flipped, heads, dim), t["out"])
    ones = dict(aw)
    ones["q_norm.weight"] = torch.full_like(aw["q_norm.weight"], 2.0)
    with pytest.raises(AssertionError):
        _parity(ho.vdn_forward(t["x"], layout, ones, bw, heads, dim), t["out"])


def test_full_cover_skips_branch_and_runs_dense():
    """7 frames, chunk 5, radius 1 cover every frame: dense attention, no branch delta."""
    from vdn_h3_amd.layout import text_first_layout

    heads, dim, hidden = 2, 64, 128
    layout = text_first_layout(16, 7, (8, 8))
    assert layout.full_cover
    g = torch.Generator().manual_seed(3)
    x = torch.randn(layout.seq_len, hidden, generator=g).to(torch.bfloat16)
    aw = {"qkv_proj.weight": (0.1 * torch.randn(3 * heads * dim, hidden, generator=g)).to(torch.bfloat16),
          "out_proj.weight": (0.05 * torch.randn(hidden, heads * dim, generator=g)).to(torch.bfloat16),
          "q_norm.weight": torch.ones(dim, dtype=torch.bfloat16), "k_norm.weight": torch.ones(dim, dtype=torch.bfloat16)}
    bw = {"softmax_gate.up.weight": torch.zeros(heads, hidden, dtype=torch.bfloat16),
          "softmax_gate.up.bias": torch.zeros(heads, dtype=torch.bfloat16)}
    out, parts = ho.vdn_forward(x, layout, aw, bw, heads, dim, return_parts=True)
    assert parts["delta"] is None
    q, k, v = parts["query"].float(), parts["key"].float(), parts["v_raw"].float()
    dense = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                           scale=dim ** -0.5).transpose(0, 1)
    # gate = sigmoid(0) = 1/2 exactly: the flattened input of out_proj is bf16(O) / 2
    half = (dense.to(torch.bfloat16).float() * 0.5).to(torch.bfloat16)
    torch.testing.assert_close(parts["flat"].reshape(half.shape).float(), half.float(), atol=2 * 2.0 ** -8, rtol=0)
    torch.testing.assert_close(out.float(), bo.linear_bf16(parts["flat"], aw["out_proj.weight"]).float())


def _rope_case(rows, heads, dim, rot, seed):
    g = torch.Generator().manual_seed(seed)
    x = (2 * torch.randn(rows, heads, dim, generator=g)).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    theta = torch.randn(rows, rot // 2, generator=g) * 3
    c, s_ = torch.cos(theta), torch.sin(theta)
    freqs = torch.stack([torch.stack([c, -s_], -1), torch.stack([s_, c], -1)], -2)   # [rows, rot/2, 2, 2]
    return x, w, theta, freqs


@pytest.mark.parametrize("dim,rot", [(128, 128), (128, 64), (64, 32)])
def test_rms_rope_closed_forms(dim, rot):
    """The split-half RoPE restatement: identity, quarter turn, inverse rotation, per-pair norms."""
    rows, heads, half = 37, 3, rot // 2
    x, w, theta, freqs = _rope_case(rows, heads, dim, rot, 70 + dim + rot)
    plain = ho.rms_norm_bf16(x, w, 1e-6)
    eye = torch.eye(2).expand(rows, half, 2, 2)
    assert torch.equal(ho.rms_rope_split_half(x, w, 1e-6, eye, rot), plain)
    # a quarter turn maps (y_i, y_{i+h}) to (-y_{i+h}, y_i) exactly: pairing and matrix layout
    quarter = torch.tensor([[0.0, -1.0], [1.0, 0.0]]).expand(1, half, 2, 2)
    got = ho.rms_rope_split_half(x, w, 1e-6, quarter, rot)
    assert torch.equal(got[..., :half], -plain[..., half:rot])
    assert torch.equal(got[..., half:rot], plain[..., :half])
    assert torch.equal(got[..., rot:], plain[..., rot:])
    # rotating by theta then by -theta returns the normalised vector; pair norms are kept
    y = ho.rms_rope_split_half(x, w, 1e-6, freqs, rot, rounded=False)
    back_freqs = freqs.transpose(-1, -2)                                  # R(-theta) = R(theta)^T
    yplain = ho.rms_rope_split_half(x, w, 1e-6, eye, rot, rounded=False)
    a, b = y[..., :half], y[..., half:rot]
    fb = back_freqs.reshape(rows, 1, half, 2, 2)
    a0 = fb[..., 0, 0] * a + fb[..., 0, 1] * b
    b0 = fb[..., 1, 0] * a + fb[..., 1, 1] * b
    torch.testing.assert_close(a0, yplain[..., :half], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(b0, yplain[..., half:rot], atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(a * a + b * b, yplain[..., :half] ** 2 + yplain[..., half:rot] ** 2,
                               atol=1e-4, rtol=1e-5)
    # a planted mistake (interleaved pairs instead of split halves) fails the quarter-turn check
    yi = plain.float()
    inter = torch.stack([-yi[..., 1:rot:2], yi[..., 0:rot:2]], -1).reshape(rows, heads, rot).to(torch.bfloat16)
    assert not torch.equal(inter, got[..., :rot])
