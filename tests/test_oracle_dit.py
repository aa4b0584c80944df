"""Pins of the DiT block pointwise oracle (CPU)."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import dit_oracle as do


def _case(rows=40, hidden=64, n_mod=3, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = (2 * torch.randn(rows, hidden, generator=g)).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    scale = 0.3 * torch.randn(n_mod, hidden, generator=g)
    shift = 0.3 * torch.randn(n_mod, hidden, generator=g)
    idx = torch.randint(0, n_mod, (rows,), generator=g)
    return x, w, scale, shift, idx


def test_pre_special_cases():
    x, w, scale, shift, idx = _case()
    normed = F.rms_norm(x, (x.shape[-1],), w, 1e-6)
    zero = torch.zeros_like(scale)
    assert torch.equal(do.pre(x, w, 1e-6, zero, zero, idx), normed)
    # scale = -1 zeroes the normalised term exactly: the output is the (bf16) shift of the row's segment
    assert torch.equal(do.pre(x, w, 1e-6, -torch.ones_like(scale), shift, idx),
                       shift.index_select(0, idx).to(torch.bfloat16))
    # the segment selects rows of the tables: permuting the tables and the indices together is a no-op
    perm = torch.tensor([2, 0, 1])
    inv = torch.argsort(perm)
    assert torch.equal(do.pre(x, w, 1e-6, scale[perm], shift[perm], inv[idx]), do.pre(x, w, 1e-6, scale, shift, idx))


def test_post_and_swiglu_special_cases():
    x, _, scale, _, idx = _case(seed=1)
    b = torch.randn_like(x.float()).to(torch.bfloat16)
    assert torch.equal(do.post(x, torch.zeros_like(scale), idx, b), x)
    assert torch.equal(do.post(x, torch.ones_like(scale), idx, b), x + b)
    h = torch.randn(7, 32).to(torch.bfloat16)
    g0 = h.clone()
    g0[:, :16] = 0
    assert torch.equal(do.swiglu(g0), torch.zeros(7, 16, dtype=torch.bfloat16))
    big = h.clone()
    big[:, :16] = 64.0                                   # silu(64) = 64 in bf16
    assert torch.equal(do.swiglu(big), (64.0 * big[:, 16:].float()).to(torch.bfloat16))


def test_segment_indices_brute_force_and_errors():
    segs = [(0, 5, 2), (5, 9, torch.tensor([0, 1, 1, 0])), (9, 12, torch.tensor(1))]
    want = [2] * 5 + [0, 1, 1, 0] + [1] * 3
    assert do.segment_indices(segs, 12).tolist() == want
    with pytest.raises(ValueError, match="contiguously"):
        do.segment_indices([(0, 5, 0), (6, 12, 1)], 12)
    with pytest.raises(ValueError, match="cover"):
        do.segment_indices([(0, 5, 0)], 12)


def _dit_golden():
    from pathlib import Path

    from safetensors import safe_open

    path = Path(__file__).resolve().parent / "golden" / "dit_block.safetensors"
    with safe_open(str(path), "pt") as f:
        return {k: f.get_tensor(k) for k in f.keys()}, f.metadata()


def _dit_oracle(t, mod_order=None, norms=("w.norm1.weight", "w.norm2.weight")):
    from oracle import branch_oracle as bo

    names = ("shift_msa", "scale_msa", "gate_msa", "shift_mlp", "scale_mlp", "gate_mlp")
    mod = tuple(t[f"mod.{n}"] for n in (mod_order or names))
    segments = [(0, 40, 0), (40, t["x"].shape[0], 1)]
    return do.block_forward(t["x"], mod, segments, t[norms[0]], t[norms[1]],
                            lambda h: bo.linear_bf16(h, t["w.attn.weight"]),
                            lambda h: bo.linear_bf16(h, t["w.fc1.weight"]),
                            lambda a: bo.linear_bf16(a, t["w.fc2.weight"]))


def test_block_forward_matches_reference_golden():
    """dit_oracle.block_forward against the reference's make_fast_block_forward output: the modulation
    order, which norm feeds which half and the SwiGLU MLP. Swapping two modulation tables, the two norms,
    or the SwiGLU halves each fails it."""
    t, meta = _dit_golden()
    assert meta["segments"] == "0:40:0,40:96:1"
    want = t["out"].float()
    got = _dit_oracle(t).float()
    steps = (got - want).abs() / torch.ldexp(torch.ones_like(want), torch.frexp(want)[1] - 8)
    assert steps.max().item() <= 1 and (steps == 0).float().mean().item() >= 0.99, steps.max().item()
    bar = 8 * (got - want).abs().max().item() + 1e-2
    for order in (("scale_msa", "shift_msa", "gate_msa", "shift_mlp", "scale_mlp", "gate_mlp"),
                  ("shift_mlp", "scale_mlp", "gate_mlp", "shift_msa", "scale_msa", "gate_msa"),
                  ("shift_msa", "scale_msa", "gate_mlp", "shift_mlp", "scale_mlp", "gate_msa")):
        assert (_dit_oracle(t, order).float() - want).abs().max().item() > bar, order
    swapped = _dit_oracle(t, norms=("w.norm2.weight", "w.norm1.weight")).float()
    assert (swapped - want).abs().max().item() > bar
    flipped = do.block_forward(t["x"], tuple(t[f"mod.{n}"] for n in ("shift_msa", "scale_msa", "gate_msa",
                                                                      "shift_mlp", "scale_mlp", "gate_mlp")),
                               [(0, 40, 0), (40, 96, 1)], t["w.norm1.weight"], t["w.norm2.weight"],
                               lambda h: h @ t["w.attn.weight"].t(),
                               lambda h: torch.cat((h @ t["w.fc1.weight"].t()).chunk(2, -1)[::-1], -1),
                               lambda a: a @ t["w.fc2.weight"].t()).float()
    assert (flipped - want).abs().max().item() > bar
