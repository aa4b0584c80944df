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
