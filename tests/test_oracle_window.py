"""Pins the window oracle against the reference's own known answers and independent forms.

Known answers: ``tests/test_window.py:193-202`` (window_bounds / full_coverage),
``tests/test_window.py:378-389`` (mask cases), ``tests/test_window.py:72-94``
(grouped == dense masked SDPA at 3 (chunk, radius) x 4 anchor modes, frames 11,
per_frame 3, heads 2, dim 5, 4 global rows before / 2 after, seed 1000+10*chunk+radius).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import window_oracle as wo


def test_window_bounds_known_answers():
    assert wo.window_bounds(4, 1) == [(-1, 1), (0, 2), (1, 3), (2, 4)]
    assert wo.window_bounds(6, 1, 5)[0] == (-5, 9)
    assert wo.window_bounds(6, 1, 5)[5] == (0, 14)
    assert wo.full_coverage(wo.window_bounds(6, 1, 5), 6)
    assert not wo.full_coverage(wo.window_bounds(16, 1, 5), 16)
    with pytest.raises(ValueError):
        wo.window_bounds(3, -1)
    with pytest.raises(ValueError):
        wo.full_coverage([(0, 1)], 2)


def test_full_cover_threshold_for_chunk5_radius1():
    # up to 10 frames every window covers all frames; 11 frames is the first windowed case
    assert all(wo.full_coverage(wo.window_bounds(n, 1, 5), n) for n in range(1, 11))
    assert not wo.full_coverage(wo.window_bounds(11, 1, 5), 11)
    assert wo.full_coverage(wo.window_bounds(7, 1, 5), 7)


def test_mask_hand_cases():
    # 4 global rows, 3 frames of 10 tokens, 6 trailing global rows; frame 2 only sees frame 0
    lo = torch.zeros(40, dtype=torch.long)
    hi = torch.full((40,), 2, dtype=torch.long)
    hi[24:34] = 0
    mask = wo.mask_from_tables(40, 4, 34, 3, 10, lo, hi, "none")
    assert not bool(mask[30, 18])   # frame 1 is outside frame 2's window
    assert bool(mask[30, 8])        # frame 0 inside
    assert bool(mask[30, 36])       # global key
    assert bool(mask[1, 18])        # global query
    anchored = wo.mask_from_tables(40, 4, 34, 3, 10, lo, hi, "both")
    assert bool(anchored[30, 18])   # last frame is an anchor row


def _brute_keys(row, seq, vs, ve, frames, per_frame, bounds, anchors):
    """Allowed keys by explicit enumeration (written independently of allowed_mask)."""
    if row < vs or row >= ve:
        return set(range(seq))
    frame = (row - vs) // per_frame
    if anchors in ("rows", "both") and frame in (0, frames - 1):
        return set(range(seq))
    lo, hi = bounds[frame]
    sel = set(range(max(lo, 0), min(hi, frames - 1) + 1))
    if anchors in ("columns", "both"):
        sel |= {0, frames - 1}
    keys = set(range(vs)) | set(range(ve, seq))
    for f in sel:
        keys |= set(range(vs + f * per_frame, vs + (f + 1) * per_frame))
    return keys


@pytest.mark.parametrize("anchors", wo.ANCHOR_FRAME_MODES)
@pytest.mark.parametrize("chunk,radius", [(0, 0), (0, 2), (3, 1), (4, 2)])
def test_mask_and_intervals_match_brute_force(anchors, chunk, radius):
    frames, per_frame, vs, after = 11, 3, 4, 2
    ve = vs + frames * per_frame
    seq = ve + after
    bounds = wo.window_bounds(frames, radius, chunk)
    mask = wo.allowed_mask(seq, vs, ve, frames, per_frame, bounds, anchors)
    for row in range(seq):
        want = _brute_keys(row, seq, vs, ve, frames, per_frame, bounds, anchors)
        assert set(torch.nonzero(mask[row]).flatten().tolist()) == want
        got = set()
        for a, b in wo.row_key_intervals(row, seq, vs, ve, frames, per_frame, bounds, anchors):
            got |= set(range(a, b))
        assert got == want


@pytest.mark.parametrize("chunk,radius", [(0, 2), (3, 1), (4, 2)])
@pytest.mark.parametrize("anchors", wo.ANCHOR_FRAME_MODES)
def test_grouped_matches_masked_and_sdpa(chunk, radius, anchors):
    gen = torch.Generator().manual_seed(1000 + chunk * 10 + radius)
    frames, per_frame, heads, dim = 11, 3, 2, 5
    before, after = 4, 2
    vs, ve = before, before + frames * per_frame
    seq = ve + after
    q = torch.randn(seq, heads, dim, generator=gen)
    k = torch.randn(seq, heads, dim, generator=gen)
    v = torch.randn(seq, heads, dim, generator=gen)
    bounds = wo.window_bounds(frames, radius, chunk)
    scale = dim ** -0.5
    got = wo.window_attention_grouped(q, k, v, vs, ve, frames, per_frame, bounds, scale, anchors)
    masked = wo.window_attention_masked(q, k, v, vs, ve, frames, per_frame, bounds, scale, anchors)
    allowed = wo.allowed_mask(seq, vs, ve, frames, per_frame, bounds, anchors)
    sdpa = F.scaled_dot_product_attention(q.permute(1, 0, 2).unsqueeze(0), k.permute(1, 0, 2).unsqueeze(0),
                                          v.permute(1, 0, 2).unsqueeze(0), attn_mask=allowed[None, None],
                                          scale=scale).squeeze(0).permute(1, 0, 2)
    torch.testing.assert_close(got, masked, atol=2e-6, rtol=2e-5)
    torch.testing.assert_close(got, sdpa, atol=2e-6, rtol=2e-5)
    rows = [0, vs, vs + 5, ve - 1, seq - 1]
    sampled = wo.window_attention_rows(q, k, v, rows, vs, ve, frames, per_frame, bounds, scale, anchors)
    torch.testing.assert_close(sampled, got[rows], atol=2e-6, rtol=2e-5)


def test_identical_keys_give_mean_of_allowed_values():
    # with all keys equal, softmax is uniform over the allowed set: the output is the mean of V there
    frames, per_frame, vs = 13, 4, 6
    ve = vs + frames * per_frame
    seq = ve
    bounds = wo.window_bounds(frames, 1, 5)
    q = torch.randn(seq, 1, 8)
    k = torch.ones(seq, 1, 8)
    v = torch.randn(seq, 1, 8)
    out = wo.window_attention_grouped(q, k, v, vs, ve, frames, per_frame, bounds, 0.3, "both")
    for row in (0, vs + per_frame * 3 + 1, vs + per_frame * 7, ve - 1):
        keys = sorted(_brute_keys(row, seq, vs, ve, frames, per_frame, bounds, "both"))
        torch.testing.assert_close(out[row, 0], v[keys, 0].mean(0), atol=1e-6, rtol=1e-5)


def test_full_shape_key_counts_and_pairs():
    # 512 text rows + 31 frames x 1296 tokens, chunk 5, radius 1, anchors both (S = 40 688)
    frames, tpf, text = 31, 1296, 512
    vs, ve = text, text + frames * tpf
    seq = ve
    bounds = wo.window_bounds(frames, 1, 5)
    counts = {}
    for f in range(frames):
        iv = wo.row_key_intervals(vs + f * tpf, seq, vs, ve, frames, tpf, bounds, "both")
        counts[f] = sum(b - a for a, b in iv)
    assert counts[0] == counts[30] == seq == 40688
    assert {counts[f] for f in range(1, 5)} == {14768}
    assert {counts[f] for f in range(5, 10)} == {21248}
    assert {counts[f] for f in range(10, 25)} == {22544}
    assert {counts[f] for f in range(25, 30)} == {16064}
    pairs = wo.pair_count(seq, vs, ve, frames, tpf, bounds, "both")
    assert pairs == 512 * 40688 + 2 * 1296 * 40688 + 1296 * (4 * 14768 + 5 * 21248 + 15 * 22544 + 5 * 16064)
    assert abs(pairs - 8.829e8) / 8.829e8 < 1e-3
    assert abs(4 * 128 * 40 * pairs - 1.8082e13) / 1.8082e13 < 1e-3


def test_a_wrong_anchor_mode_fails_parity():
    """With distinct q / k / v every anchor mode gives a different result, far outside the GPU tests' bar
    (the reference's autotune check, ``tests/test_autotune.py:11-41``: a backend with the wrong anchors must fail
    parity), so a kernel or plan that mixed up the modes could not pass them."""
    gen = torch.Generator().manual_seed(77)
    frames, per_frame, heads, dim = 11, 4, 2, 16
    vs = 6
    ve = vs + frames * per_frame
    seq = ve + 3
    q, k, v = (torch.randn(seq, heads, dim, generator=gen) for _ in range(3))
    bounds = wo.window_bounds(frames, 1, 5)
    outs = {m: wo.window_attention_grouped(q, k, v, vs, ve, frames, per_frame, bounds, dim ** -0.5, m)
            for m in wo.ANCHOR_FRAME_MODES}
    modes = list(outs)
    for i, a in enumerate(modes):
        for b in modes[i + 1:]:
            assert (outs[a] - outs[b]).abs().max().item() > 0.1, (a, b)
