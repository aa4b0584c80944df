"""Host planner of the window kernel (C++ in libvdnh3.so) against the oracle's key sets.

Runs on the CPU: the planner is host code. Every query row must be covered by exactly
one work item, and the union of that item's valid key ranges must equal the oracle's
allowed set, with no key counted twice.
"""

from __future__ import annotations

import pytest
import torch

from oracle import window_oracle as wo


def _check_plan(built_lib, seq, vs, ve, frames, per_frame, bounds, anchors):
    from vdn_h3_amd import window

    bm, bn = built_lib.vdnh3_window_block_m(), built_lib.vdnh3_window_block_n()
    items, tiles, pairs = window.build_plan_host(seq, vs, ve, frames, per_frame, bounds, anchors)
    counts = items[:, 3].tolist()
    assert counts == sorted(counts, reverse=True), "items are longest-first"
    covered = torch.zeros(seq, dtype=torch.int64)
    for q0, q1, off, cnt in items.tolist():
        assert 0 <= q0 < q1 <= seq and q1 - q0 <= bm
        covered[q0:q1] += 1
        keys = []
        for ks, packed in tiles[off:off + cnt].tolist():
            lo, hi = packed & 0xFFFF, packed >> 16
            assert ks % bn == 0 and 0 <= lo < hi <= bn
            keys.extend(range(ks + lo, ks + hi))
        assert len(keys) == len(set(keys)), "a key tile range is repeated"
        assert max(keys) < seq
        for row in {q0, (q0 + q1) // 2, q1 - 1}:
            want = set()
            for a, b in wo.row_key_intervals(row, seq, vs, ve, frames, per_frame, bounds, anchors):
                want |= set(range(a, b))
            assert set(keys) == want, (row, anchors)
    assert bool((covered == 1).all())
    assert pairs == wo.pair_count(seq, vs, ve, frames, per_frame, bounds, anchors)


@pytest.mark.parametrize("anchors", wo.ANCHOR_FRAME_MODES)
@pytest.mark.parametrize("chunk,radius", [(0, 0), (0, 2), (3, 1), (4, 2), (5, 1)])
def test_plan_small_geometries(built_lib, anchors, chunk, radius):
    frames, per_frame, vs, after = 11, 3, 4, 2
    ve = vs + frames * per_frame
    _check_plan(built_lib, ve + after, vs, ve, frames, per_frame, wo.window_bounds(frames, radius, chunk), anchors)


@pytest.mark.parametrize("frames,per_frame,text", [(7, 64, 16), (13, 64, 16), (31, 1296, 512), (12, 100, 0)])
def test_plan_packed_layouts(built_lib, frames, per_frame, text):
    bounds = wo.window_bounds(frames, 1, 5)
    _check_plan(built_lib, text + frames * per_frame, text, text + frames * per_frame, frames, per_frame, bounds,
                "both")


def test_plan_validation_errors(built_lib):
    from vdn_h3_amd import window

    with pytest.raises(ValueError, match="does not contain its query frame"):
        window.build_plan_host(40, 4, 34, 3, 10, [(0, 2), (0, 2), (0, 0)], "none")
    with pytest.raises(ValueError, match="one entry per frame"):
        window.build_plan_host(40, 4, 34, 3, 10, [(0, 2)] * 2, "none")
    with pytest.raises(ValueError, match="must be positive"):
        window.build_plan_host(40, 4, 4, 0, 10, [], "none")
    with pytest.raises(ValueError, match="video range does not equal"):
        window.build_plan_host(40, 4, 33, 3, 10, window.window_bounds(3, 1), "none")
    with pytest.raises(ValueError, match="anchor_frames"):
        window.build_plan_host(40, 4, 34, 3, 10, window.window_bounds(3, 1), "sideways")
