"""Oracle: VDN-H3 window geometry and exact local-window softmax attention (CPU, fp32).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates ``vdn_h3/window.py`` of hyukudan/ComfyUI-Kirei-VDN-H3 v0.3.3:

* ``window_bounds``        -> ``vdn_h3/window.py:141-153``
* ``full_coverage``        -> ``vdn_h3/window.py:156-159``
* ``validate_layout``      -> ``vdn_h3/window.py:162-178``
* ``window_runs``          -> ``vdn_h3/window.py:248-270``
* ``allowed_mask``         -> ``vdn_h3/window.py:316-344`` (``_build_window_tables`` + ``mask_mod``)
* ``window_attention_grouped`` -> ``vdn_h3/window.py:277-313`` (grouped SDPA, exact)
* ``window_attention_masked``  -> the dense masked-SDPA oracle of ``tests/test_window.py:41-69``

Pinning (independent checks in ``tests/test_oracle_window.py``):

* ``window_bounds`` / ``full_coverage``: the reference's known-answer cases
  ``tests/test_window.py:193-202``.
* ``allowed_mask``: the hand cases of ``tests/test_window.py:378-389`` and a
  brute-force set construction written independently (``tests/test_optimized_runtime.py:53-94``
  style), plus the per-row key counts of the 31-frame x 1296-token layout
  (14 768 / 21 248 / 22 544 / 16 064 / 40 688 keys, 8.829e8 pairs per head).
* ``window_attention_grouped`` vs ``window_attention_masked``: two different
  formulations (key gather per run vs additive mask on the full score matrix) must agree;
  ``window_attention_masked`` is further checked against
  ``torch.nn.functional.scaled_dot_product_attention`` with a boolean mask (a library
  routine) and against closed forms (identical keys -> mean of the allowed values).
"""

from __future__ import annotations

import torch

ANCHOR_FRAME_MODES = ("none", "columns", "rows", "both")


def window_bounds(num_frames: int, radius: int, chunk: int = 0) -> list[tuple[int, int]]:
    """Frame window ``[(f//c - r)*c, (f//c + r + 1)*c - 1]`` (``vdn_h3/window.py:141-153``)."""
    if isinstance(num_frames, bool) or not isinstance(num_frames, int) or num_frames < 0:
        raise ValueError("num_frames must be a non-negative integer")
    if isinstance(radius, bool) or not isinstance(radius, int) or radius < 0:
        raise ValueError("radius must be a non-negative integer")
    if isinstance(chunk, bool) or not isinstance(chunk, int):
        raise ValueError("chunk must be an integer")
    if chunk <= 0:
        return [(f - radius, f + radius) for f in range(num_frames)]
    return [((f // chunk - radius) * chunk, (f // chunk + radius + 1) * chunk - 1) for f in range(num_frames)]


def full_coverage(bounds, num_frames: int) -> bool:
    """Every frame's window covers every frame (``vdn_h3/window.py:156-159``)."""
    if len(bounds) != num_frames:
        raise ValueError("bounds must contain exactly one entry per frame")
    return all(lo <= 0 and hi >= num_frames - 1 for lo, hi in bounds)


def validate_layout(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames):
    """Geometry checks with the reference's ValueError messages (``vdn_h3/window.py:162-178``)."""
    if anchor_frames not in ANCHOR_FRAME_MODES:
        raise ValueError(f"anchor_frames={anchor_frames!r}; expected one of {ANCHOR_FRAME_MODES}")
    if num_frames <= 0 or tokens_per_frame <= 0:
        raise ValueError("num_frames and tokens_per_frame must be positive")
    if not 0 <= video_start <= video_end <= seq:
        raise ValueError("video range is outside the packed sequence")
    if video_end - video_start != num_frames * tokens_per_frame:
        raise ValueError("video range does not equal num_frames * tokens_per_frame")
    if len(bounds) != num_frames:
        raise ValueError("bounds must contain exactly one entry per frame")
    for frame, pair in enumerate(bounds):
        if len(pair) != 2:
            raise ValueError(f"bounds[{frame}] must be a (lo, hi) pair")
        lo, hi = pair
        if lo > frame or hi < frame or lo > hi:
            raise ValueError(f"bounds[{frame}]={pair!r} does not contain its query frame")


def window_runs(num_frames, bounds, anchor_frames):
    """Runs of consecutive frames sharing one key-frame signature (``vdn_h3/window.py:248-270``).

    Returns ``[(first_frame, stop_frame, frames_or_None)]``; ``None`` marks dense anchor rows.
    """
    anchor_columns = anchor_frames in ("columns", "both")
    anchor_rows = anchor_frames in ("rows", "both")
    last = num_frames - 1
    runs = []
    run_start = 0
    previous = object()
    for frame in range(num_frames):
        if anchor_rows and frame in (0, last):
            signature = None
        else:
            lo = max(bounds[frame][0], 0)
            hi = min(bounds[frame][1], last)
            selected = set(range(lo, hi + 1))
            if anchor_columns:
                selected.update((0, last))
            signature = tuple(sorted(selected))
        if frame and signature != previous:
            runs.append((run_start, frame, previous))
            run_start = frame
        previous = signature
    runs.append((run_start, num_frames, previous))
    return runs


def allowed_mask(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames):
    """Boolean ``[seq, seq]`` window mask (``vdn_h3/window.py:316-344``)."""
    validate_layout(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames)
    lo = torch.zeros(seq, dtype=torch.long)
    hi = torch.full((seq,), num_frames - 1, dtype=torch.long)
    for frame, (lower, upper) in enumerate(bounds):
        a = video_start + frame * tokens_per_frame
        lo[a:a + tokens_per_frame] = max(lower, 0)
        hi[a:a + tokens_per_frame] = min(upper, num_frames - 1)
    return mask_from_tables(seq, video_start, video_end, num_frames, tokens_per_frame, lo, hi, anchor_frames)


def mask_from_tables(seq, video_start, video_end, num_frames, tokens_per_frame, lo, hi, anchor_frames):
    """``mask_mod`` of ``vdn_h3/window.py:327-344`` over all (query, key) pairs, from per-row lo/hi tables."""
    qi = torch.arange(seq).view(-1, 1)
    kj = torch.arange(seq).view(1, -1)
    global_q = (qi < video_start) | (qi >= video_end)
    global_k = (kj < video_start) | (kj >= video_end)
    q_frame = torch.div(qi - video_start, tokens_per_frame, rounding_mode="floor")
    k_frame = torch.div(kj - video_start, tokens_per_frame, rounding_mode="floor")
    allowed = global_q | global_k | ((k_frame >= lo.view(-1, 1)) & (k_frame <= hi.view(-1, 1)))
    if anchor_frames in ("columns", "both"):
        allowed = allowed | (k_frame == 0) | (k_frame == num_frames - 1)
    if anchor_frames in ("rows", "both"):
        allowed = allowed | (q_frame == 0) | (q_frame == num_frames - 1)
    return allowed


def row_key_intervals(row, seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames):
    """Allowed keys of one query row as merged half-open intervals (same rule as ``allowed_mask``)."""
    if row < video_start or row >= video_end:
        return [(0, seq)]
    frame = (row - video_start) // tokens_per_frame
    if anchor_frames in ("rows", "both") and frame in (0, num_frames - 1):
        return [(0, seq)]
    lo = max(bounds[frame][0], 0)
    hi = min(bounds[frame][1], num_frames - 1)
    frames = set(range(lo, hi + 1))
    if anchor_frames in ("columns", "both"):
        frames.update((0, num_frames - 1))
    pieces = []
    if video_start:
        pieces.append((0, video_start))
    for f in sorted(frames):
        pieces.append((video_start + f * tokens_per_frame, video_start + (f + 1) * tokens_per_frame))
    if video_end < seq:
        pieces.append((video_end, seq))
    pieces.sort()
    merged = []
    for a, b in pieces:
        if merged and merged[-1][1] >= a:
            merged[-1] = (merged[-1][0], max(merged[-1][1], b))
        else:
            merged.append((a, b))
    return merged


def _softmax_rows(q_rows, k_rows, v_rows, scale, dtype):
    """``softmax(scale * q k^T) v`` for ``[rows, H, D]`` operands, computed per head in ``dtype``."""
    q = q_rows.to(dtype).permute(1, 0, 2)
    k = k_rows.to(dtype).permute(1, 0, 2)
    v = v_rows.to(dtype).permute(1, 0, 2)
    scores = torch.matmul(q, k.transpose(-1, -2)) * scale
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v).permute(1, 0, 2)


def window_attention_grouped(query, key, value, video_start, video_end, num_frames, tokens_per_frame,
                             bounds, scale, anchor_frames="none", dtype=torch.float32):
    """Exact window attention by key gather per run (``vdn_h3/window.py:277-313``).

    Operands ``[S, H, D]`` in any float dtype; math in ``dtype`` (fp32 by default), output in ``dtype``.
    """
    if query.ndim != 3 or query.shape != key.shape or query.shape != value.shape:
        raise ValueError("query, key and value must share shape [sequence, heads, dim]")
    seq = query.shape[0]
    validate_layout(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames)
    out = torch.empty(query.shape, dtype=dtype)
    glob = [r for r in ((0, video_start), (video_end, seq)) if r[0] < r[1]]
    for a, b in glob:
        out[a:b] = _softmax_rows(query[a:b], key, value, scale, dtype)
    for first, stop, frames in window_runs(num_frames, bounds, anchor_frames):
        ra = video_start + first * tokens_per_frame
        rb = video_start + stop * tokens_per_frame
        if frames is None:
            ks, vs = key, value
        else:
            idx = [torch.arange(a, b) for a, b in glob]
            idx += [torch.arange(video_start + f * tokens_per_frame, video_start + (f + 1) * tokens_per_frame)
                    for f in frames]
            sel = torch.cat(idx)
            ks, vs = key[sel], value[sel]
        out[ra:rb] = _softmax_rows(query[ra:rb], ks, vs, scale, dtype)
    return out


def window_attention_masked(query, key, value, video_start, video_end, num_frames, tokens_per_frame,
                            bounds, scale, anchor_frames="none", dtype=torch.float32):
    """Exact window attention with an additive ``-inf`` mask over the full score matrix.

    Second formulation of the same operator (``tests/test_window.py:41-69`` uses SDPA with the
    boolean mask); intended for small sequences only (it materialises ``[H, S, S]``).
    """
    seq = query.shape[0]
    mask = allowed_mask(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames)
    q = query.to(dtype).permute(1, 0, 2)
    k = key.to(dtype).permute(1, 0, 2)
    v = value.to(dtype).permute(1, 0, 2)
    scores = torch.matmul(q, k.transpose(-1, -2)) * scale
    scores = scores.masked_fill(~mask.unsqueeze(0), float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), v).permute(1, 0, 2)


def window_attention_rows(query, key, value, rows, video_start, video_end, num_frames, tokens_per_frame,
                          bounds, scale, anchor_frames="none", heads=None, dtype=torch.float32, head_chunk=8):
    """Exact outputs for selected query ``rows`` (and optionally a subset of ``heads``).

    Used to check a full-size device result on a sample of rows without running the
    whole 40 688-row problem on the CPU. Rows that share a key set are evaluated together.
    Returns ``[len(rows), len(heads), D]``.
    """
    seq = query.shape[0]
    heads = list(range(query.shape[1])) if heads is None else list(heads)
    rows = [int(r) for r in rows]
    out = torch.empty((len(rows), len(heads), query.shape[2]), dtype=dtype)
    groups = {}
    for pos, row in enumerate(rows):
        iv = tuple(row_key_intervals(row, seq, video_start, video_end, num_frames, tokens_per_frame, bounds,
                                     anchor_frames))
        groups.setdefault(iv, []).append(pos)
    for iv, positions in groups.items():
        sel = torch.cat([torch.arange(a, b) for a, b in iv])
        qrows = torch.tensor([rows[p] for p in positions])
        q_all, k_all, v_all = query[qrows], key[sel], value[sel]  # one gather per key set, all heads
        for h0 in range(0, len(heads), head_chunk):
            hs = heads[h0:h0 + head_chunk]
            q = q_all[:, hs].to(dtype).permute(1, 0, 2)      # [h, r, D]
            k = k_all[:, hs].to(dtype).permute(1, 0, 2)      # [h, n, D]
            v = v_all[:, hs].to(dtype).permute(1, 0, 2)
            p = torch.softmax(torch.matmul(q, k.transpose(-1, -2)) * scale, dim=-1)
            res = torch.matmul(p, v).permute(1, 0, 2)               # [r, h, D]
            out[torch.tensor(positions)[:, None], torch.arange(h0, h0 + len(hs))[None, :]] = res
    return out


def pair_count(seq, video_start, video_end, num_frames, tokens_per_frame, bounds, anchor_frames) -> int:
    """Number of allowed (query, key) pairs per head (the FLOP model's ``sum_i |A(i)|``)."""
    total = 0
    # rows of one frame share their key set, so count per frame
    glob_rows = video_start + (seq - video_end)
    total += glob_rows * seq
    for frame in range(num_frames):
        row = video_start + frame * tokens_per_frame
        iv = row_key_intervals(row, seq, video_start, video_end, num_frames, tokens_per_frame, bounds,
                               anchor_frames)
        total += tokens_per_frame * sum(b - a for a, b in iv)
    return total
