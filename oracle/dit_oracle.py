"""Oracle: the MiniMax-H3 DiT block pointwise passes and MLP around the hybrid attention, CPU.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates ``vdn_h3/block_kernels.py`` in eager bf16 torch, every op rounding to bf16 as the
reference's tensors do:

* ``segment_indices`` -> ``BlockPointwiseCache._fill_indices`` (``:34-62``)
* ``pre``             -> ``_pre_body`` (``:85-89``): ``rms_norm(x, w, eps) * (1 + scale[i]) + shift[i]``
* ``post``            -> ``_post_body`` (``:92-93``): ``residual + gate[i] * branch``
* ``swiglu``          -> ``_swiglu_body`` (``:113-116``): ``silu(gate) * up``
* ``block_forward``   -> ``make_fast_block_forward.forward`` (``:163-235``) with the attention and
  the two MLP projections as callables

Pinning (``tests/test_oracle_dit.py``): ``F.rms_norm`` for the norm; special cases that fix each
term: scale = -1 gives exactly the shift, scale = shift = 0 the plain norm, gate = 0 the
residual, silu(0) = 0, a large gate value gives up * gate; the segment map against a
brute-force token loop and its error cases.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def segment_indices(segments, rows):
    """Per-token modulation row of contiguous ``(start, stop, row)`` segments."""
    ids = torch.empty(rows, dtype=torch.long)
    covered = 0
    for start, stop, row in segments:
        start, stop = int(start), int(stop)
        if start != covered or stop < start or stop > rows:
            raise ValueError("MiniMax-H3 modulation segments must cover the sequence contiguously")
        if isinstance(row, torch.Tensor) and row.numel() == stop - start and row.numel() != 1:
            ids[start:stop] = row.reshape(-1).long()
        else:
            ids[start:stop] = int(row.reshape(-1)[0]) if isinstance(row, torch.Tensor) else int(row)
        covered = stop
    if covered != rows:
        raise ValueError(f"MiniMax-H3 modulation segments cover {covered}/{rows} rows")
    return ids


def pre(hidden, weight, eps, scale, shift, indices):
    """``_pre_body`` in bf16."""
    normed = F.rms_norm(hidden, (hidden.shape[-1],), weight, eps)
    return normed * (1.0 + scale.index_select(0, indices).to(normed.dtype)) + shift.index_select(0, indices).to(
        normed.dtype)


def post(residual, gate, indices, branch_out):
    """``_post_body`` in bf16."""
    return residual + gate.index_select(0, indices).to(residual.dtype) * branch_out


def swiglu(hidden):
    gate, up = hidden.chunk(2, dim=-1)
    return F.silu(gate) * up


def block_forward(x, mod, segments, norm1, norm2, attention, fc1, fc2, eps=1e-6):
    """The fused DiT block: ``mod`` = (shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp)."""
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = mod
    idx = segment_indices(segments, x.shape[0])
    h = pre(x, norm1, eps, scale_msa, shift_msa, idx)
    x = post(x, gate_msa, idx, attention(h))
    h = pre(x, norm2, eps, scale_mlp, shift_mlp, idx)
    return post(x, gate_mlp, idx, fc2(swiglu(fc1(h))))
