"""The 50-block VDN-H3 hybrid attention stack over one 8-step denoising pass, on the GPU, at the full
shape: 40,688 tokens (512 text rows + 31 frames x 1296), 40 heads x 128, hidden 5120, W8A8 int8
projections, k/v short convolutions, anchors both. Each block runs the int8 q/k/v projection, the
window softmax attention and the delta-rule branch, the sigmoid gate-and-sum and the int8
out-projection; the pass feeds ``x <- x + block(rms_norm(x))`` (random-init blocks).

No CPU oracle runs 400 full-shape block calls, so the pass is checked through properties every
correct stack has, each against the single-block path that the other GPU tests pin to the oracle:

* the output is finite, and two passes from the same input are bit-identical;
* a block called inside the pass gives, bit for bit, what the same block gives called on its own
  with the same input;
* with the linear branch switched off, that block's text rows and anchor-frame rows are unchanged
  (the branch adds nothing there) and its inner video rows change (the branch's delta).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_stack_eight_step_denoising_pass(device):
    from vdn_h3_amd import synth
    from vdn_h3_amd.hybrid import forward_scope

    w = synth.WINDOW_FULL
    lay = w.layout
    blocks, steps, hidden = 50, 8, 5120
    print(f"case stack {blocks} blocks x {steps} steps, S={lay.seq_len}", flush=True)
    state, forwards = synth.hybrid_stack(blocks, w.heads, w.head_dim, hidden, device)
    x0 = synth.randn((lay.seq_len, hidden), 0, device=device, dtype=torch.bfloat16)
    probe, seen = (5, 17), {}

    def keep(step, index, block_in, block_out):
        if (step, index) == probe:
            seen["in"], seen["out"] = block_in.clone(), block_out.clone()

    with torch.no_grad(), forward_scope(lay):
        first = synth.denoise_pass(forwards, x0.clone(), steps, keep)
        torch.cuda.synchronize()
        print("  pass 1 done", flush=True)
        second = synth.denoise_pass(forwards, x0.clone(), steps)
        alone = forwards[probe[1]](seen["in"])
        state.config["linear_enabled"] = False
        try:
            no_branch = forwards[probe[1]](seen["in"])
        finally:
            state.config["linear_enabled"] = True
    torch.cuda.synchronize()
    print("  pass 2 done", flush=True)
    assert torch.isfinite(first).all()
    assert torch.equal(first, second)
    assert torch.equal(alone, seen["out"])
    T, vs = lay.tokens_per_frame, lay.video_start
    unchanged = torch.cat([torch.arange(0, vs + T), torch.arange(vs + (lay.num_frames - 1) * T, lay.seq_len)])
    inner = torch.arange(vs + T, vs + (lay.num_frames - 1) * T)
    assert torch.equal(no_branch[unchanged.to(device)], alone[unchanged.to(device)])
    changed = (no_branch[inner.to(device)] != alone[inner.to(device)]).float().mean().item()
    print(f"  inner video values changed by the branch: {changed:.3f}", flush=True)
    assert changed > 0.5
