"""The frame-tiled VDN branch (``tile_frames``, ``vdn_h3/runtime.py:421-543``) on the GPU.

The reference tiles the branch to bound its memory: k / v features and frame statistics one tile of
frames at a time (the short convolution over the tile plus its temporal halo), the recurrence over all
frames, then the query features, gated readout and ``to_out_linear`` one tile at a time. Every frame's
statistics and readout and every row's projection depend on that frame or row alone, so the bar here is
bit-identity with the untiled call, plus the block parity bar against the reference's own golden.
"""

from __future__ import annotations

from pathlib import Path
from types import SimpleNamespace

import pytest
import torch
from safetensors import safe_open

from oracle import window_oracle as wo

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _rand(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _load(name):
    with safe_open(str(GOLDEN / name), "pt") as f:
        return {k: f.get_tensor(k) for k in f.keys()}, f.metadata()


def _parity(got, want, what, atol=2e-2, min_cos=0.9995):
    got, want = got.float().cpu().flatten(), want.float().cpu().flatten()
    err = (got - want).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.double(), want.double(), dim=0).item()
    print(f"{what}: max abs {err:.3e}, cosine {cos:.7f}", flush=True)
    assert torch.isfinite(got).all(), what
    assert err <= atol and cos >= min_cos, f"{what}: max abs {err:.3e}, cosine {cos:.7f}"


@pytest.mark.parametrize("fused", [True, False])
def test_readout_frame_range_equals_rows_of_full_call(device, fused):
    """vdnh3_readout(_fused_gate) over a frame range gives the range's rows of the all-frames call, bit for bit."""
    from vdn_h3_amd import branch

    print(f"case readout frame range fused={fused}", flush=True)
    frames, tokens, heads, dim = 11, 70, 2, 128
    bounds = [(lo - 1, hi - 1) for lo, hi in wo.window_bounds(frames + 2, 1, 5)[1:-1]]
    q = _rand((frames * tokens, heads, dim), 11, dtype=torch.bfloat16).to(device)
    prefix = _rand((frames, heads, dim, dim), 12, 0.1).to(device)
    suffix = _rand((frames, heads, dim, dim), 13, 0.1).to(device)
    alpha = (torch.rand(frames, heads, dim, generator=torch.Generator().manual_seed(14)) * 0.5 + 0.5).to(device)
    tstate = _rand((heads, dim, dim), 15, 0.1).to(device)
    norm_w = (1 + 0.1 * _rand((dim,), 17)).to(torch.bfloat16).to(device)
    if fused:
        hidden = _rand((frames * tokens, dim), 18, dtype=torch.bfloat16).to(device)
        w_up = _rand((heads * dim, dim), 19, 0.05, torch.bfloat16).to(device)
        b_up = _rand((heads * dim,), 20, 0.5, torch.bfloat16).to(device)
        gate_kw = lambda rows: dict(gate_hidden=hidden[rows], gate_up_weight=w_up, gate_up_bias=b_up)  # noqa: E731
        gate = None
    else:
        full_gate = torch.sigmoid(_rand((frames * tokens, heads * dim), 16)).to(torch.bfloat16).to(device)
        gate_kw = lambda rows: {}  # noqa: E731
    common = dict(text_state=tstate, bridge="alpha", num_frames=frames, tokens_per_frame=tokens)

    def call(start, stop):
        rows = slice(start * tokens, stop * tokens)
        g = gate if fused else full_gate[rows]
        return branch.readout_epilogue(q[rows], prefix, suffix, alpha, bounds, norm_w, g,
                                       frame_range=(start, stop), **gate_kw(rows), **common)

    full = call(0, frames)
    for start, stop in [(0, 3), (3, 8), (8, 11), (5, 6), (0, 11)]:
        part = call(start, stop)
        torch.cuda.synchronize()
        assert torch.equal(part, full[start * tokens:stop * tokens]), (start, stop)
    with pytest.raises(ValueError, match="frame_range"):
        call(4, 12)


def _branch_weights(heads, dim, hidden, conv):
    gen = {"beta_proj.weight": (heads, hidden), "alpha.down.weight": (dim, hidden),
           "alpha.up.weight": (heads * dim, dim), "output_gate.down.weight": (dim, hidden),
           "output_gate.up.weight": (heads * dim, dim), "to_out_linear.weight": (hidden, heads * dim)}
    w = {name: _rand(shape, 70 + i, 0.02, torch.bfloat16) for i, (name, shape) in enumerate(gen.items())}
    w["alpha.dt_bias"] = _rand((heads * dim,), 80, 0.5)
    w["alpha.A_log"] = _rand((heads,), 81, 0.5)
    w["output_gate.up.bias"] = _rand((heads * dim,), 82, 0.5, torch.bfloat16)
    w["norm.weight"] = (1 + 0.1 * _rand((dim,), 83)).to(torch.bfloat16)
    for i, name in enumerate("qkv"):
        if name in conv:
            w[f"short_conv.{name}_sp.weight"] = _rand((heads * dim, 1, 5, 5), 84 + i, 0.2, torch.bfloat16)
            w[f"short_conv.{name}_tm.weight"] = _rand((heads * dim, 1, 5), 87 + i, 0.4, torch.bfloat16)
    return w


@pytest.mark.parametrize("conv", [(), ("k", "v"), ("q", "k", "v")])
@pytest.mark.parametrize("skip_ends", [True, False])
def test_tiled_projected_delta_equals_untiled(device, conv, skip_ends):
    """tile_frames 1, 2, 4, 5 and one tile larger than the sequence: the same bits as the untiled branch,
    written and accumulated."""
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print(f"case tiled projected_delta conv={conv} skip_ends={skip_ends}", flush=True)
    frames, (gh, gw), text, heads, dim, hidden = 12, (6, 10), 24, 2, 128, 256
    tpf = gh * gw
    seq = text + frames * tpf
    w = {k: v.to(device) for k, v in _branch_weights(heads, dim, hidden, conv).items()}
    x = _rand((seq, hidden), 90, dtype=torch.bfloat16).to(device)
    qkv = _rand((seq, 3 * heads * dim), 91, dtype=torch.bfloat16).to(device)
    q, k, v = [y.view(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    br = OptimizedLinearBranch(w, heads, dim, short_conv=conv, enable_text_state=True)
    args = (w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds)
    kw = dict(frame_size=(gh, gw), text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=skip_ends)
    base = _rand((frames * tpf, hidden), 92, dtype=torch.bfloat16).to(device)
    with torch.no_grad():
        want = br.projected_delta(*args, tile_frames=0, **kw)
        want_acc = base.clone()
        br.projected_delta(*args, tile_frames=0, out=want_acc, accumulate=True, **kw)
        for tile in (1, 2, 4, 5, 40):
            got = br.projected_delta(*args, tile_frames=tile, **kw)
            got_acc = base.clone()
            br.projected_delta(*args, tile_frames=tile, out=got_acc, accumulate=True, **kw)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"tile_frames={tile}"
            assert torch.equal(got_acc, want_acc), f"tile_frames={tile}, accumulate"
        br.set_runtime(tile_frames=3)  # the runtime option is the default of the call
        got = br.projected_delta(*args, **kw)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    assert torch.count_nonzero(want) > 0


def test_tiled_branch_matches_reference_golden(device):
    """The short-convolution golden of the reference (13 frames of 8x8, 2 heads x 64) through tiles of 5 frames."""
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print("case tiled projected_delta short-conv golden", flush=True)
    t, meta = _load("branch_13f_conv.safetensors")
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    gh, gw = map(int, meta["grid"].split("x"))
    tpf = gh * gw
    w = {k[2:]: v.to(device) for k, v in t.items() if k.startswith("w.")}
    x, qkv = t["x"].to(device), t["qkv"].to(device)
    seq = x.shape[0]
    q, k, v = [y.view(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    br = OptimizedLinearBranch(w, heads, dim, short_conv=("k", "v"), enable_text_state=True)
    kw = dict(frame_size=(gh, gw), text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    args = (w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds)
    with torch.no_grad():
        untiled = br.projected_delta(*args, tile_frames=0, **kw)
        got = br.projected_delta(*args, tile_frames=5, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, untiled)
    _parity(got, t["delta"], "tiled short-conv projected_delta vs reference")


def test_block_with_tile_frames_equals_untiled(device):
    """VDNState(tile_frames=5) hands the option to its branches: the block output is the untiled block's, also
    with branch_execution="parallel" (a tiled branch runs in order after out_proj)."""
    from vdn_h3_amd.hybrid import VDNState, forward_scope, make_vdn_forward
    from vdn_h3_amd.layout import text_first_layout
    from vdn_h3_amd.linear import HipLinear
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print("case block tile_frames=5 (reference hybrid golden)", flush=True)
    t, meta = _load("hybrid_13f.safetensors")
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    grid = tuple(map(int, meta["grid"].split("x")))
    layout = text_first_layout(text, frames, grid, anchor_frames=meta["anchor_frames"])
    bw = {k[2:]: v.to(device) for k, v in t.items() if k.startswith("w.")}
    aw = {k[5:]: v for k, v in t.items() if k.startswith("attn.")}
    attn = SimpleNamespace(
        heads=heads, head_dim=dim, forward=None,
        qkv_proj=HipLinear(aw["qkv_proj.weight"].to(device), "bf16"),
        out_proj=HipLinear(aw["out_proj.weight"].to(device), "bf16"),
        q_norm=SimpleNamespace(weight=aw["q_norm.weight"].to(device), eps=1e-6),
        k_norm=SimpleNamespace(weight=aw["k_norm.weight"].to(device), eps=1e-6))
    cfg = {"enable_softmax_gate": True, "linear_enabled": True, "enable_text_state": True}
    outs = []
    for tile, mode in ((0, "serial"), (5, "serial"), (5, "parallel")):
        branch = OptimizedLinearBranch(bw, heads, dim, enable_text_state=True)
        state = VDNState("test", cfg, [branch], heads, dim, tile_frames=tile, branch_execution=mode)
        assert branch.tile_frames == tile
        with torch.no_grad(), forward_scope(layout):
            outs.append(make_vdn_forward(attn, state, 0)(t["x"].to(device)))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    _parity(outs[1], t["out"], "block with tile_frames=5 vs reference make_vdn_forward")
