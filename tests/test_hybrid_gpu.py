"""Parity of the HIP hybrid attention block (``make_vdn_forward``) with the reference (GPU).

Bars: max-abs 2e-2 and cosine >= 0.9995 (the block's parity bar) against the reference's own
``make_vdn_forward`` output (golden vector) and against the CPU oracle of the block; the
q/k RMSNorm pass and the standalone softmax gate within one bf16 rounding step.
"""

from __future__ import annotations

from pathlib import Path
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F
from safetensors import safe_open

from oracle import hybrid_oracle as ho
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _parity(got, want, what, atol=2e-2, min_cos=0.9995):
    got, want = got.float().cpu().flatten(), want.float().cpu().flatten()
    err = (got - want).abs().max().item()
    cos = F.cosine_similarity(got.double(), want.double(), dim=0).item()
    print(f"{what}: max abs {err:.3e}, cosine {cos:.7f}", flush=True)
    assert torch.isfinite(got).all(), what
    assert err <= atol and cos >= min_cos, f"{what}: max abs {err:.3e}, cosine {cos:.7f}"


def _attn(aw, heads, dim, device, precision="bf16"):
    from vdn_h3_amd.linear import HipLinear

    def forward(*args, **kwargs):  # the original forward must not run while a layout is published
        raise AssertionError("original attention forward called")

    return SimpleNamespace(
        heads=heads, head_dim=dim, forward=forward,
        qkv_proj=HipLinear(aw["qkv_proj.weight"].to(device), precision),
        out_proj=HipLinear(aw["out_proj.weight"].to(device), precision),
        q_norm=SimpleNamespace(weight=aw["q_norm.weight"].to(device), eps=1e-6),
        k_norm=SimpleNamespace(weight=aw["k_norm.weight"].to(device), eps=1e-6))


def _block(aw, bw, heads, dim, device, precision="bf16", config=None, branch_execution="serial", short_conv=()):
    from vdn_h3_amd.hybrid import VDNState, make_vdn_forward
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    attn = _attn(aw, heads, dim, device, precision)
    branch = OptimizedLinearBranch(bw, heads, dim, short_conv=short_conv, enable_text_state=True)
    cfg = {"enable_softmax_gate": True, "linear_enabled": True, "enable_text_state": True}
    cfg.update(config or {})
    state = VDNState("test", cfg, [branch], heads, dim, branch_execution=branch_execution)
    return make_vdn_forward(attn, state, 0), state


def _run(forward, x, layout):
    from vdn_h3_amd.hybrid import forward_scope

    with torch.no_grad(), forward_scope(layout):
        out = forward(x)
    torch.cuda.synchronize()
    return out


def _golden():
    from vdn_h3_amd.layout import text_first_layout

    with safe_open(str(GOLDEN / "hybrid_13f.safetensors"), "pt") as f:
        t, meta = {k: f.get_tensor(k) for k in f.keys()}, f.metadata()
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    grid = tuple(map(int, meta["grid"].split("x")))
    layout = text_first_layout(text, frames, grid, anchor_frames=meta["anchor_frames"])
    bw = {k[2:]: v for k, v in t.items() if k.startswith("w.")}
    aw = {k[5:]: v for k, v in t.items() if k.startswith("attn.")}
    return t, layout, aw, bw, heads, dim


def test_block_matches_reference_golden(device):
    print("case hybrid block golden (13 frames, 2 x 64)", flush=True)
    t, layout, aw, bw, heads, dim = _golden()
    forward, state = _block(aw, {k: v.to(device) for k, v in bw.items()}, heads, dim, device)
    out = _run(forward, t["x"].to(device), layout)
    assert state.last_attention_backend == "hip"
    _parity(out, t["out"], "block vs reference make_vdn_forward")
    _parity(out, ho.vdn_forward(t["x"], layout, aw, bw, heads, dim), "block vs oracle")


def _synthetic(frames, grid, text, heads, dim, hidden, seed=0):
    from vdn_h3_amd import synth
    from vdn_h3_amd.layout import text_first_layout

    layout = text_first_layout(text, frames, grid)
    x = synth.randn((layout.seq_len, hidden), seed, dtype=torch.bfloat16)
    bw = synth.branch_weights(heads, dim, hidden, seed=seed + 100)
    aw = {"qkv_proj.weight": synth.randn((3 * heads * dim, hidden), seed + 1, dtype=torch.bfloat16, scale=0.05),
          "out_proj.weight": synth.randn((hidden, heads * dim), seed + 2, dtype=torch.bfloat16, scale=0.05),
          "q_norm.weight": (1 + 0.1 * synth.randn((dim,), seed + 3)).to(torch.bfloat16),
          "k_norm.weight": (1 + 0.1 * synth.randn((dim,), seed + 4)).to(torch.bfloat16)}
    return layout, x, aw, bw


@pytest.mark.parametrize("frames", [7, 13])
def test_block_d128_vs_oracle(device, frames):
    """4 heads x 128, hidden 512, 16x16-token frames; 7 frames is full cover (dense, no branch)."""
    print(f"case hybrid block d128 frames={frames}", flush=True)
    heads, dim, hidden = 4, 128, 512
    layout, x, aw, bw = _synthetic(frames, (16, 16), 64, heads, dim, hidden)
    forward, state = _block(aw, {k: v.to(device) for k, v in bw.items()}, heads, dim, device)
    out = _run(forward, x.to(device), layout)
    assert state.last_attention_backend == ("dense_exact" if layout.full_cover else "hip")
    torch.set_num_threads(16)
    _parity(out, ho.vdn_forward(x, layout, aw, bw, heads, dim), f"block d128 {frames} frames vs oracle")


def test_block_int8_projections_vs_oracle(device):
    """W8A8 int8 qkv / out projections (per-token x per-channel) and an int8 to_out_linear."""
    from vdn_h3_amd import projection

    print("case hybrid block int8 projections", flush=True)
    heads, dim, hidden = 4, 128, 512
    layout, x, aw, bw = _synthetic(13, (16, 16), 64, heads, dim, hidden, seed=7)
    dbw = {k: v.to(device) for k, v in bw.items()}
    (qbw,), _ = projection.prepare_projection_maps([dbw], device, "int8")
    forward, _ = _block(aw, qbw, heads, dim, device, precision="int8")
    out = _run(forward, x.to(device), layout)

    def int8_project(weight):
        wq, ws = qo.int8_quantize_rows(weight)
        return lambda rows: qo.int8_linear(*qo.int8_quantize_rows(rows), wq, ws.reshape(1, -1))

    want = ho.vdn_forward(x, layout, aw, bw, heads, dim, project_qkv=int8_project(aw["qkv_proj.weight"]),
                          project_out=int8_project(aw["out_proj.weight"]),
                          branch_projector=int8_project(bw["to_out_linear.weight"]))
    _parity(out, want, "block int8 vs oracle")


@pytest.mark.parametrize("anchors", ["both", "none"])
def test_parallel_branch_execution_is_bit_identical(device, anchors):
    """branch_execution="parallel" (the branch on a second stream, joined at the to_out_linear
    accumulation) gives the serial block's bits, with anchor rows skipped or not, int8 projections and
    the k/v short convolutions; twice in a row, so the second call reuses the branch stream."""
    from vdn_h3_amd import projection, synth
    from vdn_h3_amd.layout import text_first_layout

    print(f"case hybrid block parallel branch execution anchors={anchors}", flush=True)
    heads, dim, hidden = 4, 128, 512
    _, x, aw, _ = _synthetic(13, (16, 16), 64, heads, dim, hidden, seed=9)
    layout = text_first_layout(64, 13, (16, 16), anchor_frames=anchors)
    bw = synth.branch_weights(heads, dim, hidden, seed=109, short_conv=("k", "v"))
    dbw = {k: v.to(device) for k, v in bw.items()}
    (qbw,), _ = projection.prepare_projection_maps([dbw], device, "int8")
    outs = {}
    for mode in ("serial", "parallel"):
        forward, state = _block(aw, qbw, heads, dim, device, precision="int8", branch_execution=mode,
                                short_conv=("k", "v"))
        outs[mode] = [_run(forward, x.to(device), layout).cpu() for _ in range(2)]
        state.release()
    assert torch.equal(outs["serial"][0], outs["serial"][1])
    for got in outs["parallel"]:
        assert torch.equal(got, outs["serial"][0])


def test_gate_off_and_branch_off(device):
    print("case hybrid block config switches", flush=True)
    t, layout, aw, bw, heads, dim = _golden()
    dbw = {k: v.to(device) for k, v in bw.items()}
    for cfg, kw in (({"enable_softmax_gate": False}, dict(gate_enabled=False)),
                    ({"linear_enabled": False}, dict(linear_enabled=False))):
        forward, _ = _block(aw, dbw, heads, dim, device, config=cfg)
        out = _run(forward, t["x"].to(device), layout)
        _parity(out, ho.vdn_forward(t["x"], layout, aw, bw, heads, dim, **kw), f"block {cfg} vs oracle")


@pytest.mark.parametrize("precision", ["bf16", "int8"])
@pytest.mark.parametrize("full_cover", [False, True])
def test_zero_softmax_gate_halves_the_block(device, precision, full_cover):
    """A softmax gate with zero weights and bias is sigmoid(0) = 1/2 (the reference's
    ``test_full_cover_gate_keeps_canonical_shape_and_loads_only_gate``, ``tests/test_hybrid.py``): with the
    branch off the block is exactly half the ungated block, bit for bit, since halving commutes with every
    rounding on the path (bf16 attention output, the gate product, the per-token int8 scale, the projection)."""
    from vdn_h3_amd import projection
    from vdn_h3_amd.layout import text_first_layout

    print(f"case zero softmax gate precision={precision} full_cover={full_cover}", flush=True)
    t, layout, aw, bw, heads, dim = _golden()
    if full_cover:
        layout = text_first_layout(16, 5, (8, 8))
        assert layout.full_cover
    x = t["x"][:layout.seq_len].to(device)
    dbw = {k: v.to(device) for k, v in bw.items()}
    dbw["softmax_gate.up.weight"] = torch.zeros_like(dbw["softmax_gate.up.weight"])
    dbw["softmax_gate.up.bias"] = torch.zeros_like(dbw["softmax_gate.up.bias"])
    if precision == "int8":
        (dbw,), _ = projection.prepare_projection_maps([dbw], device, "int8")
    outs = []
    for gate in (True, False):
        forward, _ = _block(aw, dbw, heads, dim, device, precision=precision,
                            config={"enable_softmax_gate": gate, "linear_enabled": False})
        outs.append(_run(forward, x, layout))
    gated, plain = outs
    assert torch.count_nonzero(plain) > 0
    assert torch.equal(gated, plain * 0.5)


def test_branch_changes_only_inner_video_rows(device):
    """The branch adds to the video rows only (the reference's ``test_linear_delta_changes_only_target_video_rows``):
    against the block with ``linear_enabled=False`` the text rows and the two anchor frames (``anchor_frames="both"``)
    keep their bits, and every inner frame changes."""
    print("case branch rows", flush=True)
    t, layout, aw, bw, heads, dim = _golden()
    assert layout.anchor_frames == "both"
    dbw = {k: v.to(device) for k, v in bw.items()}
    outs = []
    for linear in (True, False):
        forward, _ = _block(aw, dbw, heads, dim, device, config={"linear_enabled": linear})
        outs.append(_run(forward, t["x"].to(device), layout))
    on, off = outs
    tpf, vs, ve = layout.tokens_per_frame, layout.video_start, layout.video_end
    same = torch.ones(layout.seq_len, dtype=torch.bool)
    same[vs + tpf:ve - tpf] = False
    assert torch.equal(on[same.to(device)], off[same.to(device)])
    inner = (on[vs + tpf:ve - tpf] != off[vs + tpf:ve - tpf]).view(layout.num_frames - 2, tpf, -1)
    assert bool(inner.any(dim=2).any(dim=1).all()), "every inner frame carries a branch delta"


def test_without_layout_calls_original_and_grad_mode_is_forward_only(device):
    """No layout: the original forward. Gradient mode with nothing that requires grad (the reference's
    deferred-branch case, ``vdn_h3/hybrid.py:424``): the no_grad block's bits and an output that needs
    no grad. An input or a branch weight that requires grad: RuntimeError (the block has no backward)."""
    from vdn_h3_amd.hybrid import VDNState, forward_scope, make_vdn_forward
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    t, layout, aw, bw, heads, dim = _golden()
    original = lambda x, rope_freqs=None, transformer_options=None: "original"  # noqa: E731
    dbw = {k: v.to(device) for k, v in bw.items()}
    forward, _ = _block(aw, dbw, heads, dim, device)
    forward._vdn_h3_original = original  # the forward it patched
    x = t["x"].to(device)
    assert forward(x) == "original"
    want = _run(forward, x, layout)
    with forward_scope(layout):
        got = forward(x)
    torch.cuda.synchronize()
    assert not got.requires_grad
    assert torch.equal(got, want)
    with forward_scope(layout), pytest.raises(RuntimeError, match="forward-only"):
        forward(x.clone().requires_grad_(True))
    grad_w = dict(dbw)
    grad_w["to_out_linear.weight"] = grad_w["to_out_linear.weight"].clone().requires_grad_(True)
    state = VDNState("t", {}, [OptimizedLinearBranch(grad_w, heads, dim)], heads, dim)
    with forward_scope(layout), pytest.raises(RuntimeError, match="forward-only"):
        make_vdn_forward(_attn(aw, heads, dim, device), state, 0)(x)
    with torch.no_grad(), forward_scope(layout), pytest.raises(RuntimeError, match="rows"):
        forward(x[:-1])


def test_qk_rmsnorm_and_softmax_gate_ops(device):
    from vdn_h3_amd import synth
    from vdn_h3_amd.hybrid import normalise_qk
    from vdn_h3_amd.softmax_kernels import apply_softmax_gate

    print("case qk rmsnorm + softmax gate", flush=True)
    for dim in (64, 128):
        seq, heads = 1000, 5
        qkv = (3 * synth.randn((seq, 3 * heads * dim), 60)).to(torch.bfloat16)
        q, k, _ = synth.split_qkv(qkv, heads, dim)
        wq = (1 + 0.1 * synth.randn((dim,), 61)).to(torch.bfloat16)
        wk = (1 + 0.1 * synth.randn((dim,), 62)).to(torch.bfloat16)
        dq, dk, _ = synth.split_qkv(qkv.to(device), heads, dim)
        qn, kn = normalise_qk(dq, dk, wq.to(device), wk.to(device))
        for got, x, w in ((qn, q, wq), (kn, k, wk)):
            want = F.rms_norm(x, (dim,), w, 1e-6).float()
            ulp = torch.ldexp(torch.ones_like(want), torch.frexp(want)[1] - 8)   # bf16 spacing at want
            ulps = (got.cpu().float() - want).abs() / ulp
            assert ulps.max().item() <= 1.0, ulps.max().item()
        o = synth.randn((seq, heads, dim), 63, dtype=torch.bfloat16)
        g = torch.sigmoid(synth.randn((seq, heads), 64)).to(torch.bfloat16)
        got = apply_softmax_gate(o.to(device), g.to(device).unsqueeze(-1))
        assert torch.equal(got.cpu(), (o * g.unsqueeze(-1)).reshape(seq, heads * dim))


@pytest.mark.parametrize("dim,rot,shared", [(128, 128, False), (128, 64, True), (64, 64, False), (64, 32, False)])
def test_qk_rmsnorm_rope_op(device, dim, rot, shared):
    """Fused RMSNorm + split-half RoPE vs the oracle (one bf16 rounding; fp32 FMA order may move it)."""
    from vdn_h3_amd import synth
    from vdn_h3_amd.hybrid import normalise_qk

    print(f"case qk rmsnorm+rope D={dim} rot={rot} shared={shared}", flush=True)
    seq, heads = 777, 3
    qkv = (3 * synth.randn((seq, 3 * heads * dim), 65)).to(torch.bfloat16)
    q, k, _ = synth.split_qkv(qkv, heads, dim)
    wq = (1 + 0.1 * synth.randn((dim,), 66)).to(torch.bfloat16)
    wk = (1 + 0.1 * synth.randn((dim,), 67)).to(torch.bfloat16)
    rows = 1 if shared else seq
    theta = synth.randn((rows, rot // 2), 68) * 3
    c, s_ = torch.cos(theta), torch.sin(theta)
    freqs = torch.stack([torch.stack([c, -s_], -1), torch.stack([s_, c], -1)], -2)
    freqs = freqs.reshape(1, rows, 1, rot // 2, 2, 2)                       # a ComfyUI-style broadcast shape
    dq, dk, _ = synth.split_qkv(qkv.to(device), heads, dim)
    qn, kn = normalise_qk(dq, dk, wq.to(device), wk.to(device), 1e-6, rope_freqs=freqs.to(device))
    for got, x, w in ((qn, q, wq), (kn, k, wk)):
        want = ho.rms_rope_split_half(x, w, 1e-6, freqs, rot).float()
        exact = ho.rms_rope_split_half(x, w, 1e-6, freqs, rot, rounded=False)
        g32 = got.cpu().float()
        # one bf16 step at the exact value, plus fp32 rounding of the rotation's two terms (|y| <~ 8)
        # for results that nearly cancel: the kernel fuses a * y + b * y' into one FMA
        ulp = torch.ldexp(torch.ones_like(want), torch.frexp(exact)[1] - 8) + 2.0 ** -19
        excess = ((g32 - exact).abs() / ulp).max().item()
        assert excess <= 1.0, excess
        assert (g32 == want).float().mean().item() >= 0.99


def test_block_with_rope_vs_oracle(device):
    """The block forward with rope_freqs (RoPE on the softmax q/k; the branch reads the raw q/k)."""
    print("case hybrid block with rope", flush=True)
    heads, dim, hidden = 4, 128, 512
    layout, x, aw, bw = _synthetic(13, (16, 16), 64, heads, dim, hidden, seed=9)
    g = torch.Generator().manual_seed(90)
    theta = torch.randn(layout.seq_len, dim // 2, generator=g) * 3
    c, s_ = torch.cos(theta), torch.sin(theta)
    freqs = torch.stack([torch.stack([c, -s_], -1), torch.stack([s_, c], -1)], -2).reshape(
        1, layout.seq_len, 1, dim // 2, 2, 2)
    forward, _ = _block(aw, {k: v.to(device) for k, v in bw.items()}, heads, dim, device)
    from vdn_h3_amd.hybrid import forward_scope

    with torch.no_grad(), forward_scope(layout):
        out = forward(x.to(device), rope_freqs=freqs.to(device))
    torch.cuda.synchronize()
    torch.set_num_threads(16)
    _parity(out, ho.vdn_forward(x, layout, aw, bw, heads, dim, rope_freqs=freqs), "block with rope vs oracle")


def test_shared_gate_branch_gemm_is_bit_identical(device, monkeypatch):
    """The softmax gate, the branch's beta and its gate down-projection from one GEMM over x give the
    same block output, bit for bit, as the separate GEMMs."""
    from vdn_h3_amd import hybrid

    print("case hybrid block shared gate GEMM", flush=True)
    heads, dim, hidden = 4, 128, 512
    layout, x, aw, bw = _synthetic(13, (16, 16), 64, heads, dim, hidden)
    bwd = {k: v.to(device) for k, v in bw.items()}
    forward, state = _block(aw, bwd, heads, dim, device)
    shared = _run(forward, x.to(device), layout)
    assert state.__dict__.get("_gate_branch_cache"), "the shared GEMM did not run"
    monkeypatch.setattr(hybrid, "_gate_branch_weights", lambda *args: None)
    forward, _ = _block(aw, bwd, heads, dim, device)
    separate = _run(forward, x.to(device), layout)
    assert torch.equal(shared, separate)
