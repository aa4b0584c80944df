"""Parity of the HIP Video Delta Attention kernels with the CPU oracle (GPU).

Bars (the block parity bar: delta-rule outputs within max-abs 2e-2 and cosine >= 0.9995 of the fp32
reference path): per-stage checks are tighter where the arithmetic allows - A to fp32
rounding, B / bf16 outputs to one or two bf16 steps, the factor and scans to ~1e-4
relative (fp32 Cholesky and MFMA summation order).
"""

from __future__ import annotations

from pathlib import Path

import pytest
import torch
from safetensors import safe_open

from oracle import branch_oracle as bo
from oracle import window_oracle as wo

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _rand(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def _close(got, want, rtol, atol, what):
    got, want = got.float().cpu(), want.float().cpu()
    err = (got - want).abs()
    bad = err > atol + rtol * want.abs()
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} off, max err {err.max().item():.3e}"


def _parity(got, want, what, atol=2e-2, min_cos=0.9995):
    got, want = got.float().cpu().flatten(), want.float().cpu().flatten()
    err = (got - want).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.double(), want.double(), dim=0).item()
    assert torch.isfinite(got).all(), what
    assert err <= atol and cos >= min_cos, f"{what}: max abs {err:.3e}, cosine {cos:.6f}"


@pytest.mark.parametrize("dim", [64, 128])
def test_frame_statistics(device, dim):
    from vdn_h3_amd import branch

    print(f"case frame stats D={dim}", flush=True)
    frames, tokens, heads = 3, 100, 2
    k = _rand((frames * tokens, heads, dim), 1, dtype=torch.bfloat16)
    v = _rand((frames * tokens, heads, dim), 2, dtype=torch.bfloat16)
    beta = torch.sigmoid(_rand((frames * tokens, heads), 3)).to(torch.bfloat16)
    a, b = branch.frame_statistics_raw(k.to(device), v.to(device), beta.to(device), frames, tokens)
    kf = bo.to_fhsd(bo.activate(k, True), frames, heads, dim)
    vf = bo.to_fhsd(bo.activate(v, False), frames, heads, dim)
    bt = beta.reshape(frames, tokens, heads).permute(0, 2, 1)
    wa, wb = bo.frame_statistics(kf, vf, bt)
    _close(a, wa, 1e-5, 1e-5, "A")
    assert torch.equal(a.cpu(), a.cpu().transpose(-1, -2))
    _close(b, wb, 2 * 2.0 ** -8, 1e-6, "B")


@pytest.mark.parametrize("dim", [64, 128])
def test_frame_statistics_bf16_a(device, dim):
    """a_fp32=False: S = bf16(bf16(k~ beta)^T k~) and A = (S + S^T) / 2. The GPU's fp32 sums run in another
    order than the oracle's, so where one straddles a bf16 midpoint S moves by one of its bf16 steps: every
    A value within one bf16 step of the oracle's (at |A|), at least 99% of them exact; B as before."""
    from vdn_h3_amd import branch

    print(f"case frame stats bf16 A D={dim}", flush=True)
    frames, tokens, heads = 3, 100, 2
    k = _rand((frames * tokens, heads, dim), 21, dtype=torch.bfloat16)
    v = _rand((frames * tokens, heads, dim), 22, dtype=torch.bfloat16)
    beta = torch.sigmoid(_rand((frames * tokens, heads), 23)).to(torch.bfloat16)
    a, b = branch.frame_statistics_raw(k.to(device), v.to(device), beta.to(device), frames, tokens, a_fp32=False)
    a32, _ = branch.frame_statistics_raw(k.to(device), v.to(device), beta.to(device), frames, tokens)
    kf = bo.to_fhsd(bo.activate(k, True), frames, heads, dim)
    vf = bo.to_fhsd(bo.activate(v, False), frames, heads, dim)
    bt = beta.reshape(frames, tokens, heads).permute(0, 2, 1)
    wa, wb = bo.frame_statistics(kf, vf, bt, a_fp32=False)
    ga = a.cpu()
    assert torch.equal(ga, ga.transpose(-1, -2))
    step = torch.ldexp(torch.ones_like(wa), torch.frexp(wa)[1] - 8).clamp_min(2.0 ** -133)
    off = ((ga - wa).abs() / step)
    print(f"  A: {(off > 0).float().mean():.2e} of values off, max {off.max().item():.2f} steps", flush=True)
    assert off.max().item() <= 1.0 and (off == 0).float().mean().item() >= 0.99
    assert not torch.equal(ga, a32.cpu())                      # the bf16 rounding is applied
    _close(b, wb, 2 * 2.0 ** -8, 1e-6, "B")


def test_factor_and_status(device):
    from vdn_h3_amd import branch

    print("case factor", flush=True)
    frames, heads, dim, tokens = 3, 2, 128, 300
    kf = torch.nn.functional.normalize(_rand((frames, heads, tokens, dim), 4), dim=-1)
    beta = torch.sigmoid(_rand((frames, heads, tokens), 5))
    a = (kf * beta.unsqueeze(-1)).transpose(-1, -2) @ kf
    b = _rand((frames, heads, dim, dim), 6)
    alpha = torch.rand(frames, heads, dim, generator=torch.Generator().manual_seed(7))
    with branch.cholesky_runtime_scope():
        phi, jay = branch.VdnDelta().factor_apply(alpha.to(device), a.to(device), b.to(device))
    wphi, wjay, _ = bo.vdn_factor(alpha, a, b)
    _close(phi, wphi, 2e-4, 1e-6, "Phi")
    _close(jay, wjay, 2e-4, 2e-5, "J")
    bad = a.clone()
    bad[1, 1] = -2.0 * torch.eye(dim)
    with pytest.raises(torch.linalg.LinAlgError, match="factor 0, batch 3: leading minor of order 1"):
        with branch.cholesky_runtime_scope():
            branch.VdnDelta().factor_apply(alpha.to(device), bad.to(device), b.to(device))


def test_factor_status_scopes_nest_and_validate_outside_a_scope(device):
    """Outside a scope a bad factor raises at once; an inner scope's failure leaves the outer scope's recorded
    statuses in place, and the outer scope validates them on exit (the reference's
    ``tests/test_cholesky.py`` nesting and immediate-check cases)."""
    from vdn_h3_amd import branch

    print("case factor status scopes", flush=True)
    frames, heads, dim, tokens = 2, 1, 64, 200
    kf = torch.nn.functional.normalize(_rand((frames, heads, tokens, dim), 14), dim=-1)
    a = (kf * 0.5).transpose(-1, -2) @ kf
    b = _rand((frames, heads, dim, dim), 15)
    alpha = torch.rand(frames, heads, dim, generator=torch.Generator().manual_seed(16))
    bad = a.clone()
    bad[0, 0] = -2.0 * torch.eye(dim)
    good = (alpha.to(device), a.to(device), b.to(device))
    invalid = (alpha.to(device), bad.to(device), b.to(device))
    with pytest.raises(torch.linalg.LinAlgError, match="leading minor of order 1"):
        branch.VdnDelta().factor_apply(*invalid)
    assert branch._CHOLESKY_CHECKS.get() is None
    with branch.cholesky_runtime_scope() as outer:
        branch.VdnDelta().factor_apply(*good)
        with pytest.raises(torch.linalg.LinAlgError):
            with branch.cholesky_runtime_scope() as inner:
                branch.VdnDelta().factor_apply(*invalid)
        assert branch._CHOLESKY_CHECKS.get() is outer
        assert len(outer.statuses) == 1 and outer.factor_calls == 1 and not inner.statuses
    assert branch._CHOLESKY_CHECKS.get() is None


@pytest.mark.parametrize("text", [False, True])
def test_scans(device, text):
    from vdn_h3_amd import branch

    print(f"case scans text={text}", flush=True)
    frames, heads, dim = 7, 2, 128
    phi = _rand((frames, heads, dim, dim), 8, 0.05)
    jay = _rand((frames, heads, dim, dim), 9)
    init = _rand((heads, dim, dim), 10) if text else torch.zeros(heads, dim, dim)
    p, s = branch.run_scans_from_factors(phi.to(device), jay.to(device), init.to(device) if text else None)
    wp, ws = bo.run_scans(phi, jay, init)
    _close(p, wp, 1e-4, 1e-5, "prefix")
    _close(s, ws, 1e-4, 1e-5, "suffix")


@pytest.mark.parametrize("text,bridge", [(False, "alpha"), (True, "alpha"), (True, "none")])
def test_readout_epilogue(device, text, bridge):
    from vdn_h3_amd import branch

    print(f"case readout text={text} bridge={bridge}", flush=True)
    frames, tokens, heads, dim = 11, 70, 2, 128
    bounds = [(lo - 1, hi - 1) for lo, hi in wo.window_bounds(frames + 2, 1, 5)[1:-1]]
    q = _rand((frames * tokens, heads, dim), 11, dtype=torch.bfloat16)
    prefix = _rand((frames, heads, dim, dim), 12, 0.1)
    suffix = _rand((frames, heads, dim, dim), 13, 0.1)
    alpha = torch.rand(frames, heads, dim, generator=torch.Generator().manual_seed(14)) * 0.5 + 0.5
    tstate = _rand((heads, dim, dim), 15, 0.1) if text else None
    gate = torch.sigmoid(_rand((frames * tokens, heads * dim), 16)).to(torch.bfloat16)
    norm_w = (1 + 0.1 * _rand((dim,), 17)).to(torch.bfloat16)
    got = branch.readout_epilogue(q.to(device), prefix.to(device), suffix.to(device), alpha.to(device), bounds,
                                  norm_w.to(device), gate.to(device),
                                  text_state=None if tstate is None else tstate.to(device), bridge=bridge,
                                  num_frames=frames, tokens_per_frame=tokens)
    qf = bo.to_fhsd(bo.activate(q, True), frames, heads, dim)
    state = bo.gather_linear_state(prefix, suffix, alpha, bounds, bridge=bridge, text_state=tstate,
                                   out_dtype=torch.bfloat16)
    want = bo.linear_epilogue(bo.bf16_matmul(qf, state.transpose(-1, -2)), norm_w, gate)
    _parity(got, want, "readout", atol=2e-2, min_cos=0.9999)
    _close(got, want, 4 * 2.0 ** -8, 4 * 2.0 ** -8, "readout")



@pytest.mark.parametrize("m,n,k,w_bf16,bias", [(29, 128, 5120, True, False), (29, 5120, 128, True, True),
                                               (5, 7, 1100, False, True), (1, 3, 64, False, False)])
def test_linear_f32(device, m, n, k, w_bf16, bias):
    """The fp32 alpha projections (vdnh3_linear_f32): both the long-K (split over a workgroup) and the
    short-K (one wavefront per column) kernels against a float64 product."""
    from vdn_h3_amd import branch

    print(f"case linear_f32 m={m} n={n} k={k}", flush=True)
    x = _rand((m, k), 41)
    w = _rand((n, k), 42, 0.05, torch.bfloat16 if w_bf16 else torch.float32)
    b = _rand((n,), 43) if bias else None
    got = branch.linear_f32(x.to(device), w.to(device), None if b is None else b.to(device))
    torch.cuda.synchronize()
    want = x.double() @ w.double().t() + (0 if b is None else b.double())
    err = (got.double().cpu() - want).abs().max().item()
    assert err <= 1e-5 * (1 + want.abs().max().item()), err

@pytest.mark.parametrize("dim,qf,bias", [(128, False, True), (128, True, False), (64, False, True)])
def test_readout_fused_gate_equals_gemm_then_readout(device, dim, qf, bias):
    """The output gate computed inside the readout kernel (vdnh3_readout_fused_gate) gives the same
    bits as the bf16 sigmoid GEMM (vdnh3_gemm) followed by vdnh3_readout."""
    from vdn_h3_amd import branch
    from vdn_h3_amd import linear as L

    print(f"case readout fused gate D={dim} q_features={qf} bias={bias}", flush=True)
    frames, tokens, heads = 5, 77, 3
    rows = frames * tokens
    bounds = [(lo - 1, hi - 1) for lo, hi in wo.window_bounds(frames + 2, 1, 5)[1:-1]]
    q = _rand((rows, heads, dim), 31, dtype=torch.bfloat16).to(device)
    prefix = _rand((frames, heads, dim, dim), 32, 0.1).to(device)
    suffix = _rand((frames, heads, dim, dim), 33, 0.1).to(device)
    alpha = (torch.rand(frames, heads, dim, generator=torch.Generator().manual_seed(34)) * 0.5 + 0.5).to(device)
    norm_w = (1 + 0.1 * _rand((dim,), 35)).to(torch.bfloat16).to(device)
    x = _rand((rows, 3 * dim), 36, dtype=torch.bfloat16).to(device)
    hidden = x[:, dim:2 * dim]                                   # a strided view, as in the branch
    w_up = _rand((heads * dim, dim), 37, 0.1, torch.bfloat16).to(device)
    b_up = _rand((heads * dim,), 38, 0.5, torch.bfloat16).to(device) if bias else None
    kw = dict(text_state=None, bridge="alpha", num_frames=frames, tokens_per_frame=tokens, q_features=qf)
    gate = L.sigmoid_linear(hidden, w_up, b_up)
    want = branch.readout_epilogue(q, prefix, suffix, alpha, bounds, norm_w, gate, **kw)
    got = branch.readout_epilogue(q, prefix, suffix, alpha, bounds, norm_w, None, gate_hidden=hidden,
                                  gate_up_weight=w_up, gate_up_bias=b_up, **kw)
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got.float() - want.float()).abs().max().item()


@pytest.mark.parametrize("dim,ks,kt,l2,grid,frames", [
    (128, 5, 5, True, (48, 27), 4), (128, 5, 5, False, (48, 27), 3), (128, 5, 5, True, (8, 8), 1),
    (64, 3, 3, True, (7, 5), 6), (64, 5, 3, False, (2, 2), 5), (128, 3, 5, True, (17, 40), 3)])
def test_short_conv_kernel(device, dim, ks, kt, l2, grid, frames):
    """vdnh3_short_conv vs the CUDA spelling of the oracle (bf16 spatial sum, fp32 temporal / SiLU / norm)."""
    from vdn_h3_amd import branch

    print(f"case short conv D={dim} k={ks}x{ks}x{kt} l2={l2} grid={grid} frames={frames}", flush=True)
    heads = 2
    gh, gw = grid
    rows, ch = frames * gh * gw, heads * dim
    fused = _rand((rows, 3 * ch), 60, dtype=torch.bfloat16)          # the kernel reads a strided q/k/v view
    x = fused[:, ch:2 * ch].reshape(rows, heads, dim)
    sp = _rand((ch, 1, ks, ks), 61, 0.2, torch.bfloat16)
    tm = _rand((ch, 1, kt), 62, 0.4, torch.bfloat16)
    dx = fused.to(device)[:, ch:2 * ch].view(rows, heads, dim)
    got = branch.conv_features(dx, sp.to(device), tm.to(device), frames, grid, l2)
    torch.cuda.synchronize()
    want = bo.conv_features_fused(x, sp, tm, frames, grid, l2)
    g32, w32 = got.float().cpu(), want.float()
    step = 2.0 ** -7 * w32.abs() + 2.0 ** -30
    assert ((g32 - w32).abs() <= step).all(), f"max err {(g32 - w32).abs().max().item():.3e}"
    exact = (g32 == w32).float().mean().item()
    assert exact >= 0.99, exact


def _load(name):
    with safe_open(str(GOLDEN / name), "pt") as f:
        return {k: f.get_tensor(k) for k in f.keys()}, f.metadata()


def test_projected_delta_matches_reference_golden(device):
    """The whole branch (13 frames of 8x8, 2 heads x 64, text state, anchors both) vs the reference."""
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print("case projected_delta golden", flush=True)
    t, meta = _load("branch_13f.safetensors")
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    gh, gw = map(int, meta["grid"].split("x"))
    tpf = gh * gw
    w = {k[2:]: v.to(device) for k, v in t.items() if k.startswith("w.")}
    x, qkv = t["x"].to(device), t["qkv"].to(device)
    seq = x.shape[0]
    q, k, v = [y.view(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    br = OptimizedLinearBranch(w, heads, dim, short_conv=(), enable_text_state=True)
    with torch.no_grad():
        got = br.projected_delta(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, frame_size=(gh, gw),
                                 text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
        readout = br.readout(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, text_x=x[:text],
                             text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    torch.cuda.synchronize()
    assert torch.count_nonzero(got[:tpf]) == 0 and torch.count_nonzero(got[-tpf:]) == 0
    _parity(got, t["delta"], "projected_delta vs reference")
    _parity(readout, t["readout"], "readout vs reference")



def test_short_conv_batch_equals_single_calls(device):
    """k (with the L2 norm) and v (without) convolved in one vdnh3_short_conv_batch launch give the
    same bits as two vdnh3_short_conv calls."""
    from vdn_h3_amd import branch

    print("case short conv batch", flush=True)
    frames, (gh, gw), heads, dim = 5, (12, 9), 3, 128
    rows, ch = frames * gh * gw, heads * dim
    fused = _rand((rows, 3 * ch), 70, dtype=torch.bfloat16).to(device)
    k = fused[:, ch:2 * ch].view(rows, heads, dim)
    v = fused[:, 2 * ch:].view(rows, heads, dim)
    w = [_rand((ch, 1, 5, 5), 71 + i, 0.2, torch.bfloat16).to(device) for i in range(2)]
    t = [_rand((ch, 1, 5), 73 + i, 0.4, torch.bfloat16).to(device) for i in range(2)]
    kb, vb = branch.conv_features_batch([(k, w[0], t[0], True, None), (v, w[1], t[1], False, None)], frames, (gh, gw))
    ks = branch.conv_features(k, w[0], t[0], frames, (gh, gw), True)
    vs = branch.conv_features(v, w[1], t[1], frames, (gh, gw), False)
    torch.cuda.synchronize()
    assert torch.equal(kb, ks) and torch.equal(vb, vs)

def test_projected_delta_short_conv_matches_reference_golden(device):
    """The branch with K/V short convolutions (13 frames of 8x8, 2 heads x 64) vs the reference."""
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print("case projected_delta short-conv golden", flush=True)
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
    with torch.no_grad():
        got = br.projected_delta(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, **kw)
        readout = br.readout(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, **kw)
        with pytest.raises(ValueError, match="short convolution requires frame_size"):
            br.readout(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, text_x=x[:text],
                       text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    torch.cuda.synchronize()
    assert torch.count_nonzero(got[:tpf]) == 0 and torch.count_nonzero(got[-tpf:]) == 0
    _parity(got, t["delta"], "short-conv projected_delta vs reference")
    # the readout is RMS-normalised (values up to ~6, where one bf16 step is 2^-5): compare it in
    # bf16 steps; the reference's golden used the eager (bf16) temporal sum, this path the fused one
    _parity(readout, t["readout"], "short-conv readout vs reference", atol=2 ** -4, min_cos=0.9999)
    _close(readout, t["readout"], 2.0 ** -6, 2e-2, "short-conv readout vs reference")


def test_projected_delta_qkv_short_conv(device):
    """Short convolutions on q, k and v (any subset is a valid checkpoint config) vs the oracle."""
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print("case projected_delta q/k/v short conv", flush=True)
    frames, (gh, gw), text, heads, dim, hidden = 12, (6, 10), 24, 2, 128, 256
    tpf = gh * gw
    seq = text + frames * tpf
    gen = {"beta_proj.weight": (heads, hidden), "alpha.down.weight": (dim, hidden),
           "alpha.up.weight": (heads * dim, dim), "output_gate.down.weight": (dim, hidden),
           "output_gate.up.weight": (heads * dim, dim), "to_out_linear.weight": (hidden, heads * dim)}
    w = {name: _rand(shape, 70 + i, 0.02, torch.bfloat16) for i, (name, shape) in enumerate(gen.items())}
    w["alpha.dt_bias"] = _rand((heads * dim,), 80, 0.5)
    w["alpha.A_log"] = _rand((heads,), 81, 0.5)
    w["output_gate.up.bias"] = _rand((heads * dim,), 82, 0.5, torch.bfloat16)
    w["norm.weight"] = (1 + 0.1 * _rand((dim,), 83)).to(torch.bfloat16)
    for i, name in enumerate("qkv"):
        w[f"short_conv.{name}_sp.weight"] = _rand((heads * dim, 1, 5, 5), 84 + i, 0.2, torch.bfloat16)
        w[f"short_conv.{name}_tm.weight"] = _rand((heads * dim, 1, 5), 87 + i, 0.4, torch.bfloat16)
    x = _rand((seq, hidden), 90, dtype=torch.bfloat16)
    qkv = _rand((seq, 3 * heads * dim), 91, dtype=torch.bfloat16)
    q, k, v = [y.reshape(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    kw = dict(frame_size=(gh, gw), text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    want = bo.projected_delta(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds,
                              short_conv=("q", "k", "v"), fused_conv=True, **kw)
    dw = {name: t.to(device) for name, t in w.items()}
    dx, dqkv = x.to(device), qkv.to(device)
    dq, dk, dv = [y.view(seq, heads, dim) for y in dqkv.split(heads * dim, dim=-1)]
    br = OptimizedLinearBranch(dw, heads, dim, short_conv=("q", "k", "v"), enable_text_state=True)
    dkw = dict(frame_size=(gh, gw), text_x=dx[:text], text_k_raw=dk[:text], text_v_raw=dv[:text], skip_ends=True)
    with torch.no_grad():
        got = br.projected_delta(dw, dx[text:], dq[text:], dk[text:], dv[text:], frames, tpf, bounds, **dkw)
    torch.cuda.synchronize()
    _parity(got, want, "q/k/v short-conv projected_delta vs oracle")


def test_full_shape_branch(device):
    """31 frames x 1296 tokens x 40 heads x 128 (29 inner frames after skip_ends), 512 text rows.

    The oracle runs the whole branch on the CPU. The readout (RMS-normalised, values up to ~6) is
    compared element-wise: at most 0.5% of values more than two bf16 ulps of the oracle value off and
    0.15% more than eight, every value within eight ulps of max(|v|, 1), cosine >= 0.9999; the isolation
    check below pins the path after the statistics tighter. The projected delta (O(1) values) at sampled
    rows against the absolute bar (max-abs 2e-2, cosine >= 0.9995).
    """
    from vdn_h3_amd import synth
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print("case full-shape branch", flush=True)
    frames, tpf, text, heads, dim, hidden = 31, 1296, 512, 40, 128, 5120
    seq = text + frames * tpf
    qkv = synth.randn((seq, 3 * heads * dim), 40, device=device, dtype=torch.bfloat16)
    x = synth.randn((seq, hidden), 41, device=device, dtype=torch.bfloat16)
    w = {
        "beta_proj.weight": synth.randn((heads, hidden), 42, device=device, dtype=torch.bfloat16, scale=0.02),
        "alpha.down.weight": synth.randn((dim, hidden), 43, device=device, dtype=torch.bfloat16, scale=0.02),
        "alpha.up.weight": synth.randn((heads * dim, dim), 44, device=device, dtype=torch.bfloat16, scale=0.02),
        "alpha.dt_bias": synth.randn((heads * dim,), 45, device=device, scale=0.5),
        "alpha.A_log": synth.randn((heads,), 46, device=device, scale=0.5),
        "output_gate.down.weight": synth.randn((dim, hidden), 47, device=device, dtype=torch.bfloat16, scale=0.02),
        "output_gate.up.weight": synth.randn((heads * dim, dim), 48, device=device, dtype=torch.bfloat16, scale=0.02),
        "output_gate.up.bias": synth.randn((heads * dim,), 49, device=device, dtype=torch.bfloat16, scale=0.5),
        "norm.weight": (1 + 0.1 * synth.randn((dim,), 50, device=device)).to(torch.bfloat16),
        "to_out_linear.weight": synth.randn((hidden, heads * dim), 51, device=device, dtype=torch.bfloat16,
                                            scale=0.02),
    }
    q, k, v = synth.split_qkv(qkv, heads, dim)
    bounds = wo.window_bounds(frames, 1, 5)
    br = OptimizedLinearBranch(w, heads, dim)
    va = text
    kw = dict(text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    with torch.no_grad():
        readout = br.readout(w, x[va:], q[va:], k[va:], v[va:], frames, tpf, bounds, **kw)
        delta = br.projected_delta(w, x[va:], q[va:], k[va:], v[va:], frames, tpf, bounds, **kw)
    torch.cuda.synchronize()
    readout, delta = readout.cpu(), delta.cpu()
    hq, hk, hv = synth.split_qkv(qkv.cpu(), heads, dim)
    hx = x.cpu()
    hw = {kk: vv.cpu() for kk, vv in w.items()}
    inner = slice(va + tpf, va + (frames - 1) * tpf)
    ibounds = [(lo - 1, hi - 1) for lo, hi in bounds[1:-1]]
    torch.set_num_threads(16)
    want = bo.readout(hw, hx[inner], hq[inner], hk[inner], hv[inner], frames - 2, tpf, ibounds,
                      text_x=hx[:text], text_k_raw=hk[:text], text_v_raw=hv[:text])
    got = readout[tpf:-tpf]
    g32, w32 = got.float(), want.float()
    ulp = torch.ldexp(torch.ones_like(w32), torch.frexp(w32)[1] - 8).clamp_min(2.0 ** -133)
    steps = (g32 - w32).abs() / ulp                                   # error in bf16 ulps of the oracle value
    small = w32.abs() < 2
    err_small = (g32 - w32).abs()[small].max().item()
    cos = torch.nn.functional.cosine_similarity(g32.double().flatten(), w32.double().flatten(), dim=0).item()
    rows = torch.arange(0, 37584, 64)
    want_delta = bo.linear_bf16(want[rows], hw["to_out_linear.weight"])
    steps1 = (g32 - w32).abs() / torch.maximum(ulp, torch.full_like(ulp, 2.0 ** -7))
    print(f"readout: ulps of max(|v|, 1): max {steps1.max().item():.1f}, frac > 2 {(steps1 > 2).float().mean():.2e}, "
          f"frac > 8 {(steps1 > 8).float().mean():.2e}", flush=True)
    print(f"readout: cosine {cos:.7f}, ulps: max {steps.max().item():.1f}, frac > 2 {(steps > 2).float().mean():.2e}, "
          f"frac > 4 {(steps > 4).float().mean():.2e}, frac > 8 {(steps > 8).float().mean():.2e}; "
          f"max abs where |want| < 2: {err_small:.3e}; max |want| {w32.abs().max().item():.2f}", flush=True)
    # B is rounded to bf16 (the reference's bf16 matmul output): where the fp32 sums of the two
    # paths straddle a rounding boundary, B moves by one bf16 step and J = B M carries it into
    # the state, so a small fraction of readout values differ by more than the local rounding.
    assert cos >= 0.9999, cos
    assert (steps > 2).float().mean().item() <= 5e-3
    assert (steps > 8).float().mean().item() <= 1.5e-3
    # every value within 8 ulps of max(|v|, 1): the values far off in their own ulps lie near zero
    assert steps1.max().item() <= 8
    assert torch.count_nonzero(readout[:tpf]) == 0 and torch.count_nonzero(readout[-tpf:]) == 0
    _parity(delta[tpf:-tpf][rows], want_delta, "full-shape projected delta")
    assert torch.count_nonzero(delta[:tpf]) == 0 and torch.count_nonzero(delta[-tpf:]) == 0

    # The tail above comes from the bf16 roundings before the factor: B (the reference's bf16 matmul
    # output), beta and the gate's down-projection, whose fp32 sums differ in summation order between the
    # two paths and so round differently where they straddle a bf16 midpoint. With the GPU's own A, B (video
    # and text rows) and gate down-projection handed to the oracle, everything after them - alpha, factor,
    # scans, gather, readout, RMSNorm and the gate - is held to <= 2 ulps for 99.9% of values, <= 8 ulps where
    # |value| >= 2 and max-abs 2^-5 (4 ulps at 1) where |value| < 2: the bf16 cast of the gathered state and
    # of the readout r still round in both paths, and a one-ulp flip of r in a row whose RMS is small moves the
    # normalised value by a few of its ulps.
    from vdn_h3_amd import branch
    from vdn_h3_amd import linear as lin

    inner_rows = slice(va + tpf, va + (frames - 1) * tpf)
    with torch.no_grad():
        both = lin.sigmoid_linear_split(x[inner_rows], torch.cat([w["beta_proj.weight"],
                                                                   w["output_gate.down.weight"]]).contiguous(), heads)
        a, b = branch.frame_statistics_raw(k[inner_rows], v[inner_rows], both[:, :heads], frames - 2, tpf)
        at, bt = branch.frame_statistics_raw(k[:text], v[:text], lin.sigmoid_linear(x[:text], w["beta_proj.weight"]),
                                             1, text)
    torch.cuda.synchronize()
    iso = bo.readout(hw, hx[inner], hq[inner], hk[inner], hv[inner], frames - 2, tpf, ibounds, text_x=hx[:text],
                     text_k_raw=hk[:text], text_v_raw=hv[:text], stats=(a.cpu(), b.cpu()),
                     text_stats=(at.cpu(), bt.cpu()), gate_hidden=both[:, heads:].cpu()).float()
    isteps = (g32 - iso).abs() / torch.ldexp(torch.ones_like(iso), torch.frexp(iso)[1] - 8).clamp_min(2.0 ** -133)
    ismall = (g32 - iso).abs()[iso.abs() < 2].max().item()
    print(f"readout after the GPU's statistics: ulps max {isteps.max().item():.1f}, frac > 2 "
          f"{(isteps > 2).float().mean():.2e}, frac > 4 {(isteps > 4).float().mean():.2e}; max abs where "
          f"|value| < 2: {ismall:.3e}", flush=True)
    big = iso.abs() >= 2
    assert (isteps <= 2).float().mean().item() >= 0.999
    assert not bool(big.any()) or isteps[big].max().item() <= 8
    assert ismall <= 2.0 ** -5


@pytest.mark.parametrize("dim,alpha_ones", [(128, False), (64, False), (128, True)])
def test_sana_factor(device, dim, alpha_ones):
    """SanaDelta.factor_apply (vdnh3_sana_factor) against the oracle's torch formula: the same fp32
    products and differences, so bit-identical; the text state's 1/2 and alpha = None (ones) included."""
    from vdn_h3_amd import branch

    print(f"case sana factor D={dim} alpha_ones={alpha_ones}", flush=True)
    frames, heads, tokens = 3, 2, 1296
    kf = torch.nn.functional.normalize(_rand((frames, heads, 200, dim), 60), dim=-1)
    a = kf.transpose(-1, -2) @ kf
    b = _rand((frames, heads, dim, dim), 61)
    alpha = torch.ones(frames, heads, dim) if alpha_ones else torch.rand(frames, heads, dim,
                                                                         generator=torch.Generator().manual_seed(62))
    backend = branch.SanaDelta(tokens)
    phi, jay = backend.factor_apply(None if alpha_ones else alpha.to(device), a.to(device), b.to(device))
    wphi, wjay = bo.sana_factor(alpha, a, b, tokens)
    assert torch.equal(phi.cpu(), wphi) and torch.equal(jay.cpu(), wjay)
    none_phi, half = backend.factor_apply(None, a.to(device), b.to(device), jay_scale=0.5, need_phi=False)
    assert none_phi is None and torch.equal(half.cpu(), 0.5 * wjay)
    with pytest.raises(ValueError, match="alpha"):
        backend.factor_apply(alpha[:, :, :-1].to(device), a.to(device), b.to(device))


def test_projected_delta_a_bf16_matches_reference_golden(device):
    """The branch with a_fp32=False (13 frames of 8x8, 2 heads x 64, text state) vs the reference's own output
    and vs the oracle; the text state's statistics take the same flag."""
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print("case projected_delta a_fp32=False golden", flush=True)
    t, meta = _load("branch_13f_abf16.safetensors")
    assert meta["a_fp32"] == "false"
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    gh, gw = map(int, meta["grid"].split("x"))
    tpf = gh * gw
    w = {k[2:]: v.to(device) for k, v in t.items() if k.startswith("w.")}
    x, qkv = t["x"].to(device), t["qkv"].to(device)
    seq = x.shape[0]
    q, k, v = [y.view(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    br = OptimizedLinearBranch(w, heads, dim, a_fp32=False, short_conv=(), enable_text_state=True)
    kw = dict(frame_size=(gh, gw), text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    with torch.no_grad():
        got = br.projected_delta(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, **kw)
        readout = br.readout(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, **kw)
    torch.cuda.synchronize()
    assert torch.count_nonzero(got[:tpf]) == 0 and torch.count_nonzero(got[-tpf:]) == 0
    _parity(got, t["delta"], "a_fp32=False projected_delta vs reference")
    _parity(readout, t["readout"], "a_fp32=False readout vs reference", atol=2 ** -5, min_cos=0.9999)
    hw = {k2[2:]: v2 for k2, v2 in t.items() if k2.startswith("w.")}
    hq, hk, hv = [y.reshape(seq, heads, dim) for y in t["qkv"].split(heads * dim, dim=-1)]
    hx = t["x"]
    want = bo.projected_delta(hw, hx[text:], hq[text:], hk[text:], hv[text:], frames, tpf, bounds, frame_size=(gh, gw),
                              text_x=hx[:text], text_k_raw=hk[:text], text_v_raw=hv[:text], skip_ends=True,
                              a_fp32=False)
    _parity(got, want, "a_fp32=False projected_delta vs oracle")


def test_projected_delta_sana_matches_reference_golden(device):
    """The branch with delta_rule='sana_scaled' (13 frames of 8x8, 2 heads x 64, text state) vs the
    reference's own output and vs the oracle."""
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    print("case projected_delta sana golden", flush=True)
    t, meta = _load("branch_13f_sana.safetensors")
    assert meta["delta_rule"] == "sana_scaled"
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    gh, gw = map(int, meta["grid"].split("x"))
    tpf = gh * gw
    w = {k[2:]: v.to(device) for k, v in t.items() if k.startswith("w.")}
    x, qkv = t["x"].to(device), t["qkv"].to(device)
    seq = x.shape[0]
    q, k, v = [y.view(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    br = OptimizedLinearBranch(w, heads, dim, delta_rule="sana_scaled", short_conv=(), enable_text_state=True)
    kw = dict(frame_size=(gh, gw), text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    with torch.no_grad():
        got = br.projected_delta(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, **kw)
        readout = br.readout(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, **kw)
    torch.cuda.synchronize()
    assert torch.count_nonzero(got[:tpf]) == 0 and torch.count_nonzero(got[-tpf:]) == 0
    _parity(got, t["delta"], "sana projected_delta vs reference")
    _parity(readout, t["readout"], "sana readout vs reference", atol=2 ** -5, min_cos=0.9999)
    hw = {k2[2:]: v2 for k2, v2 in t.items() if k2.startswith("w.")}
    hq, hk, hv = [y.reshape(seq, heads, dim) for y in t["qkv"].split(heads * dim, dim=-1)]
    hx = t["x"]
    want = bo.projected_delta(hw, hx[text:], hq[text:], hk[text:], hv[text:], frames, tpf, bounds, frame_size=(gh, gw),
                              text_x=hx[:text], text_k_raw=hk[:text], text_v_raw=hv[:text], skip_ends=True,
                              delta_rule="sana_scaled")
    _parity(got, want, "sana projected_delta vs oracle")
