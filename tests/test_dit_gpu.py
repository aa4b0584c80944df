"""Parity of the DiT block pointwise kernels and the fused block forward with the oracle (GPU).

The pointwise passes follow the reference's bf16 ops, so they are compared element by element
(bit-exact where every input of an op is exact, otherwise within one bf16 step where the fp32
statistics of the RMSNorm or the exponential of SiLU may round a midpoint differently); the
whole block against the block parity bar (max-abs 2e-2, cosine >= 0.9995).
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle import branch_oracle as bo
from oracle import dit_oracle as do
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu


def _steps(got, want):
    g, w = got.float().cpu(), want.float()
    ulp = torch.ldexp(torch.ones_like(w), torch.frexp(w)[1] - 8).clamp_min(2.0 ** -133)
    return (g - w).abs() / ulp


def _steps_mag(got, want, mag):
    """|got - want| in ulps (bf16, 8 significant bits) of ``mag``."""
    g, w = got.float().cpu(), want.float()
    ulp = torch.ldexp(torch.ones_like(mag), torch.frexp(mag)[1] - 8).clamp_min(2.0 ** -133)
    return (g - w).abs() / ulp


def _case(rows, hidden, n_mod, seed, mod_dtype):
    g = torch.Generator().manual_seed(seed)
    x = (2 * torch.randn(rows, hidden, generator=g)).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)
    scale = (0.3 * torch.randn(n_mod, hidden, generator=g)).to(mod_dtype)
    shift = (0.3 * torch.randn(n_mod, hidden, generator=g)).to(mod_dtype)
    idx = torch.randint(0, n_mod, (rows,), generator=g)
    return x, w, scale, shift, idx


@pytest.mark.parametrize("hidden,mod_dtype", [(5120, torch.float32), (192, torch.bfloat16), (8192, torch.float32)])
def test_rmsnorm_modulate(device, hidden, mod_dtype):
    from vdn_h3_amd import block_kernels as bk

    print(f"case rmsnorm_modulate hidden={hidden} {mod_dtype}", flush=True)
    x, w, scale, shift, idx = _case(300, hidden, 3, 1, mod_dtype)
    got = bk.rmsnorm_modulate(x.to(device), w.to(device), 1e-6, scale.to(device), shift.to(device),
                              idx.to(torch.int32).to(device))
    want = do.pre(x, w, 1e-6, scale, shift, idx)
    # The result is p + shift with p = bf16(rms_norm(x) * (1 + scale)). The fp32 sum of squares depends
    # on the summation order (torch's CPU kernel and the GPU's wavefront tree differ), which can move p
    # by one of its own ulps; where p + shift cancels, that is many ulps of the result. So the steps are
    # counted in ulps of max(|result|, |p|).
    prod = do.pre(x, w, 1e-6, scale, torch.zeros_like(shift), idx)
    steps = _steps_mag(got, want, torch.maximum(want.float().abs(), prod.float().abs()))
    print(f"  steps > 0: {(steps > 0).sum().item()} of {steps.numel()}, max {steps.max().item()}", flush=True)
    assert steps.max().item() <= 2, steps.max().item()
    assert (steps == 0).float().mean().item() >= 0.99


@pytest.mark.parametrize("rows,hidden,pattern", [(4001, 192, "random"), (40688, 5120, "runs")])
def test_rmsnorm_modulate_multi_row_walk(device, rows, hidden, pattern):
    """More than 768 rows: each of the kernel's workgroups walks a block of consecutive rows (4001 rows: 6
    per workgroup, 667 workgroups; 40,688: 53 per workgroup, 768 workgroups; both end in an odd-length
    last block), with two x buffers in flight, alternating reduction slots, and the segment's bf16(1 +
    scale) and shift cached in registers and reloaded where the index changes inside a block ("random":
    a new segment on most rows; "runs": segments of 37 rows, so most blocks keep theirs). Against the oracle
    with the one-row bar, and bit for bit against the same rows run in slices of at most 768 rows, where
    every workgroup takes a single row."""
    from vdn_h3_amd import block_kernels as bk

    print(f"case rmsnorm_modulate multi-row rows={rows} hidden={hidden} {pattern}", flush=True)
    x, w, scale, shift, idx = _case(rows, hidden, 3, 11, torch.float32)
    if pattern == "runs":
        g = torch.Generator().manual_seed(12)
        idx = torch.randint(0, 3, ((rows + 36) // 37,), generator=g).repeat_interleave(37)[:rows]
    dx, dw, dsc, dsh = x.to(device), w.to(device), scale.to(device), shift.to(device)
    didx = idx.to(torch.int32).to(device)
    got = bk.rmsnorm_modulate(dx, dw, 1e-6, dsc, dsh, didx)
    parts = [bk.rmsnorm_modulate(dx[i:i + 768], dw, 1e-6, dsc, dsh, didx[i:i + 768]) for i in range(0, rows, 768)]
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.cat(parts).cpu())
    want = do.pre(x, w, 1e-6, scale, shift, idx)
    prod = do.pre(x, w, 1e-6, scale, torch.zeros_like(shift), idx)
    steps = _steps_mag(got, want, torch.maximum(want.float().abs(), prod.float().abs()))
    print(f"  steps > 0: {(steps > 0).sum().item()} of {steps.numel()}, max {steps.max().item()}", flush=True)
    assert steps.max().item() <= 2, steps.max().item()
    assert (steps == 0).float().mean().item() >= 0.99


def test_out_of_range_device_index_gives_nan_rows(device):
    """A modulation index held in a device tensor is not range-checked on the host; an index outside the
    table (2 and -1 for a 2-row table) makes both passes read row 0 and write NaN for exactly those rows,
    in the single-row and the multi-row walk of rmsnorm_modulate; every other row equals the oracle."""
    from vdn_h3_amd import block_kernels as bk

    print("case out-of-range device modulation index", flush=True)
    for rows in (300, 2000):
        x, w, scale, shift, idx = _case(rows, 256, 2, 13, torch.float32)
        bad = torch.zeros(rows, dtype=torch.bool)
        bad[[3, 4, rows // 2, rows - 1]] = True
        dev_idx = idx.clone()
        dev_idx[[3, rows // 2]] = 2
        dev_idx[[4, rows - 1]] = -1
        didx = dev_idx.to(torch.int32).to(device)
        got = bk.rmsnorm_modulate(x.to(device), w.to(device), 1e-6, scale.to(device), shift.to(device), didx).cpu()
        want = do.pre(x, w, 1e-6, scale, shift, idx)
        assert bool(torch.isnan(got[bad].float()).all())
        good = ~bad
        assert not bool(torch.isnan(got[good].float()).any())
        prod = do.pre(x, w, 1e-6, scale, torch.zeros_like(shift), idx)
        steps = _steps_mag(got[good], want[good], torch.maximum(want[good].float().abs(), prod[good].float().abs()))
        assert steps.max().item() <= 2
        b = torch.randn(x.shape, generator=torch.Generator().manual_seed(14)).to(torch.bfloat16)
        got_r = bk.gated_residual(x.to(device), scale.to(device), didx, b.to(device)).cpu()
        want_r = do.post(x, scale, idx, b)
        assert bool(torch.isnan(got_r[bad].float()).all())
        assert torch.equal(got_r[good], want_r[good])
        with pytest.raises(ValueError, match="out of range"):  # a host tensor is checked before the launch
            bk.rmsnorm_modulate(x.to(device), w.to(device), 1e-6, scale.to(device), shift.to(device), dev_idx)


@pytest.mark.parametrize("gate_dtype", [torch.float32, torch.bfloat16])
def test_gated_residual(device, gate_dtype):
    from vdn_h3_amd import block_kernels as bk

    print(f"case gated_residual {gate_dtype}", flush=True)
    x, _, gate, _, idx = _case(257, 5120, 4, 2, gate_dtype)
    b = torch.randn(x.shape, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    want = do.post(x, gate, idx, b)
    dx = x.to(device)
    got = bk.gated_residual(dx, gate.to(device), idx.to(torch.int32).to(device), b.to(device))
    assert torch.equal(got.cpu(), want)
    bk.gated_residual(dx, gate.to(device), idx.to(torch.int32).to(device), b.to(device), out=dx)  # in place
    assert torch.equal(dx.cpu(), want)


def test_swiglu_and_fused_quantisation(device):
    from vdn_h3_amd import block_kernels as bk
    from vdn_h3_amd import linear

    print("case swiglu + quantisation", flush=True)
    h = (3 * torch.randn(333, 2 * 1040, generator=torch.Generator().manual_seed(4))).to(torch.bfloat16)
    dh = h.to(device)
    got = bk.swiglu(dh)
    steps = _steps(got, do.swiglu(h))
    assert steps.max().item() <= 1 and (steps == 0).float().mean().item() >= 0.999
    for kind in (linear.KIND_I8, linear.KIND_F8):
        q, s = bk.swiglu_quantize_rows(dh, kind)
        q2, s2 = linear.quantize_rows(got, kind)
        assert torch.equal(q.view(torch.uint8).cpu(), q2.view(torch.uint8).cpu()) and torch.equal(s.cpu(), s2.cpu())
    wq, ws = qo.int8_quantize_rows(got.cpu())
    q, s = bk.swiglu_quantize_rows(dh, linear.KIND_I8)
    assert torch.equal(q.cpu(), wq) and torch.equal(s.cpu().reshape(-1), ws.reshape(-1))


@pytest.mark.parametrize("ffn", [13824, 16384, 16392])
def test_fused_quantisation_wide_rows(device, ffn):
    """One workgroup per row up to ffn 16,384 (the row kept in registers), one wavefront per row with a
    second sweep beyond it: both give the codes and scales of quantising the SwiGLU output."""
    from vdn_h3_amd import block_kernels as bk
    from vdn_h3_amd import linear

    print(f"case swiglu quantisation ffn={ffn}", flush=True)
    h = (3 * torch.randn(37, 2 * ffn, generator=torch.Generator().manual_seed(ffn))).to(torch.bfloat16)
    dh = h.to(device)
    a = bk.swiglu(dh)
    for kind in (linear.KIND_I8, linear.KIND_F8):
        q, s = bk.swiglu_quantize_rows(dh, kind)
        q2, s2 = linear.quantize_rows(a, kind)
        assert torch.equal(q.view(torch.uint8).cpu(), q2.view(torch.uint8).cpu()) and torch.equal(s.cpu(), s2.cpu())
    wq, ws = qo.int8_quantize_rows(a.cpu())
    q, s = bk.swiglu_quantize_rows(dh, linear.KIND_I8)
    assert torch.equal(q.cpu(), wq) and torch.equal(s.cpu().reshape(-1), ws.reshape(-1))


def _block(hidden, ffn, heads, device, precision, seed=5):
    from vdn_h3_amd.diagnostics import DiagnosticsRecorder
    from vdn_h3_amd.linear import HipLinear

    g = torch.Generator().manual_seed(seed)
    w = {"attn": (0.05 * torch.randn(hidden, hidden, generator=g)).to(torch.bfloat16),
         "fc1": (0.05 * torch.randn(2 * ffn, hidden, generator=g)).to(torch.bfloat16),
         "fc2": (0.05 * torch.randn(hidden, ffn, generator=g)).to(torch.bfloat16),
         "norm1": (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16),
         "norm2": (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16)}
    mod = tuple(0.3 * torch.randn(2, hidden, generator=g) for _ in range(6))
    attn_lin = HipLinear(w["attn"].to(device), "bf16")
    calls = []

    def attn(h, rope_freqs=None, transformer_options=None):
        calls.append(rope_freqs)
        return attn_lin(h)

    block = SimpleNamespace(
        norm1=SimpleNamespace(weight=w["norm1"].to(device), eps=1e-6),
        norm2=SimpleNamespace(weight=w["norm2"].to(device), eps=1e-6),
        adaln_proj=lambda t_emb: tuple(m.to(device) for m in mod),
        attn=attn,
        mlp=SimpleNamespace(fc1=HipLinear(w["fc1"].to(device), "bf16"), fc2=HipLinear(w["fc2"].to(device), precision)),
        forward=lambda *a, **k: "original")
    state = SimpleNamespace(block_fusion=True, inference=True, weight_mode="resident",
                            diagnostics=DiagnosticsRecorder(False))
    return block, state, w, mod, calls


@pytest.mark.parametrize("precision", ["bf16", "int8"])
def test_fast_block_forward_vs_oracle(device, precision):
    from vdn_h3_amd.block_kernels import make_fast_block_forward

    print(f"case fast block forward fc2={precision}", flush=True)
    hidden, ffn, rows = 512, 1024, 300
    block, state, w, mod, calls = _block(hidden, ffn, 4, device, precision)
    x = torch.randn(rows, hidden, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    segments = [(0, 40, 0), (40, rows, 1)]
    forward = make_fast_block_forward(block, state, 0)
    with torch.no_grad():
        got = forward(x.to(device), torch.zeros(1), segments, "freqs")
    torch.cuda.synchronize()
    assert calls == ["freqs"]

    def fc2(a):
        if precision == "bf16":
            return bo.linear_bf16(a, w["fc2"])
        wq, ws = qo.int8_quantize_rows(w["fc2"])
        return qo.int8_linear(*qo.int8_quantize_rows(a), wq, ws.reshape(1, -1))

    want = do.block_forward(x, mod, segments, w["norm1"], w["norm2"], lambda h: bo.linear_bf16(h, w["attn"]),
                            lambda h: bo.linear_bf16(h, w["fc1"]), fc2)
    g32, w32 = got.float().cpu(), want.float()
    err = (g32 - w32).abs().max().item()
    cos = F.cosine_similarity(g32.flatten().double(), w32.flatten().double(), dim=0).item()
    print(f"fast block {precision}: max abs {err:.3e}, cosine {cos:.7f}", flush=True)
    # max-abs 2e-2, or one bf16 step of the largest output where that step is coarser
    assert err <= max(2e-2, w32.abs().max().item() * 2.0 ** -7) and cos >= 0.9995
    # the reference's fallbacks: an explicit attention callable, or fusion switched off
    assert forward(x.to(device), torch.zeros(1), segments, None, attention=object()) == "original"
    state.block_fusion = False
    assert forward(x.to(device), torch.zeros(1), segments, None) == "original"


def test_fast_block_forward_matches_reference_golden(device):
    """make_fast_block_forward on the GPU against the reference's own make_fast_block_forward output
    (tests/golden/dit_block.safetensors: two modulation segments, bf16 attention stand-in and SwiGLU MLP).
    Error in bf16 ulps of the reference value: <= 2 ulps for >= 99.9% of values, <= 4 at most, and
    max-abs 2e-2 where |value| < 2."""
    from safetensors import safe_open

    from vdn_h3_amd.block_kernels import make_fast_block_forward
    from vdn_h3_amd.diagnostics import DiagnosticsRecorder
    from vdn_h3_amd.linear import HipLinear

    print("case fast block forward vs reference golden", flush=True)
    from pathlib import Path

    with safe_open(str(Path(__file__).resolve().parent / "golden" / "dit_block.safetensors"), "pt") as f:
        t = {k: f.get_tensor(k) for k in f.keys()}
    names = ("shift_msa", "scale_msa", "gate_msa", "shift_mlp", "scale_mlp", "gate_mlp")
    attn_lin = HipLinear(t["w.attn.weight"].to(device), "bf16")
    block = SimpleNamespace(
        norm1=SimpleNamespace(weight=t["w.norm1.weight"].to(device), eps=1e-6),
        norm2=SimpleNamespace(weight=t["w.norm2.weight"].to(device), eps=1e-6),
        adaln_proj=lambda t_emb: tuple(t[f"mod.{n}"].to(device) for n in names),
        attn=lambda h, rope_freqs=None, transformer_options=None: attn_lin(h),
        mlp=SimpleNamespace(fc1=HipLinear(t["w.fc1.weight"].to(device), "bf16"),
                            fc2=HipLinear(t["w.fc2.weight"].to(device), "bf16")),
        forward=lambda *a, **k: "original")
    state = SimpleNamespace(block_fusion=True, inference=True, weight_mode="resident",
                            diagnostics=DiagnosticsRecorder(False))
    forward = make_fast_block_forward(block, state, 0)
    segments = [(0, 40, 0), (40, t["x"].shape[0], torch.tensor(1))]
    with torch.no_grad():
        got = forward(t["x"].to(device), torch.zeros(1), segments, None)
    torch.cuda.synchronize()
    want = t["out"].float()
    steps = _steps(got, want)
    err = (got.float().cpu() - want).abs()
    print(f"  ulps: max {steps.max().item():.1f}, > 2: {(steps > 2).float().mean().item():.2e}", flush=True)
    assert (steps <= 2).float().mean().item() >= 0.999 and steps.max().item() <= 4
    assert err[want.abs() < 2].max().item() <= 2e-2
