"""Pins the branch oracle: closed forms per function (the reference's own test strategy,
``tests/test_branch.py``), and the composites against golden vectors written from the
reference (``tests/golden/make_golden.py``)."""

from __future__ import annotations

from pathlib import Path

import pytest
import torch
import torch.nn.functional as F
from safetensors import safe_open

from oracle import branch_oracle as bo
from oracle import window_oracle as wo

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_vdn_factor_matches_inverse_closed_form():
    # tests/test_branch.py:11-23
    torch.manual_seed(1)
    frames, heads, dim, tokens = 4, 2, 5, 7
    key = torch.randn(frames, heads, tokens, dim)
    beta = torch.rand(frames, heads, tokens)
    a = (key * beta.unsqueeze(-1)).transpose(-1, -2) @ key
    b = torch.randn(frames, heads, dim, dim)
    alpha = torch.rand(frames, heads, dim)
    phi, jay, info = bo.vdn_factor(alpha, a, b)
    inv = torch.linalg.inv(torch.eye(dim).expand_as(a) + a)
    torch.testing.assert_close(phi, alpha.unsqueeze(-1) * inv, atol=3e-5, rtol=3e-5)
    torch.testing.assert_close(jay, b @ inv, atol=3e-5, rtol=3e-5)
    assert int(info.abs().sum()) == 0


def test_vdn_factor_reports_first_failing_minor():
    # tests/test_cholesky.py:57-69: a -2*I block makes I + A indefinite
    a = torch.zeros(3, 2, 4, 4)
    a[1, 0] = -2.0 * torch.eye(4)
    _, _, info = bo.vdn_factor(torch.ones(3, 2, 4), a, torch.zeros_like(a))
    assert info.tolist() == [[0, 0], [1, 0], [0, 0]]


def test_frame_statistics_equations_and_bf16_rounding():
    # tests/test_branch.py:26-36 (fp32), then the bf16 model's B rounding
    torch.manual_seed(2)
    key = torch.randn(3, 2, 6, 4)
    value = torch.randn_like(key)
    beta = torch.rand(3, 2, 6)
    a, b = bo.frame_statistics(key, value, beta)
    torch.testing.assert_close(a, torch.einsum("fhsk,fhsl,fhs->fhkl", key, key, beta))
    torch.testing.assert_close(b, torch.einsum("fhsv,fhsk,fhs->fhvk", value, key, beta))
    torch.testing.assert_close(a, a.transpose(-1, -2))
    k16, v16 = key.to(torch.bfloat16), value.to(torch.bfloat16)
    a16, b16 = bo.frame_statistics(k16, v16, beta)
    vb = (v16 * beta.to(torch.bfloat16).unsqueeze(-1)).float()
    want_b = torch.einsum("fhsv,fhsk->fhvk", vb.double(), k16.double()).to(torch.bfloat16).float()
    torch.testing.assert_close(b16, want_b, atol=0, rtol=0)
    torch.testing.assert_close(a16, torch.einsum("fhsk,fhsl,fhs->fhkl", k16.float(), k16.float(), beta),
                               atol=1e-5, rtol=1e-5)


def test_scans_match_naive_recurrence():
    # tests/test_branch.py:51-76
    torch.manual_seed(3)
    frames, heads, dim = 5, 2, 4
    alpha = torch.rand(frames, heads, dim) * 0.5 + 0.25
    feats = torch.randn(frames, heads, 6, dim)
    a = feats.transpose(-1, -2) @ feats
    b = torch.randn(frames, heads, dim, dim)
    text = torch.randn(heads, dim, dim)
    phi, jay, _ = bo.vdn_factor(alpha, a, b)
    fwd, bwd = bo.run_scans(phi, jay, text)
    state, want_f = text, []
    for f in range(frames):
        state = state @ phi[f] + jay[f]
        want_f.append(state)
    state, want_b = text, [None] * frames
    for f in range(frames - 1, -1, -1):
        state = state @ phi[f] + jay[f]
        want_b[f] = state
    torch.testing.assert_close(fwd, torch.stack(want_f), atol=2e-5, rtol=2e-5)
    torch.testing.assert_close(bwd, torch.stack(want_b), atol=2e-5, rtol=2e-5)


def _naive_gather(prefix, suffix, alpha, bounds, text=None):
    frames = prefix.shape[0]
    log_prefix = torch.cat((torch.zeros_like(alpha[:1]), alpha.clamp_min(1e-12).log().cumsum(0)))
    zero = torch.zeros_like(prefix[0])
    out = []
    for f, (raw_lo, raw_hi) in enumerate(bounds):
        lo, hi = max(raw_lo, 0), min(raw_hi, frames - 1)
        before = prefix[lo - 1] if lo else (zero if text is None else text)
        after = suffix[hi + 1] if hi + 1 < frames else (zero if text is None else text)
        before = before * torch.exp(log_prefix[f + 1] - log_prefix[lo]).unsqueeze(1)
        after = after * torch.exp(log_prefix[hi + 1] - log_prefix[f]).unsqueeze(1)
        out.append(before + after)
    return torch.stack(out)


def test_gather_matches_naive_with_and_without_text():
    # tests/test_branch.py:79-113
    torch.manual_seed(4)
    frames, heads, dim = 13, 2, 3
    prefix = torch.randn(frames, heads, dim, dim)
    suffix = torch.randn_like(prefix)
    alpha = torch.rand(frames, heads, dim) * 0.8 + 0.1
    bounds = wo.window_bounds(frames, 1, 4)
    text = torch.randn(heads, dim, dim)
    for initial in (None, text):
        got = bo.gather_linear_state(prefix, suffix, alpha, bounds, text_state=initial)
        torch.testing.assert_close(got, _naive_gather(prefix, suffix, alpha, bounds, initial), atol=2e-6, rtol=2e-5)


def test_alpha_gate_rms_norm_and_activate_closed_forms():
    torch.manual_seed(5)
    mean = torch.randn(3, 7)
    down, up = torch.randn(4, 7), torch.randn(2 * 5, 4)
    dt, a_log = torch.randn(10), torch.randn(2)
    got = bo.alpha_gate(mean, down, up, dt, a_log, 2, 5)
    z = (mean @ down.t() @ up.t() + dt).reshape(3, 2, 5)
    want = torch.exp(-torch.exp(a_log).reshape(2, 1) * torch.log1p(torch.exp(z)))
    torch.testing.assert_close(got, want, atol=1e-6, rtol=1e-5)
    x = torch.randn(4, 6)
    w = torch.randn(6)
    torch.testing.assert_close(bo.rms_norm(x, w), x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w,
                               atol=1e-6, rtol=1e-5)
    t = torch.randn(5, 2, 8)
    s = t * torch.sigmoid(t)
    torch.testing.assert_close(bo.activate(t, True), s / s.norm(dim=-1, keepdim=True).clamp_min(1e-6))
    torch.testing.assert_close(bo.activate(t, False), s)


def test_conv_features_unit_norm_and_conv3d_form():
    # tests/test_branch.py:130-146 checks shape and unit norm; the conv3d form pins the numbers
    torch.manual_seed(6)
    frames, gh, gw, heads, dim = 4, 3, 5, 2, 3
    ch = heads * dim
    tokens = torch.randn(frames * gh * gw, heads, dim)
    sp = torch.randn(ch, 1, 3, 3)
    tm = torch.randn(ch, 1, 3)
    got = bo.conv_features(tokens, sp, tm, frames, (gh, gw), True)
    assert got.shape == tokens.shape
    torch.testing.assert_close(got.norm(dim=-1), torch.ones(got.shape[:-1]), atol=2e-5, rtol=2e-5)
    vol = tokens.reshape(frames, gh, gw, ch).permute(3, 0, 1, 2).unsqueeze(0)       # [1, C, F, gh, gw]
    y = F.conv3d(vol, sp.unsqueeze(2), padding=(0, 1, 1), groups=ch)
    y = F.conv3d(y, tm.reshape(ch, 1, 3, 1, 1), padding=(1, 0, 0), groups=ch)
    raw = y[0].permute(1, 2, 3, 0).reshape(-1, heads, dim)
    torch.testing.assert_close(got, bo.activate(raw, True), atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("ks,kt,l2", [(3, 3, True), (5, 5, True), (5, 5, False), (5, 3, True)])
def test_conv_features_fused_float64_form(ks, kt, l2):
    """The CUDA spelling: bf16 spatial output, then temporal sum / SiLU / norm without rounding."""
    frames, gh, gw, heads, dim = 6, 7, 5, 2, 16
    ch = heads * dim
    g = torch.Generator().manual_seed(61)
    tokens = torch.randn(frames * gh * gw, heads, dim, generator=g).to(torch.bfloat16)
    sp = (torch.randn(ch, 1, ks, ks, generator=g) * 0.2).to(torch.bfloat16)
    tm = (torch.randn(ch, 1, kt, generator=g) * 0.4).to(torch.bfloat16)
    got = bo.conv_features_fused(tokens, sp, tm, frames, (gh, gw), l2)
    vol = tokens.double().reshape(frames, gh, gw, ch).permute(3, 0, 1, 2).unsqueeze(0)       # [1, C, F, gh, gw]
    s64 = F.conv3d(vol, sp.double().unsqueeze(2), padding=(0, ks // 2, ks // 2), groups=ch)
    s64 = s64.to(torch.bfloat16).double()                                                    # the bf16 Conv2d output
    a = F.conv3d(s64, tm.double().reshape(ch, 1, kt, 1, 1), padding=(kt // 2, 0, 0), groups=ch)
    y = a[0].permute(1, 2, 3, 0).reshape(-1, heads, dim)
    y = y * torch.sigmoid(y)
    if l2:
        y = y / y.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    step = 2.0 ** -7 * y.abs() + 2.0 ** -24                                                  # one bf16 step
    assert ((got.double() - y).abs() <= step).all()
    # a planted mistake fails it: temporal taps reversed
    bad = bo.conv_features_fused(tokens, sp, tm.flip(-1), frames, (gh, gw), l2)
    assert not ((bad.double() - y).abs() <= step).all()
    # the eager spelling (bf16 products and sums over the taps) differs by its extra roundings only
    eager = bo.conv_features(tokens, sp, tm, frames, (gh, gw), l2).double()
    assert F.cosine_similarity(eager.flatten(), y.flatten(), dim=0).item() >= 0.9999


def _load(name):
    with safe_open(str(GOLDEN / name), "pt") as f:
        return {k: f.get_tensor(k) for k in f.keys()}, f.metadata()


def test_fused_conv_branch_matches_reference_golden():
    """The CUDA spelling of the short convolutions meets the parity bar on the reference's golden."""
    t, meta = _load("branch_13f_conv.safetensors")
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    gh, gw = map(int, meta["grid"].split("x"))
    w = {k[2:]: v for k, v in t.items() if k.startswith("w.")}
    x, qkv = t["x"], t["qkv"]
    seq = x.shape[0]
    q, k, v = [y.reshape(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    delta = bo.projected_delta(w, x[text:], q[text:], k[text:], v[text:], frames, gh * gw,
                               wo.window_bounds(frames, 1, 5), frame_size=(gh, gw), text_x=x[:text],
                               text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True, short_conv=("k", "v"),
                               fused_conv=True)
    want = t["delta"].float()
    err = (delta.float() - want).abs().max().item()
    cos = F.cosine_similarity(delta.double().flatten(), want.double().flatten(), dim=0).item()
    assert err <= 2e-2 and cos >= 0.9995, (err, cos)


@pytest.mark.parametrize("name", ["branch_13f.safetensors", "branch_13f_conv.safetensors"])
def test_branch_oracle_matches_reference_golden(name):
    t, meta = _load(name)
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    gh, gw = map(int, meta["grid"].split("x"))
    tpf = gh * gw
    conv = tuple(x for x in meta["short_conv"].split(",") if x)
    w = {k[2:]: v for k, v in t.items() if k.startswith("w.")}
    x, qkv = t["x"], t["qkv"]
    seq = x.shape[0]
    q, k, v = [y.reshape(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    delta = bo.projected_delta(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, frame_size=(gh, gw),
                               text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True,
                               short_conv=conv)
    want = t["delta"].float()
    err = (delta.float() - want).abs().max().item()
    scale = want.abs().max().item()
    # the oracle reproduces the reference's bf16 values; a few differ by one rounding step
    assert err <= 4e-3 * max(1.0, scale), (err, scale)
    assert (delta.float() == want).float().mean().item() >= 0.999
    cos = F.cosine_similarity(delta.double().flatten(), want.double().flatten(), dim=0).item()
    assert cos >= 0.99999, cos
    assert torch.count_nonzero(delta[:tpf]) == 0 and torch.count_nonzero(delta[-tpf:]) == 0


def test_branch_oracle_a_bf16_matches_reference_golden():
    """a_fp32=False (A = bf16(bf16(k~ beta)^T k~), symmetrised; vdn_h3/branch.py:238-240): the oracle
    reproduces the reference's own branch output, and the fp32 statistics on the same inputs do not."""
    t, meta = _load("branch_13f_abf16.safetensors")
    assert meta["a_fp32"] == "false"
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    gh, gw = map(int, meta["grid"].split("x"))
    tpf = gh * gw
    w = {k[2:]: v for k, v in t.items() if k.startswith("w.")}
    x, qkv = t["x"], t["qkv"]
    seq = x.shape[0]
    q, k, v = [y.reshape(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    args = (w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds)
    kw = dict(frame_size=(gh, gw), text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    want = t["delta"].float()
    delta = bo.projected_delta(*args, **kw, a_fp32=False).float()
    err = (delta - want).abs().max().item()
    assert err <= 4e-3 * max(1.0, want.abs().max().item()), err
    assert (delta == want).float().mean().item() >= 0.999
    other = bo.projected_delta(*args, **kw).float()        # the fp32 statistics: a different output
    assert (other == want).float().mean().item() < 0.9


def test_frame_statistics_bf16_a_closed_form():
    """With a_fp32=False, A is the symmetrised bf16 rounding of the bf16 product of bf16(k beta) and k:
    exact when every product and sum is representable (keys in {0, +-1/2, +-1}, betas in {1/4 .. 1}, 8
    tokens: multiples of 1/16 up to 8, at most 7 significant bits), and off by the bf16 rounding of that
    product otherwise (a dropped rounding fails it)."""
    g = torch.Generator().manual_seed(3)
    key = (torch.randint(-2, 3, (2, 2, 8, 6), generator=g).float() / 2).to(torch.bfloat16)
    beta = (torch.randint(1, 5, (2, 2, 8), generator=g).float() / 4).to(torch.bfloat16)
    a16, _ = bo.frame_statistics(key, key, beta, a_fp32=False)
    exact = torch.einsum("fhsk,fhsl,fhs->fhkl", key.double(), key.double(), beta.double())
    assert torch.equal(a16.double(), exact)
    key = torch.randn(2, 2, 40, 6, generator=g).to(torch.bfloat16)
    beta = torch.rand(2, 2, 40, generator=g).to(torch.bfloat16)
    a16, _ = bo.frame_statistics(key, key, beta, a_fp32=False)
    wk = (key.float() * beta.float().unsqueeze(-1)).to(torch.bfloat16).double()
    s = torch.einsum("fhsk,fhsl->fhkl", wk, key.double()).to(torch.bfloat16).float()
    torch.testing.assert_close(a16, 0.5 * (s + s.transpose(-1, -2)), atol=0, rtol=0)
    a32, _ = bo.frame_statistics(key, key, beta)
    assert not torch.equal(a16, a32)


def test_sana_factor_closed_forms():
    """SanaDelta (vdn_h3/branch.py:163-177): A = 0 gives Phi = diag(alpha); A = T I gives Phi = 0; B = I gives
    J = I / sqrt(T); alpha scales rows (a transposed product fails it); Phi is linear in A."""
    g = torch.Generator().manual_seed(7)
    tokens, d = 49, 8
    alpha = torch.rand(3, 2, d, generator=g) + 0.5
    eye = torch.eye(d).expand(3, 2, d, d)
    phi, jay = bo.sana_factor(alpha, torch.zeros(3, 2, d, d), eye.clone(), tokens)
    assert torch.equal(phi, torch.diag_embed(alpha))
    assert torch.allclose(jay, eye / 7.0, rtol=0, atol=1e-7)
    phi, _ = bo.sana_factor(alpha, tokens * eye.clone(), eye.clone(), tokens)
    assert torch.count_nonzero(phi) == 0
    a = torch.randn(3, 2, d, d, generator=g)
    phi, _ = bo.sana_factor(alpha, a, a, tokens)
    want = alpha[..., :, None] * (torch.eye(d) - a / tokens)           # row i scaled by alpha[i]
    assert torch.allclose(phi, want, rtol=1e-6, atol=1e-7)
    assert not torch.allclose(phi, alpha[..., None, :] * (torch.eye(d) - a / tokens), rtol=1e-3, atol=1e-4)
    p1, _ = bo.sana_factor(alpha, a, a, tokens)
    p2, _ = bo.sana_factor(alpha, 2 * a, a, tokens)
    p0, _ = bo.sana_factor(alpha, torch.zeros_like(a), a, tokens)
    assert torch.allclose(p2 - p0, 2 * (p1 - p0), rtol=1e-5, atol=1e-6)


def test_sana_branch_oracle_matches_reference_golden():
    """The oracle's sana_scaled branch (frames and text state) reproduces the reference's own output."""
    t, meta = _load("branch_13f_sana.safetensors")
    assert meta["delta_rule"] == "sana_scaled"
    frames, text, heads, dim = int(meta["frames"]), int(meta["text"]), int(meta["heads"]), int(meta["dim"])
    gh, gw = map(int, meta["grid"].split("x"))
    tpf = gh * gw
    w = {k[2:]: v for k, v in t.items() if k.startswith("w.")}
    x, qkv = t["x"], t["qkv"]
    seq = x.shape[0]
    q, k, v = [y.reshape(seq, heads, dim) for y in qkv.split(heads * dim, dim=-1)]
    bounds = wo.window_bounds(frames, 1, 5)
    args = (w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds)
    kw = dict(frame_size=(gh, gw), text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True)
    delta = bo.projected_delta(*args, **kw, delta_rule="sana_scaled")
    want = t["delta"].float()
    err = (delta.float() - want).abs().max().item()
    assert err <= 4e-3 * max(1.0, want.abs().max().item()), err
    assert (delta.float() == want).float().mean().item() >= 0.999
    # the vdn_solve rule on the same inputs is far from it: the golden pins the rule
    other = bo.projected_delta(*args, **kw)
    assert (other.float() - want).abs().max().item() > 50 * max(err, 1e-3)
