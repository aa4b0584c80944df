"""Parity of the benchmarked hybrid attention block at its full shape (GPU).

The block is the one ``bench.py`` times: 40,688 tokens (31 frames of 48 x 27 + 512 text rows), 40 heads x
128, hidden 5120, W8A8 int8 ``qkv_proj`` / ``out_proj`` / ``to_out_linear`` (per-token x per-channel), a
per-row split-half RoPE table, k / v short convolutions in the branch, the text state and the softmax gate
(``vdn_h3/hybrid.py:409-579``). The whole block runs on the GPU; the oracle checks it in layers, each
from the GPU's own input to that layer where a CPU pass over the full problem would take too long:

* the fused qkv projection, one row of every 256-row M tile: bit-identical to the int8 oracle;
* from those q / k / v: the q / k RMSNorm + RoPE of every row, the window attention of one row of every
  work item plus the layout's boundary rows (all 40 heads), the softmax gate and the int8 ``out_proj``;
* the whole VDN branch (short convolutions, statistics, factor, scans, readout) on the CPU for all
  37,584 video rows, its ``to_out_linear`` on the sampled rows;
* the block output at the sampled rows: max-abs 2e-2 and cosine >= 0.9995 (the block's parity bar);
* the branch readout of every row (the GPU branch alone, the same kernels the block runs) in bf16 ulps.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import branch_oracle as bo
from oracle import hybrid_oracle as ho
from oracle import quant_oracle as qo
from oracle import window_oracle as wo

pytestmark = pytest.mark.gpu

SHORT_CONV = ("k", "v")


def _exact_int8_rows(x_rows, w_q, w_scale):
    """The int8 oracle on a few rows, with the int32 accumulators formed in float64: every product is at
    most 127^2 and a row of 5120 of them sums to < 2^27, so the float64 sums are exact."""
    xq, xs = qo.int8_quantize_rows(x_rows)
    acc = (xq.double() @ w_q.double().T).float()
    return (acc * xs.float().reshape(-1, 1) * w_scale.float().reshape(1, -1)).to(torch.bfloat16), xq


def _tile_rows(m, tile=256):
    rows = [t + (37 * i) % min(tile, m - t) for i, t in enumerate(range(0, m, tile))]
    return sorted(set(rows + [m - 1]))


def _parity(got, want, what, atol=2e-2, min_cos=0.9995):
    g, w = got.float().flatten(), want.float().flatten()
    err = (g - w).abs().max().item()
    cos = F.cosine_similarity(g.double(), w.double(), dim=0).item()
    print(f"  {what}: max abs {err:.3e}, cosine {cos:.7f}", flush=True)
    assert torch.isfinite(g).all(), what
    assert err <= atol and cos >= min_cos, f"{what}: max abs {err:.3e}, cosine {cos:.7f}"


def test_full_shape_block_int8_rope_short_conv(device):
    from vdn_h3_amd import projection, synth, window
    from vdn_h3_amd.hybrid import forward_scope
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    w = synth.WINDOW_FULL
    lay = w.layout
    heads, dim, hidden = w.heads, w.head_dim, 5120
    seq, va, vb, tpf, frames, text = lay.seq_len, lay.video_start, lay.video_end, lay.tokens_per_frame, \
        lay.num_frames, lay.text_len
    print(f"case full-shape block S={seq} H={heads} D={dim} hidden={hidden} int8 rope short_conv={SHORT_CONV}",
          flush=True)
    seed = 1000  # the seeds synth.hybrid_stack gives block 0
    state, (forward,) = synth.hybrid_stack(1, heads, dim, hidden, device, short_conv=SHORT_CONV, precision="int8",
                                           first_seed=seed)
    attn = synth.attention_module(heads, dim, hidden, device, seed, "int8")
    bw = synth.branch_weights(heads, dim, hidden, device=device, seed=seed + 42, short_conv=SHORT_CONV)
    x = synth.randn((seq, hidden), 0, device=device, dtype=torch.bfloat16)
    freqs = synth.rope_freqs(seq, dim, device)
    with torch.no_grad(), forward_scope(lay):
        out = forward(x, rope_freqs=freqs)
        qkv = attn.qkv_proj(x)  # the block's qkv_proj kernel on the same input: the q / k / v the block used
    torch.cuda.synchronize()
    assert state.last_attention_backend == "hip"
    out, qkv_h, hx = out.cpu(), qkv.cpu(), x.cpu()
    hw = {kk: vv.cpu() for kk, vv in bw.items()}
    aw = {"q_norm.weight": attn.q_norm.weight.cpu(), "k_norm.weight": attn.k_norm.weight.cpu()}
    torch.set_num_threads(16)

    # the projection weights as synth drew them (on the device's generator), and their int8 codes: the
    # GPU's weight quantisation must give the oracle's codes and scales
    w_qkv = synth.randn((3 * heads * dim, hidden), seed + 1, device=device, dtype=torch.bfloat16, scale=0.02).cpu()
    w_out = synth.randn((hidden, heads * dim), seed + 2, device=device, dtype=torch.bfloat16, scale=0.02).cpu()
    codes = {}
    for name, wt, lin in (("qkv_proj", w_qkv, attn.qkv_proj), ("out_proj", w_out, attn.out_proj)):
        codes[name] = qo.int8_quantize_rows(wt)
        assert torch.equal(lin.weight.cpu(), codes[name][0]), name
        assert torch.equal(lin.weight_scale.cpu().reshape(-1), codes[name][1].reshape(-1)), name
    (qbw,), _ = projection.prepare_projection_maps([bw], device, "int8")
    codes["to_out_linear"] = qo.int8_quantize_rows(hw["to_out_linear.weight"])
    assert torch.equal(qbw["to_out_linear.weight_fp8"].cpu(), codes["to_out_linear"][0])
    assert torch.equal(qbw["to_out_linear.weight_scale"].cpu().reshape(-1), codes["to_out_linear"][1].reshape(-1))

    # 1. qkv_proj: one row per 256-row M tile, bit-identical to the int8 oracle (codes, accumulators, epilogue)
    wq_qkv, ws_qkv = codes["qkv_proj"]
    trows = _tile_rows(seq)
    want_qkv, _ = _exact_int8_rows(hx[trows], wq_qkv, ws_qkv)
    assert torch.equal(qkv_h[trows].view(torch.int16), want_qkv.view(torch.int16))
    print(f"  qkv_proj: {len(trows)} rows bit-identical to the int8 oracle", flush=True)

    # 2. the softmax path at sampled rows, from the GPU's q / k / v
    q_raw, k_raw, v_raw = synth.split_qkv(qkv_h, heads, dim)
    hf = freqs.cpu()
    key = ho.rms_rope_split_half(k_raw, aw["k_norm.weight"], 1e-6, hf, dim)
    items, _, _ = window.build_plan_host(seq, va, vb, frames, tpf, lay.bounds, lay.anchor_frames)
    rows = {0, text - 1, va, va + tpf - 1, va + tpf, va + 5 * tpf - 1, va + 5 * tpf, va + 15 * tpf + 700,
            va + 30 * tpf - 1, va + 30 * tpf, seq - 1}
    for i, (q0, q1, _, _) in enumerate(items.tolist()):
        rows.add(q0 + (53 * i) % (q1 - q0))
    rows = sorted(rows)
    r_t = torch.tensor(rows)
    query = ho.rms_rope_split_half(q_raw[r_t], aw["q_norm.weight"], 1e-6, hf.reshape(seq, -1)[r_t].reshape(
        1, len(rows), 1, dim // 2, 2, 2), dim)
    qfull = torch.zeros(seq, heads, dim, dtype=torch.bfloat16)
    qfull[r_t] = query
    soft = wo.window_attention_rows(qfull, key, v_raw, rows, va, vb, frames, tpf, lay.bounds, dim ** -0.5,
                                    lay.anchor_frames).to(torch.bfloat16)
    gate = torch.sigmoid(bo.linear_bf16(hx[r_t], hw["softmax_gate.up.weight"], hw["softmax_gate.up.bias"]))
    flat = (soft * gate.reshape(len(rows), heads, 1).to(soft.dtype)).reshape(len(rows), heads * dim)
    proj, _ = _exact_int8_rows(flat, *codes["out_proj"])

    # 3. the branch on the CPU for every video row (anchor frames 0 and F-1 skipped), to_out_linear at the
    #    sampled video rows
    inner = slice(va + tpf, va + (frames - 1) * tpf)
    ibounds = [(lo - 1, hi - 1) for lo, hi in lay.bounds[1:-1]]
    readout = bo.readout(hw, hx[inner], q_raw[inner], k_raw[inner], v_raw[inner], frames - 2, tpf, ibounds,
                         frame_size=lay.frame_size, short_conv=SHORT_CONV, fused_conv=True, text_x=hx[:text],
                         text_k_raw=k_raw[:text], text_v_raw=v_raw[:text])
    in_branch = [i for i, r in enumerate(rows) if inner.start <= r < inner.stop]
    b_rows = torch.tensor([rows[i] - inner.start for i in in_branch])
    delta, _ = _exact_int8_rows(readout[b_rows], *codes["to_out_linear"])
    want = proj.clone()
    want[in_branch] = (proj[in_branch].float() + delta.float()).to(torch.bfloat16)

    # 4. the GPU branch alone (the kernels the block runs, the same int8 to_out_linear codes): its readout of
    #    every row and its delta at the sampled rows
    br = OptimizedLinearBranch(qbw, heads, dim, short_conv=SHORT_CONV, enable_text_state=True)
    dq, dk, dv = synth.split_qkv(qkv, heads, dim)
    kw = dict(frame_size=lay.frame_size, text_x=x[:text], text_k_raw=dk[:text], text_v_raw=dv[:text], skip_ends=True)
    with torch.no_grad():
        got_read = br.readout(qbw, x[va:], dq[va:], dk[va:], dv[va:], frames, tpf, lay.bounds, **kw)
        got_delta = br.projected_delta(qbw, x[va:], dq[va:], dk[va:], dv[va:], frames, tpf, lay.bounds, **kw)
    torch.cuda.synchronize()
    got_read, got_delta = got_read.cpu(), got_delta.cpu()

    print(f"  {len(rows)} sampled rows ({items.shape[0]} work items), {len(in_branch)} of them in branch frames",
          flush=True)
    # the int8 to_out_linear of the GPU's own readout rows is the int8 oracle's, bit for bit
    gb_rows = torch.tensor([rows[i] - va for i in in_branch])
    delta_iso, _ = _exact_int8_rows(got_read[gb_rows], *codes["to_out_linear"])
    assert torch.equal(got_delta[gb_rows].view(torch.int16), delta_iso.view(torch.int16))
    dd = (got_delta[gb_rows].float() - delta.float()).abs()
    print(f"  branch delta at the sampled rows: bit-identical to the int8 oracle of the GPU's readout; against "
          f"the oracle's readout max abs {dd.max().item():.3e} (max |delta| {delta.float().abs().max().item():.2f})",
          flush=True)

    # 5. the block output at the sampled rows, (a) with the branch delta of the GPU's readout (checked above)
    #    and (b) end to end with the oracle's own readout
    want_iso = proj.clone()
    want_iso[in_branch] = (proj[in_branch].float() + delta_iso.float()).to(torch.bfloat16)
    g = out[r_t].float()
    stats = {}
    for name, ref in (("isolated", want_iso), ("end to end", want)):
        wv = ref.float()
        diff = (g - wv).abs()
        small = wv.abs() < 2
        steps = diff / torch.ldexp(torch.ones_like(wv), torch.frexp(wv)[1] - 8)
        cos = F.cosine_similarity(g.double().flatten(), wv.double().flatten(), dim=0).item()
        stats[name] = (cos, diff, small, steps)
        print(f"  block output ({name}): cosine {cos:.7f}; max abs where |want| < 2: {diff[small].max().item():.3e}; "
              f"ulps of the value where |want| >= 2 ({int((~small).sum())} values, max |want| "
              f"{wv.abs().max().item():.2f}): max {steps[~small].max().item():.2f}; max abs {diff.max().item():.3e}",
              flush=True)

    # 6. the readout of every row against the oracle's
    assert torch.count_nonzero(got_read[:tpf]) == 0 and torch.count_nonzero(got_read[-tpf:]) == 0
    g32, w32 = got_read[tpf:-tpf].float(), readout.float()
    ulp = torch.ldexp(torch.ones_like(w32), torch.frexp(w32)[1] - 8).clamp_min(2.0 ** -133)
    rsteps = (g32 - w32).abs() / ulp
    # in ulps of max(|want|, 1): values below 1 in magnitude (the readout is RMS-normalised per row and
    # gated, so most lie in (-4, 4)) are held to an absolute bound of that many ulps of 1
    steps1 = (g32 - w32).abs() / torch.maximum(ulp, torch.full_like(ulp, 2.0 ** -7))
    rcos = F.cosine_similarity(g32.double().flatten(), w32.double().flatten(), dim=0).item()
    print(f"  readout ({g32.numel()} values): cosine {rcos:.7f}; ulps of the oracle value: frac > 2 "
          f"{(rsteps > 2).float().mean():.2e}, frac > 8 {(rsteps > 8).float().mean():.2e}; ulps of max(|v|, 1): max "
          f"{steps1.max().item():.1f}, frac > 2 {(steps1 > 2).float().mean():.2e}", flush=True)

    # (a) the block's parity bar: max-abs 2e-2 where |v| < 2, within two bf16 steps of the value above
    #     (out_proj and the delta are each rounded to bf16 before their bf16 sum), cosine >= 0.9995
    cos, diff, small, steps = stats["isolated"]
    assert torch.isfinite(g).all()
    assert cos >= 0.9995, cos
    assert diff[small].max().item() <= 2e-2
    assert steps[~small].max().item() <= 2
    # (b) end to end: a readout value a few ulps off (below) can move its row's int8 scale (amax / 127); the
    #     row's W8A8 to_out_linear then carries a different rounding of every code, noise of about
    #     sqrt(5120) * (scale / sqrt(12)) * 0.02 ~ 1e-2 per output on rows with |readout| ~ 4
    cos, diff, _, _ = stats["end to end"]
    assert cos >= 0.9999, cos
    assert diff.max().item() <= 5e-2
    # the readout: at most 0.5% of values beyond two ulps of the value, 0.15% beyond eight (the fp32
    # statistics round differently from the oracle's where a bf16 midpoint is straddled), and every value
    # within 8 ulps of max(|v|, 1)
    assert rcos >= 0.9999, rcos
    assert (rsteps > 2).float().mean().item() <= 5e-3
    assert (rsteps > 8).float().mean().item() <= 1.5e-3
    assert steps1.max().item() <= 8
