#!/usr/bin/env python3
"""Benchmark of the VDN-H3 hybrid attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload block]

Prints one JSON line. Inputs and weights are resident in HBM before timing; synthetic
seeded data, random-init weights.

Workload ``block`` (default): one hybrid attention block, the patched ``attn.forward``, at the
full shape: 512 text rows + 31 frames x 1296 tokens = 40 688 rows, hidden 5120, 40 heads x
128, chunk 5, radius 1, anchors both, a per-row split-half RoPE table (``--rope off`` drops it).
A step is one block forward: W8A8 int8 qkv projection, softmax gate, window attention (q/k
RMSNorm + RoPE fused into its pre-pass and query load, the gate into its epilogue), W8A8 out
projection, and the VDN branch (29 inner frames) with its int8 to_out_linear accumulated into
the output.
``value`` is the block's algorithmic work per second (int8 OPs + bf16/fp32 FLOPs, listed per
stage in ``config.work_per_step``); ``roofline`` is the window attention kernel (the dominant
kernel), timed with HIP events on the stream it runs on; ``stages_ms`` are per-stage event
timings of the same timed steps. ``roofline_vs_sustained_mfma`` sets the same kernel rate against
the part's sustained MFMA rate on random operands (``--workload mfma_peak``), measured after the
timed region: the datasheet ``peak`` assumes a clock the power limit allows only on operands that
barely toggle.

Other workloads: ``stack`` (50 blocks x ``--steps`` denoising steps, ``x <- x + block(rms_norm(x))``; use
``--steps 8 --warmup 1`` for the 8-step pass), ``window`` (attention alone), ``branch`` (VDN branch alone),
``gemm_{i8,f8}_{qkv,out}`` (W8A8 GEMMs alone), ``gdn`` (token-level chunk-64 Gated DeltaNet), ``dit``
(the DiT block pointwise passes), ``rope`` (q/k RMSNorm + RoPE),
``hbm_copy`` (counter calibration), ``mfma_peak`` (sustained MFMA rates, the ceiling calibration),
``cpu_configs`` (the fp32 CPU oracle timed per configuration at full size on the host cores, a few minutes).
``cpu_baseline`` times the fp32 CPU oracle on the host cores (16 threads, the host's CPU share for one GPU) on bounded
samples (1 warm-up, median of 3): for ``block``, the window attention on sampled query rows, the projections
on sampled rows and the VDN branch on 7 of its 29 inner frames, combined at the block's per-part work.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "comfyui-kirei-vdn-h3_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "VDN hybrid block ms + TFLOP/s (% MFMA peak) at 40,688 tok x 40 heads, 1 GPU"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
PEAK_I8_TOPS = 5000.0       # dense int8 MFMA
PEAK_F8_TFLOPS = 5000.0     # dense fp8 MFMA


def _parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="block", choices=["block", "stack", "window", "hbm_copy", "branch",
                                                             "gemm_i8_qkv", "gemm_i8_out", "gemm_f8_qkv",
                                                             "gemm_f8_out", "gdn", "dit", "rope", "mfma_peak",
                                                             "cpu_configs"],
                    help="hbm_copy: a plain 1 GiB device copy, the reference point for scaling rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes")
    ap.add_argument("--short-conv", default="k,v",
                    help="branch short-convolution targets of the block / branch workloads (the released "
                         "checkpoints convolve k and v); '' for none")
    ap.add_argument("--rope", default="on", choices=["on", "off"],
                    help="block / stack workloads: hand every block a per-row split-half RoPE table "
                         "(rot_dim = head_dim), as a DiT does, or no rope_freqs")
    ap.add_argument("--branch-execution", default="serial", choices=["serial", "parallel"],
                    help="block / stack workloads: the VDN branch after the attention on the same stream "
                         "(serial) or beside it on a second stream, joined at to_out_linear (parallel)")
    ap.add_argument("--cpu-sample-rows", type=int, default=2304,
                    help="query rows of the CPU-oracle baseline sample (0 disables it)")
    ap.add_argument("--traffic-json", default=str(ROOT / "profiles" / "traffic.json"),
                    help="HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def _traffic(path, kernel):
    try:
        data = json.loads(Path(path).read_text())
        return data[kernel]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def bench_window(args, torch, device):
    from vdn_h3_amd import _lib, synth, window

    w = synth.WINDOW_FULL
    qkv, q, k, v, lay, _ = synth.window_inputs(w, device=device)   # q, k, v ~ N(0, 1) / sqrt(128)
    plan = window.make_plan(lay.seq_len, lay.video_start, lay.video_end, lay.num_frames, lay.tokens_per_frame,
                            lay.bounds, lay.anchor_frames, device)
    lib = _lib.lib()
    seq, heads, dim = q.shape
    ws_bytes = lib.vdnh3_window_workspace_bytes(seq, heads, dim)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((seq, heads, dim), dtype=torch.bfloat16, device=device)
    stream = torch.cuda.current_stream(device)
    sh = _lib.stream_handle(device)

    def prepass():
        _lib.check(lib.vdnh3_window_vt_prepass(_lib.ptr(v), v.stride(0), v.stride(1), seq, heads, dim,
                                               _lib.ptr(ws), ws_bytes, sh), "prepass")

    def attention():
        _lib.check(lib.vdnh3_window_attn_prepared(
            _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
            _lib.ptr(out), out.stride(0), out.stride(1), None, 0, seq, heads, dim, float(w.scale),
            _lib.ptr(plan.items), plan.n_items, _lib.ptr(plan.tiles), _lib.ptr(ws), ws_bytes, sh), "attention")

    for _ in range(args.warmup):
        prepass()
        attention()
    torch.cuda.synchronize()
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    t0, t1 = ev(), ev()
    a0 = [ev() for _ in range(args.steps)]
    a1 = [ev() for _ in range(args.steps)]
    t0.record(stream)
    for i in range(args.steps):
        prepass()
        a0[i].record(stream)
        attention()
        a1[i].record(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / args.steps
    attn_ms = sum(a0[i].elapsed_time(a1[i]) for i in range(args.steps)) / args.steps
    flops = window.attention_flops(plan.pairs_per_head, heads, dim)
    tflops = flops / (ms_step * 1e-3) / 1e12
    attn_tflops = flops / (attn_ms * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms_step, 4),
        "dtype": "bf16",
        "config": {"workload": w.name, "seq_len": seq, "heads": heads, "head_dim": dim, "frames": lay.num_frames,
                   "tokens_per_frame": lay.tokens_per_frame, "text_rows": lay.text_len, "chunk": w.chunk,
                   "radius": w.radius, "anchor_frames": lay.anchor_frames,
                   "allowed_pairs_per_head": plan.pairs_per_head, "flop_per_step": flops},
        "roofline": {"bound": "mfma", "kernel": "window_attn_kernel<128,false>", "achieved": round(attn_tflops, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4),
                     "kernel_ms": round(attn_ms, 4), "traffic": _traffic(args.traffic_json, "window_attn_kernel")},
        "breakdown_ms": {"vt_prepass": round(ms_step - attn_ms, 4), "window_attn": round(attn_ms, 4)},
        "roofline_vs_sustained_mfma": ceiling_entry(torch, device, 0, attn_tflops),
    }
    if args.cpu_sample_rows > 0:
        result["cpu_baseline"] = cpu_baseline_window(torch, qkv, w, lay, args.cpu_sample_rows)
    return result


def bench_hbm_copy(args, torch, device):
    """Copy of 2**30 bytes (bf16), timed like a step: the HBM-counter calibration kernel."""
    n = 1 << 29
    src = torch.ones(n, dtype=torch.bfloat16, device=device)
    dst = torch.empty_like(src)
    for _ in range(args.warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    gbs = 2 * (1 << 30) / (ms * 1e-3) / 1e9
    return {"metric": "HBM copy bandwidth (counter calibration)", "value": round(gbs, 1), "unit": "GB/s",
            "ms_per_step": round(ms, 4), "dtype": "bf16",
            "config": {"workload": "hbm_copy_1GiB", "bytes_read": 1 << 30, "bytes_written": 1 << 30},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None}}


def _time_steps(torch, stream, steps, warmup, fn):
    """Mean ms per call of ``fn`` over ``steps`` timed calls (HIP events on ``stream``)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        fn()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def _short_conv(args):
    return tuple(t for t in args.short_conv.split(",") if t)


def _rope_desc(args, dim):
    return (f"split-half RoPE, rot_dim {dim}, per-row table (fused into the attention's q/k RMSNorm)"
            if args.rope == "on" else "none")


def block_flops(lay, heads, dim, hidden, pairs_per_head, short_conv=()):
    """Algorithmic work of one hybrid block (int8 OPs of the W8A8 GEMMs + bf16/fp32 FLOPs), by stage."""
    s, inner = lay.seq_len, heads * dim
    fi = lay.num_frames - 2 if lay.anchor_frames == "both" else lay.num_frames
    r, t = fi * lay.tokens_per_frame, lay.tokens_per_frame
    return {
        "branch_short_conv": len(short_conv) * 2.0 * (25 + 5) * r * inner,
        "qkv_proj": 2.0 * s * hidden * 3 * inner,
        "softmax_gate": 2.0 * s * hidden * heads,
        "window_attention": 4.0 * dim * heads * pairs_per_head,
        "out_proj": 2.0 * s * inner * hidden,
        "branch_core": fi * heads * (6.0 * t * dim * dim + (11.0 / 3.0) * dim ** 3 + 4.0 * dim ** 3),
        "branch_gates": 2.0 * r * hidden * dim + 2.0 * r * dim * inner + 2.0 * r * hidden * heads,
        "branch_text_state": heads * (4.0 * lay.text_len * dim * dim + (11.0 / 3.0) * dim ** 3)
                             + 2.0 * lay.text_len * hidden * heads,
        "to_out_linear": 2.0 * r * inner * hidden,
    }


def bench_block(args, torch, device):
    """One VDN-H3 hybrid attention block at the full shape (the patched attn.forward)."""
    from vdn_h3_amd import synth
    from vdn_h3_amd.hybrid import forward_scope

    w = synth.WINDOW_FULL
    lay = w.layout
    heads, dim, hidden = w.heads, w.head_dim, 5120
    x = synth.randn((lay.seq_len, hidden), 0, device=device, dtype=torch.bfloat16)
    conv = _short_conv(args)
    state, (forward,) = synth.hybrid_stack(1, heads, dim, hidden, device, short_conv=conv, precision="int8",
                                           branch_execution=args.branch_execution)
    state.diagnostics.enabled = True
    freqs = synth.rope_freqs(lay.seq_len, dim, device) if args.rope == "on" else None
    stream = torch.cuda.current_stream(device)
    with torch.no_grad(), forward_scope(lay):
        for _ in range(args.warmup):
            forward(x, rope_freqs=freqs)
        torch.cuda.synchronize()
        state.diagnostics.clear()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(args.steps):
            forward(x, rope_freqs=freqs)
        t1.record(stream)
        torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    stages = {k: v["mean_ms"] for k, v in state.diagnostics.snapshot()["stages"].items()}
    plan = state.window_cache.plan(lay.seq_len, lay.video_start, lay.video_end, lay.num_frames,
                                   lay.tokens_per_frame, lay.bounds, lay.anchor_frames, device)
    work = block_flops(lay, heads, dim, hidden, plan.pairs_per_head, conv)
    total = sum(work.values())
    attn_ms = stages["attention.softmax.kernel"]
    attn_tflops = work["window_attention"] / (attn_ms * 1e-3) / 1e12
    qkv_tops = work["qkv_proj"] / (stages["attention.qkv"] * 1e-3) / 1e12
    out_tops = work["out_proj"] / (stages["attention.out_proj"] * 1e-3) / 1e12
    return {
        "metric": METRIC,
        "value": round(total / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4),
        "dtype": "int8+bf16",
        "config": {"workload": "hybrid_block_s40688_h40_d128_hidden5120_int8proj", "seq_len": lay.seq_len,
                   "heads": heads, "head_dim": dim, "hidden": hidden, "frames": lay.num_frames,
                   "tokens_per_frame": lay.tokens_per_frame, "text_rows": lay.text_len, "chunk": w.chunk,
                   "radius": w.radius, "anchor_frames": lay.anchor_frames,
                   "projections": "W8A8 int8 qkv/out/to_out_linear (per-token x per-channel)",
                   "rope": _rope_desc(args, dim),
                   "branch_short_conv": ",".join(conv) or "none", "branch_execution": args.branch_execution,
                   "allowed_pairs_per_head": plan.pairs_per_head, "work_per_step": work,
                   "work_total": total},
        "roofline": {"bound": "mfma", "kernel": "window_attn_kernel<128,%s>" % ("false" if freqs is not None else "true"), "achieved": round(attn_tflops, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4),
                     "kernel_ms": round(attn_ms, 4), "traffic": _traffic(args.traffic_json, "window_attn_kernel")},
        "stages_ms": {k: round(v, 4) for k, v in stages.items()},
        "stage_rooflines": {
            "qkv_proj (quant + int8 GEMM)": {"achieved_TOPs": round(qkv_tops, 1),
                                             "frac_int8_peak": round(qkv_tops / PEAK_I8_TOPS, 4)},
            "out_proj (quant + int8 GEMM)": {"achieved_TOPs": round(out_tops, 1),
                                             "frac_int8_peak": round(out_tops / PEAK_I8_TOPS, 4)},
            "window_attention": {"achieved_TFLOPs": round(attn_tflops, 1),
                                 "frac_bf16_peak": round(attn_tflops / PEAK_BF16_TFLOPS, 4)},
        },
        "linear_to_softmax_ratio": round((stages["attention.linear_branch"]
                                          + stages.get("attention.branch_projection", 0.0))
                                         / stages["attention.softmax"], 4),
        "roofline_vs_sustained_mfma": ceiling_entry(torch, device, 0, attn_tflops),
    }


def bench_stack(args, torch, device):
    """The 50-block hybrid attention stack over one 8-step denoising pass (x <- x + block(rms_norm(x)))."""
    from vdn_h3_amd import synth
    from vdn_h3_amd.hybrid import forward_scope

    w = synth.WINDOW_FULL
    lay = w.layout
    heads, dim, hidden, blocks = w.heads, w.head_dim, 5120, 50
    conv = _short_conv(args)
    state, forwards = synth.hybrid_stack(blocks, heads, dim, hidden, device, short_conv=conv, precision="int8",
                                         branch_execution=args.branch_execution)
    x0 = synth.randn((lay.seq_len, hidden), 0, device=device, dtype=torch.bfloat16)
    freqs = synth.rope_freqs(lay.seq_len, dim, device) if args.rope == "on" else None
    stream = torch.cuda.current_stream(device)
    with torch.no_grad(), forward_scope(lay):
        synth.denoise_pass(forwards, x0.clone(), args.warmup, rope_freqs=freqs)
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        x = x0.clone()
        ev[0].record(stream)
        for i in range(args.steps):
            x = synth.denoise_pass(forwards, x, 1, rope_freqs=freqs)
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
    step_ms = [ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)]
    total_ms = ev[0].elapsed_time(ev[-1])
    plan = state.window_cache.plan(lay.seq_len, lay.video_start, lay.video_end, lay.num_frames,
                                   lay.tokens_per_frame, lay.bounds, lay.anchor_frames, device)
    work = block_flops(lay, heads, dim, hidden, plan.pairs_per_head, conv)
    per_block = sum(work.values())
    total_work = per_block * blocks * args.steps
    finite = bool(torch.isfinite(x).all().item())
    return {
        "metric": "VDN-H3 50-block hybrid attention stack, 8-step denoising pass: ms per step + TFLOP/s, 1 GPU",
        "value": round(total_work / (total_ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(total_ms / args.steps, 3),
        "dtype": "int8+bf16",
        "config": {"workload": "stack_50blocks_s40688_h40_d128_hidden5120_int8proj", "blocks": blocks,
                   "denoising_steps": args.steps, "seq_len": lay.seq_len, "heads": heads, "head_dim": dim,
                   "hidden": hidden, "branch_short_conv": ",".join(conv) or "none", "rope": _rope_desc(args, dim),
                   "branch_execution": args.branch_execution,
                   "residual": "x <- x + block(rms_norm(x)) per block (bf16, torch rms_norm)", "work_per_block": per_block},
        "total_ms": round(total_ms, 2),
        "step_ms": [round(v, 3) for v in step_ms],
        "block_ms_mean": round(total_ms / (args.steps * blocks), 4),
        "output_finite": finite,
    }


def bench_gemm(args, torch, device):
    """W8A8 projection GEMM at the block's shapes: M=40,688 tokens, K=5,120, N=15,360 (qkv) or 5,120 (out)."""
    from vdn_h3_amd import linear, synth

    kind_name, which = args.workload.split("_")[1:]
    m, k = 40688, 5120
    n = 15360 if which == "qkv" else 5120
    x = synth.randn((m, k), 30, device=device, dtype=torch.bfloat16)
    w = synth.randn((n, k), 31, device=device, dtype=torch.bfloat16, scale=0.02)
    if kind_name == "i8":
        wq, ws = linear.quantize_rows(w, linear.KIND_I8)
        quant = lambda: linear.quantize_rows(x, linear.KIND_I8)  # noqa: E731
        peak, dtype = PEAK_I8_TOPS, "int8"
    else:
        wq, ws = linear.quantize_tensor_fp8(w)
        quant = lambda: linear.quantize_tensor_fp8(x)  # noqa: E731
        peak, dtype = PEAK_F8_TFLOPS, "fp8_e4m3"
    xq, xs = quant()
    out = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    stream = torch.cuda.current_stream(device)
    gemm_ms = _time_steps(torch, stream, args.steps, args.warmup,
                          lambda: linear.gemm_w8a8(xq, xs, wq, ws, out=out))
    quant_ms = _time_steps(torch, stream, args.steps, args.warmup, quant)
    ops = 2.0 * m * n * k
    tops = ops / (gemm_ms * 1e-3) / 1e12
    qbytes = m * k * 2 + m * k + 4 * m
    return {
        "metric": f"W8A8 {which} projection GEMM TOP/s ({dtype} MFMA)",
        "value": round(tops, 2), "unit": "TOP/s", "ms_per_step": round(gemm_ms, 4), "dtype": dtype,
        "config": {"workload": f"gemm_{kind_name}_{which}_m{m}_k{k}_n{n}", "M": m, "N": n, "K": k,
                   "scales": "per-token x per-channel" if kind_name == "i8" else "per-tensor", "ops_per_step": ops},
        "roofline": {"bound": "mfma", "kernel": f"gemm_nt_kernel<{kind_name}>", "achieved": round(tops, 2),
                     "peak": peak, "unit": "TOP/s", "frac": round(tops / peak, 4), "kernel_ms": round(gemm_ms, 4),
                     "traffic": _traffic(args.traffic_json, f"gemm_nt_kernel<{kind_name}>:{which}")},
        "breakdown_ms": {"activation_quant": round(quant_ms, 4), "gemm": round(gemm_ms, 4),
                         "activation_quant_GBs": round(qbytes / (quant_ms * 1e-3) / 1e9, 1)},
        "roofline_vs_sustained_mfma": ceiling_entry(torch, device, 1 if kind_name == "i8" else 2, tops),
        "library_same_box": library_gemm_rate(torch, device, stream, args, kind_name, xq, xs, wq, ws, ops),
    }


def library_gemm_rate(torch, device, stream, args, kind_name, xq, xs, wq, ws, ops):
    """hipBLASLt on the same operands and machine, timed like the kernel above (a comparison, not this library's
    path): torch._scaled_mm (fp8 per-tensor, bf16 out) or torch._int_mm (int8, int32 accumulators out, no
    scales applied)."""
    if kind_name == "i8":
        fn = lambda: torch._int_mm(xq, wq.t())  # noqa: E731
        what = "torch._int_mm (hipBLASLt), int32 output, scales not applied"
    else:
        sa, sb = xs.reshape(()).float(), ws.reshape(()).float()
        fn = lambda: torch._scaled_mm(xq.view(torch.float8_e4m3fn), wq.view(torch.float8_e4m3fn).t(),  # noqa: E731
                                      scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
        what = "torch._scaled_mm (hipBLASLt), per-tensor scales, bf16 output"
    try:
        ms = _time_steps(torch, stream, args.steps, args.warmup, fn)
    except RuntimeError as err:  # the library path is a comparison only
        return {"kernel": what, "error": str(err)[:200]}
    return {"kernel": what, "ms": round(ms, 4), "TOPs": round(ops / (ms * 1e-3) / 1e12, 1)}


def bench_branch(args, torch, device):
    """Video Delta Attention branch at the full shape: projected_delta over 31 frames x 1296 tokens, 40 x 128."""
    from vdn_h3_amd import synth
    from vdn_h3_amd.runtime import OptimizedLinearBranch
    from vdn_h3_amd.window import window_bounds

    frames, tpf, text, heads, dim, hidden = 31, 1296, 512, 40, 128, 5120
    seq = text + frames * tpf
    qkv = synth.fused_qkv(seq, heads, dim, device=device, seed=40)
    x = synth.randn((seq, hidden), 41, device=device, dtype=torch.bfloat16)
    conv = _short_conv(args)
    w = synth.branch_weights(heads, dim, hidden, device=device, short_conv=conv)
    q, k, v = synth.split_qkv(qkv, heads, dim)
    bounds = window_bounds(frames, 1, 5)
    br = OptimizedLinearBranch(w, heads, dim, short_conv=conv)
    out = torch.empty((frames * tpf, hidden), dtype=torch.bfloat16, device=device)
    kw = dict(frame_size=(48, 27), text_x=x[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True,
              out=out)
    stream = torch.cuda.current_stream(device)

    def step():
        br.projected_delta(w, x[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, **kw)

    with torch.no_grad():
        ms = _time_steps(torch, stream, args.steps, args.warmup, step)
    fi, r = frames - 2, (frames - 2) * tpf
    core = fi * heads * (6.0 * tpf * dim * dim + (11.0 / 3.0) * dim ** 3 + 4.0 * dim ** 3)
    gates = 2.0 * r * hidden * dim + 2.0 * r * dim * heads * dim + 2.0 * r * hidden * heads
    proj = 2.0 * r * heads * dim * hidden
    conv_flops = len(conv) * 2.0 * (25 + 5) * r * heads * dim
    flops = core + gates + proj + conv_flops
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "metric": "VDN delta-rule branch ms + TFLOP/s at 29 inner frames x 1296 tok x 40 heads, 1 GPU",
        "value": round(tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4), "dtype": "bf16",
        "config": {"workload": "branch_f31_t1296_h40_d128", "frames": frames, "inner_frames": fi,
                   "tokens_per_frame": tpf, "text_rows": text, "heads": heads, "head_dim": dim, "hidden": hidden,
                   "short_conv": ",".join(conv) or "none", "flop_core": core, "flop_gates": gates,
                   "flop_short_conv": conv_flops, "flop_to_out_linear": proj},
        "roofline": {"bound": "mfma", "kernel": "projected_delta (all kernels)", "achieved": round(tflops, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": _traffic(args.traffic_json, "projected_delta")},
    }


def bench_gdn(args, torch, device):
    """Token-level chunk-64 Gated DeltaNet (the delta rule over all tokens, not per frame) at 40,688 x 40 x 128."""
    import torch.nn.functional as F

    from vdn_h3_amd import _lib
    from vdn_h3_amd.gdn import gdn_flops, gdn_forward_into

    tokens, heads, dim = 40688, 40, 128
    g = torch.Generator(device=device).manual_seed(50)
    qkv = torch.randn(tokens, heads, 3 * dim, generator=g, device=device).to(torch.bfloat16)
    q, v = qkv[..., :dim], qkv[..., 2 * dim:]
    k = qkv[..., dim:2 * dim]
    k.copy_(F.normalize(k.float(), dim=-1).to(torch.bfloat16))
    beta = torch.sigmoid(torch.randn(tokens, heads, generator=g, device=device))
    lg = -F.softplus(torch.randn(tokens, heads, generator=g, device=device))
    out = torch.empty((tokens, heads, dim), dtype=torch.bfloat16, device=device)
    lib = _lib.lib()
    ws_bytes = lib.vdnh3_gdn_workspace_bytes(tokens, heads, dim)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device)

    def step():  # the segments' preps on a second stream beside the scans (vdn_h3_amd.gdn)
        gdn_forward_into(q, k, v, beta, lg, out, ws)

    ms = _time_steps(torch, stream, args.steps, args.warmup, step)
    flops = gdn_flops(tokens, heads, dim)
    io_bytes = 4.0 * tokens * heads * dim * 2 + 2.0 * tokens * heads * 4     # q, k, v in; o out; beta, g in
    gbs = io_bytes / (ms * 1e-3) / 1e9
    result = {
        "metric": "chunk-64 Gated DeltaNet forward ms + TFLOP/s at 40,688 tok x 40 heads x 128, 1 GPU",
        "value": round(flops / (ms * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
        "dtype": "bf16",
        "config": {"workload": "gdn_chunk64_t40688_h40_d128", "tokens": tokens, "heads": heads, "head_dim": dim,
                   "chunk": 64, "flop_per_step": flops, "io_bytes_per_step": io_bytes,
                   "workspace_bytes": ws_bytes},
        "roofline": {"bound": "hbm", "kernel": "gdn_prep_kernel + gdn_scan_kernel", "achieved": round(gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": _traffic(args.traffic_json, "gdn")},
    }
    if args.cpu_sample_rows > 0:
        from oracle import gdn_oracle as go

        sel = list(range(8))  # 8 of the heads: the same work per head, a bounded CPU sample
        hq, hk, hv, hb, hg = (t[:, sel].cpu() for t in (q, k, v, beta, lg))
        dt, runs = _median_seconds(lambda: go.chunked(hq, hk, hv, hb, hg))
        model, physical = _cpu_description()
        result["cpu_baseline"] = {
            "value": round(gdn_flops(tokens, len(sel), dim) / dt / 1e12, 5), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port", "seconds_median": round(dt, 3),
            "seconds_runs": [round(t, 3) for t in runs], "cpu": model, "physical_cores": physical,
            "sample": f"all {tokens} tokens x {len(sel)} of the {heads} heads, float64 chunk-form oracle "
                      "(oracle/gdn_oracle.py); 1 warm-up, median of 3"}
    return result


def bench_dit(args, torch, device):
    """The DiT block pointwise passes around the attention at 40,688 rows x hidden 5120: RMSNorm + AdaLN
    modulation, the gated residual, and the SwiGLU fused into fc2's per-token int8 quantisation (MLP
    width 13,824 = 2 x 6,912 per half is an assumption: the reference does not pin it)."""
    from vdn_h3_amd import block_kernels as bk
    from vdn_h3_amd import linear as L
    from vdn_h3_amd import synth

    rows, hidden, ffn = 40688, 5120, 13824
    x = synth.randn((rows, hidden), 60, device=device, dtype=torch.bfloat16)
    b = synth.randn((rows, hidden), 61, device=device, dtype=torch.bfloat16)
    w = (1 + 0.1 * synth.randn((hidden,), 62, device=device)).to(torch.bfloat16)
    scale = 0.3 * synth.randn((1, hidden), 63, device=device)
    shift = 0.3 * synth.randn((1, hidden), 64, device=device)
    gate = 0.3 * synth.randn((1, hidden), 65, device=device)
    idx = torch.zeros(rows, dtype=torch.int32, device=device)
    h = synth.randn((rows, 2 * ffn), 66, device=device, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream(device)
    with torch.no_grad():
        t_mod = _time_steps(torch, stream, args.steps, args.warmup, lambda: bk.rmsnorm_modulate(x, w, 1e-6, scale, shift, idx))
        t_res = _time_steps(torch, stream, args.steps, args.warmup, lambda: bk.gated_residual(x, gate, idx, b))
        t_swq = _time_steps(torch, stream, args.steps, args.warmup, lambda: bk.swiglu_quantize_rows(h, L.KIND_I8))
    mb = {"rmsnorm_modulate": 2 * rows * hidden * 2, "gated_residual": 3 * rows * hidden * 2,
          "swiglu_quant_rows_i8": rows * 2 * ffn * 2 + rows * ffn + rows * 4}
    ms = {"rmsnorm_modulate": t_mod, "gated_residual": t_res, "swiglu_quant_rows_i8": t_swq}
    total_ms = sum(ms.values())
    gbs = {k: mb[k] / (ms[k] * 1e-3) / 1e9 for k in ms}
    return {
        "metric": "DiT block pointwise passes (RMSNorm+AdaLN, gated residual, SwiGLU->int8) ms + GB/s at 40,688 x 5120, 1 GPU",
        "value": round(sum(mb.values()) / (total_ms * 1e-3) / 1e9, 1), "unit": "GB/s", "ms_per_step": round(total_ms, 4),
        "dtype": "bf16",
        "config": {"workload": "dit_pointwise_r40688_h5120_ffn13824", "rows": rows, "hidden": hidden, "ffn": ffn,
                   "bytes_per_kernel": mb},
        "roofline": {"bound": "hbm", "kernel": "swiglu_quant_row_kernel<int8>", "achieved": round(gbs["swiglu_quant_rows_i8"], 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs["swiglu_quant_rows_i8"] / PEAK_HBM_GBS, 4),
                     "traffic": None},
        "breakdown": {k: {"ms": round(ms[k], 4), "GBs": round(gbs[k], 1)} for k in ms},
    }


def bench_rope(args, torch, device):
    """q/k RMSNorm with split-half RoPE (one 2x2 rotation per row and pair, rot_dim 128) on the raw q / k
    views of the fused qkv rows at 40,688 x 40 x 128, beside the plain q/k RMSNorm."""
    import math

    from vdn_h3_amd import synth
    from vdn_h3_amd.hybrid import normalise_qk

    seq, heads, dim = 40688, 40, 128
    qkv = synth.fused_qkv(seq, heads, dim, device=device, seed=70)
    q, k, _ = synth.split_qkv(qkv, heads, dim)
    wq = (1 + 0.1 * synth.randn((dim,), 71, device=device)).to(torch.bfloat16)
    wk = (1 + 0.1 * synth.randn((dim,), 72, device=device)).to(torch.bfloat16)
    pos = torch.arange(seq, device=device, dtype=torch.float32)[:, None]
    inv = torch.pow(10000.0, -torch.arange(dim // 2, device=device, dtype=torch.float32) / (dim // 2))[None, :]
    ang = pos * inv
    c, s_ = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([c, -s_], -1), torch.stack([s_, c], -1)], -2).view(1, seq, 1, dim // 2, 2, 2)
    stream = torch.cuda.current_stream(device)
    with torch.no_grad():
        t_rope = _time_steps(torch, stream, args.steps, args.warmup, lambda: normalise_qk(q, k, wq, wk, 1e-6, rope_freqs=freqs))
        t_norm = _time_steps(torch, stream, args.steps, args.warmup, lambda: normalise_qk(q, k, wq, wk, 1e-6))
    io = 4 * seq * heads * dim * 2                        # q, k read; normalised q, k written
    table = seq * (dim // 2) * 4 * 4                      # the fp32 rotation table
    gbs = (io + table) / (t_rope * 1e-3) / 1e9
    return {
        "metric": "q/k RMSNorm + split-half RoPE ms + GB/s at 40,688 tok x 40 heads x 128, 1 GPU",
        "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": round(t_rope, 4), "dtype": "bf16",
        "config": {"workload": "qk_rmsnorm_rope_s40688_h40_d128", "seq_len": seq, "heads": heads, "head_dim": dim,
                   "rot_dim": dim, "bytes_per_step": io + table, "note": "rope table built in the timed call"},
        "roofline": {"bound": "hbm", "kernel": "qk_rmsnorm_rope_kernel<128>", "achieved": round(gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None},
        "plain_qk_rmsnorm_ms": round(t_norm, 4),
    }


CPU_THREADS = 16   # host threads of the CPU baseline: the host's CPU share for one GPU on the benchmark machine


MFMA_KINDS = {0: ("bf16_32x32x16", PEAK_BF16_TFLOPS), 1: ("int8_32x32x32", PEAK_I8_TOPS),
              2: ("fp8_e4m3_32x32x64", PEAK_F8_TFLOPS)}


def mfma_rate(torch, device, kind, data="random", reps=3, warmup=1):
    """Sustained MFMA rate (T(FL)OP/s, median of ``reps`` launches of 10-20 ms) of ``kind`` (0 bf16,
    1 int8, 2 fp8 e4m3) on register-resident operands (vdnh3_mfma_peak): random operands (what the
    kernels see: bf16 N(0,1), int8 uniform in [-127, 127], e4m3 codes of N(0,1)) or zeros, two
    workgroups of 4 wavefronts per CU, independent accumulators."""
    from vdn_h3_amd import _lib

    lib = _lib.lib()
    sh = _lib.stream_handle(device)
    stream = torch.cuda.current_stream(device)
    n = 8 * 64 * 32  # bytes per operand buffer
    gen = torch.Generator().manual_seed(20261202)
    if data == "zero":
        src = torch.zeros(n, dtype=torch.uint8)
    elif kind == 0:
        src = torch.randn(n // 2, generator=gen).to(torch.bfloat16).view(torch.uint8)
    elif kind == 1:
        src = torch.randint(-127, 128, (n,), generator=gen, dtype=torch.int8).view(torch.uint8)
    else:
        src = torch.randn(n, generator=gen).to(torch.float8_e4m3fn).view(torch.uint8)
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    blocks = 2 * cus  # one round: two workgroups per CU for the whole run
    out = torch.empty(blocks * 256, dtype=torch.float32, device=device)
    iters = {0: 40000, 1: 40000, 2: 20000}[kind]
    ops = lib.vdnh3_mfma_peak_ops(kind, iters, blocks)
    a, b = src.to(device), src.roll(4096).to(device)

    def run():
        _lib.check(lib.vdnh3_mfma_peak(kind, _lib.ptr(a), _lib.ptr(b), iters, blocks, _lib.ptr(out), sh), "mfma_peak")

    for _ in range(warmup):
        run()
    times = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run()
        e1.record(stream)
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1))
    times.sort()
    ms = times[len(times) // 2]
    return ops / (ms * 1e-3) / 1e12, ms


def ceiling_entry(torch, device, kind, achieved):
    """The kernel's rate against the part's sustained random-operand MFMA rate of the same kind,
    measured after the timed region (the datasheet ``roofline.peak`` assumes a clock the part holds
    only on operands that barely toggle)."""
    rate, _ = mfma_rate(torch, device, kind)
    return {"mfma": MFMA_KINDS[kind][0], "operands": "random", "rate": round(rate, 1),
            "achieved": round(achieved, 2), "frac": round(achieved / rate, 4),
            "source": "vdnh3_mfma_peak (bench.py --workload mfma_peak)"}


def bench_mfma_peak(args, torch, device):
    """Sustained MFMA rate of the part for every MFMA kind on random and zero operands: the ceiling
    the kernels' rates are read against besides the datasheet peak."""
    rates = {}
    for kind, (name, peak) in MFMA_KINDS.items():
        for data in ("random", "zero"):
            tops, ms = mfma_rate(torch, device, kind, data, reps=max(3, args.steps), warmup=max(1, args.warmup))
            rates[f"{name}_{data}"] = {"T_per_s": round(tops, 1), "frac_of_peak": round(tops / peak, 4),
                                       "ms": round(ms, 4)}
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    return {
        "metric": "sustained MFMA rate (register-resident operands)",
        "value": rates["bf16_32x32x16_random"]["T_per_s"],
        "unit": "TFLOP/s",
        "ms_per_step": rates["bf16_32x32x16_random"]["ms"],
        "dtype": "bf16/int8/fp8",
        "config": {"workload": "mfma_peak", "blocks": 2 * cus, "waves_per_cu": 8, "mfmas_per_wave_iter": 8},
        "rates": rates,
    }


def _cpu_description():
    """``(model name, physical cores)`` from /proc/cpuinfo (``platform.machine()`` / None if unreadable)."""
    model, cores, phys = None, set(), None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, value = line.partition(":")
            key, value = key.strip(), value.strip()
            if key == "model name" and model is None:
                model = value
            elif key == "physical id":
                phys = value
            elif key == "core id":
                cores.add((phys, value))
    except OSError:
        pass
    return model or platform.machine(), len(cores) or None


def _median_seconds(fn, reps=3):
    """Median wall time of ``reps`` runs of ``fn`` after one untimed warm-up run, and all the times."""
    fn()
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return sorted(times)[len(times) // 2], times


def _sample_rows(seq, n_rows, block=768):
    """About ``n_rows`` query rows as evenly spaced blocks of ``block`` consecutive rows (the first, middle
    and last of the sequence for 2304 rows: text and anchor rows with every key, interior frames with their
    window): rows of one block share a key set, so the oracle evaluates them as one product, as it does for
    the whole sequence; its key gather is paid once per block (scattered rows, or small blocks, time gathers
    and small products the full run amortises: 256-row blocks ran at 0.8x the 768-row rate)."""
    blocks = max(1, n_rows // block)
    starts = [round(i * (seq - block) / max(1, blocks - 1)) for i in range(blocks)]
    return [r for s in starts for r in range(s, min(seq, s + block))]


def _cpu_window_sample(torch, w, lay, qkv_host, n_rows):
    """``(FLOP, median s, times)`` of the window-attention oracle on ``n_rows`` query rows (``_sample_rows``)."""
    from oracle import window_oracle as wo
    from vdn_h3_amd import synth

    hq, hk, hv = synth.split_qkv(qkv_host, w.heads, w.head_dim)
    rows = _sample_rows(lay.seq_len, n_rows)
    keys = sum(b - a for r in rows for a, b in wo.row_key_intervals(
        r, lay.seq_len, lay.video_start, lay.video_end, lay.num_frames, lay.tokens_per_frame, lay.bounds,
        lay.anchor_frames))
    med, times = _median_seconds(lambda: wo.window_attention_rows(
        hq, hk, hv, rows, lay.video_start, lay.video_end, lay.num_frames, lay.tokens_per_frame, lay.bounds, w.scale,
        lay.anchor_frames))
    return 4.0 * w.head_dim * w.heads * keys, med, times


def cpu_baseline_window(torch, qkv, w, lay, n_rows):
    """The window-attention oracle (``oracle/window_oracle.py``) on the host cores, on ``n_rows`` query rows."""
    model, physical = _cpu_description()
    flops, med, times = _cpu_window_sample(torch, w, lay, qkv.cpu(), n_rows)
    return {"value": round(flops / med / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "seconds_median": round(med, 3), "seconds_runs": [round(t, 3) for t in times],
            "cpu": model, "physical_cores": physical,
            "sample": f"{n_rows} query rows (evenly spaced blocks of 768) x {w.heads} heads of the 40,688-row "
                      "layout, fp32 oracle (oracle/window_oracle.py); 1 warm-up, median of 3"}


def cpu_baseline_block(torch, device, lay, work, conv, n_rows):
    """CPU throughput of one hybrid block from bounded samples of its three parts, each the median of 3
    runs after a warm-up of the fp32 oracle on the host cores:

    * window attention: ``n_rows`` query rows (evenly spaced blocks of 768 rows) x 40 heads of the 40,688-row
      layout;
    * projections: ``oracle.branch_oracle.linear_bf16`` (fp32 GEMM, bf16 out) on 512 rows x K 5120 x N 15,360;
    * VDN branch: ``oracle.branch_oracle.projected_delta`` on 9 frames (7 inner) of 1296 tokens, 40 x 128,
      hidden 5120, text state and k/v short convolutions, scaled to the block's 29 inner frames.

    The block's CPU time is the sum of each part's work at its sampled rate; ``value`` is the block's
    work over that time. ``stack_extrapolated_s`` is 400 block calls (50 blocks x 8 steps) at that time.
    """
    from oracle import branch_oracle as bo
    from oracle import window_oracle as wo
    from vdn_h3_amd import synth

    model, physical = _cpu_description()
    w = synth.WINDOW_FULL
    qkv_host = synth.fused_qkv(lay.seq_len, w.heads, w.head_dim, device=device, seed=0, scale=w.scale).cpu()
    win_flop, win_s, win_times = _cpu_window_sample(torch, w, lay, qkv_host, n_rows)
    del qkv_host
    x = synth.randn((512, 5120), 60, dtype=torch.bfloat16)
    wt = synth.randn((15360, 5120), 61, dtype=torch.bfloat16, scale=0.02)
    proj_s, proj_times = _median_seconds(lambda: bo.linear_bf16(x, wt))
    proj_flop = 2.0 * 512 * 5120 * 15360
    del x, wt
    frames, inner, text, heads, dim, hidden, tpf = 9, 7, 512, w.heads, w.head_dim, 5120, lay.tokens_per_frame
    seq = text + frames * tpf
    bqkv = synth.fused_qkv(seq, heads, dim, seed=40)
    bx = synth.randn((seq, hidden), 41, dtype=torch.bfloat16)
    bw = synth.branch_weights(heads, dim, hidden, short_conv=conv)
    q, k, v = synth.split_qkv(bqkv, heads, dim)
    bounds = wo.window_bounds(frames, 1, 5)
    branch_s, branch_times = _median_seconds(lambda: bo.projected_delta(
        bw, bx[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, frame_size=lay.frame_size,
        text_x=bx[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True, short_conv=conv,
        fused_conv=True))
    inner_block = lay.num_frames - 2
    gemm_work = work["qkv_proj"] + work["out_proj"] + work["softmax_gate"]
    block_s = (work["window_attention"] / (win_flop / win_s) + gemm_work / (proj_flop / proj_s)
               + branch_s * inner_block / inner)
    total = sum(work.values())
    return {"value": round(total / block_s / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "cpu": model, "physical_cores": physical,
            "block_seconds_estimated": round(block_s, 2), "stack_extrapolated_s": round(400 * block_s, 1),
            "stack_note": "extrapolation: 50 blocks x 8 steps at the estimated CPU block time, not measured",
            "parts": {
                "window_attention": {"TFLOP/s": round(win_flop / win_s / 1e12, 5), "seconds_median": round(win_s, 3),
                                     "seconds_runs": [round(t, 3) for t in win_times],
                                     "sample": f"{n_rows} query rows (blocks of 768) x {heads} heads"},
                "projections": {"TFLOP/s": round(proj_flop / proj_s / 1e12, 5), "seconds_median": round(proj_s, 3),
                                "seconds_runs": [round(t, 3) for t in proj_times],
                                "sample": "512 x 5120 x 15360 fp32 GEMM, bf16 out"},
                "branch": {"seconds_median": round(branch_s, 3), "seconds_runs": [round(t, 3) for t in branch_times],
                           "sample": f"projected_delta, {frames} frames ({inner} inner) x {tpf} tokens, scaled by "
                                     f"{inner_block}/{inner}"}},
            "sample": "fp32 oracle on the host cores: window attention on sampled query rows, the projections on "
                      "sampled rows, the VDN branch on 7 of the 29 inner frames; each part the median of 3 runs after "
                      "a warm-up, combined at the block's per-part work"}


def bench_cpu_configs(args, torch, device):
    """The fp32 CPU oracle timed per benchmark configuration on the host cores, at full size (no sampling):
    1 warm-up, then the median of 3 (config 2: the warm-up runs on 2304 sampled rows, each full run is about a
    minute). Nothing here runs on the GPU.

    * config 1 / 1b: one hybrid block forward, 2 heads x 64, hidden 128, 16 text rows + 7 / 13 frames of 8 x 8
      tokens (7 frames is full cover: dense attention, no branch), ``oracle.hybrid_oracle.vdn_forward``;
    * config 2: the window attention at 40,688 x 40 x 128, ``oracle.window_oracle.window_attention_rows`` over
      every row (rows that share a key set batched, 8 heads at a time);
    * config 3: the VDN branch at the full shape (31 frames x 1296 tokens, skip_ends: 29 inner frames, 40 x
      128, hidden 5120, text state, k/v short convolutions), ``oracle.branch_oracle.projected_delta``; and the
      chunk-64 Gated DeltaNet at 40,688 x 40 x 128, ``oracle.gdn_oracle.chunked`` (float64);
    * config 4: the qkv (N 15,360) and out (N 5,120) projections at M 40,688, K 5,120 as the dequantised fp32
      ``F.linear`` the reference's projection falls back to on the CPU (``vdn_h3/fp8.py:253-266``).
    """
    import torch.nn.functional as F

    from oracle import branch_oracle as bo
    from oracle import gdn_oracle as go
    from oracle import hybrid_oracle as ho
    from oracle import window_oracle as wo
    from vdn_h3_amd import synth, window
    from vdn_h3_amd.gdn import gdn_flops
    from vdn_h3_amd.layout import text_first_layout

    del device
    model, physical = _cpu_description()
    parts = {}

    def record(name, work, unit, med, times, sample):
        parts[name] = {"seconds_median": round(med, 4), "seconds_runs": [round(t, 4) for t in times],
                       "work": work, "rate": round(work / med / 1e12, 5), "rate_unit": unit, "sample": sample}
        print(f"cpu_configs: {name}: {med:.3f} s ({work / med / 1e12:.4f} {unit})", file=sys.stderr, flush=True)

    # configs 1 and 1b: the CPU-plumbing block
    for name, frames in (("config1_block_s464_h2_d64", 7), ("config1b_block_s848_h2_d64_13f", 13)):
        heads, dim, hidden = 2, 64, 128
        lay = text_first_layout(16, frames, (8, 8))
        x = synth.randn((lay.seq_len, hidden), 70, dtype=torch.bfloat16)
        bw = synth.branch_weights(heads, dim, hidden, seed=170)
        aw = {"qkv_proj.weight": synth.randn((3 * heads * dim, hidden), 71, dtype=torch.bfloat16, scale=0.02),
              "out_proj.weight": synth.randn((hidden, heads * dim), 72, dtype=torch.bfloat16, scale=0.02),
              "q_norm.weight": (1 + 0.1 * synth.randn((dim,), 73)).to(torch.bfloat16),
              "k_norm.weight": (1 + 0.1 * synth.randn((dim,), 74)).to(torch.bfloat16)}
        pairs = wo.pair_count(lay.seq_len, lay.video_start, lay.video_end, lay.num_frames, lay.tokens_per_frame,
                              list(lay.bounds), lay.anchor_frames)
        flop = window.attention_flops(pairs, heads, dim) + 2.0 * lay.seq_len * hidden * 4 * heads * dim
        med, times = _median_seconds(lambda: ho.vdn_forward(x, lay, aw, bw, heads, dim))
        record(name, flop, "TFLOP/s", med, times,
               f"whole block ({'full cover, dense' if lay.full_cover else 'window + branch'}); work = attention "
               "+ qkv / out projections")

    # config 2: the window attention at the full shape
    w = synth.WINDOW_FULL
    lay = w.layout
    qkv = synth.fused_qkv(lay.seq_len, w.heads, w.head_dim, seed=0, scale=w.scale)
    q, k, v = synth.split_qkv(qkv, w.heads, w.head_dim)
    geo = (lay.video_start, lay.video_end, lay.num_frames, lay.tokens_per_frame, lay.bounds, w.scale,
           lay.anchor_frames)
    wo.window_attention_rows(q, k, v, torch.linspace(0, lay.seq_len - 1, 2304).long().tolist(), *geo)
    rows = list(range(lay.seq_len))
    times = []
    for _ in range(3):
        t = time.perf_counter()
        wo.window_attention_rows(q, k, v, rows, *geo)
        times.append(time.perf_counter() - t)
        print(f"cpu_configs: window full run {len(times)}: {times[-1]:.1f} s", file=sys.stderr, flush=True)
    pairs = wo.pair_count(lay.seq_len, lay.video_start, lay.video_end, lay.num_frames, lay.tokens_per_frame,
                          list(lay.bounds), lay.anchor_frames)
    record("config2_window_s40688_h40_d128", window.attention_flops(pairs, w.heads, w.head_dim), "TFLOP/s",
           sorted(times)[1], times, "every query row, fp32; warm-up on 2304 sampled rows")
    del qkv, q, k, v

    # config 3: the VDN branch at the full shape, and the chunk-64 Gated DeltaNet
    heads, dim, hidden, tpf, text = w.heads, w.head_dim, 5120, lay.tokens_per_frame, lay.text_len
    frames = lay.num_frames
    seq = text + frames * tpf
    conv = ("k", "v")
    bqkv = synth.fused_qkv(seq, heads, dim, seed=40)
    bx = synth.randn((seq, hidden), 41, dtype=torch.bfloat16)
    bw = synth.branch_weights(heads, dim, hidden, short_conv=conv)
    q, k, v = synth.split_qkv(bqkv, heads, dim)
    bounds = wo.window_bounds(frames, 1, 5)
    work = block_flops(lay, heads, dim, hidden, pairs, conv)
    branch_work = (work["branch_core"] + work["branch_gates"] + work["branch_text_state"]
                   + work["branch_short_conv"] + work["to_out_linear"])
    med, times = _median_seconds(lambda: bo.projected_delta(
        bw, bx[text:], q[text:], k[text:], v[text:], frames, tpf, bounds, frame_size=lay.frame_size,
        text_x=bx[:text], text_k_raw=k[:text], text_v_raw=v[:text], skip_ends=True, short_conv=conv,
        fused_conv=True))
    record("config3_vdn_branch_f31_t1296_h40_d128", branch_work, "TFLOP/s", med, times,
           "projected_delta, 31 frames (29 inner) x 1296 tokens, text state, k/v short convolutions, "
           "to_out_linear")
    del bqkv, bx, q, k, v
    tokens = lay.seq_len
    g = torch.Generator().manual_seed(50)
    gq = torch.randn(tokens, heads, dim, generator=g).to(torch.bfloat16)
    gk = F.normalize(torch.randn(tokens, heads, dim, generator=g), dim=-1).to(torch.bfloat16)
    gv = torch.randn(tokens, heads, dim, generator=g).to(torch.bfloat16)
    gb = torch.sigmoid(torch.randn(tokens, heads, generator=g))
    gg = -F.softplus(torch.randn(tokens, heads, generator=g))
    med, times = _median_seconds(lambda: go.chunked(gq, gk, gv, gb, gg))
    record("config3_gdn_chunk64_t40688_h40_d128", gdn_flops(tokens, heads, dim), "TFLOP/s", med, times,
           "all tokens and heads, float64 chunk form")
    del gq, gk, gv

    # config 4: the projections as the CPU fallback computes them
    x = synth.randn((tokens, hidden), 60, dtype=torch.float32)
    for name, n in (("config4_qkv_m40688_k5120_n15360", 3 * heads * dim), ("config4_out_m40688_k5120_n5120", hidden)):
        wt = synth.randn((n, hidden), 61, scale=0.02)
        med, times = _median_seconds(lambda: F.linear(x, wt))
        record(name, 2.0 * tokens * hidden * n, "TFLOP/s", med, times, "dequantised fp32 F.linear")
        del wt
    return {
        "metric": "fp32 CPU oracle seconds per benchmark configuration on the host cores",
        "value": parts["config2_window_s40688_h40_d128"]["rate"],
        "unit": "TFLOP/s",
        "ms_per_step": round(1e3 * parts["config2_window_s40688_h40_d128"]["seconds_median"], 1),
        "dtype": "f32",
        "config": {"workload": "cpu_configs", "cpu": model, "physical_cores": physical,
                   "threads": torch.get_num_threads(), "kind": "port"},
        "parts": parts,
    }


def main():
    args = _parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} (WORLD_SIZE={world}) is not supported: this "
              "library has no multi-GPU path; the hot path would shard by head, one process per GPU.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(1)
    torch.set_num_threads(min(CPU_THREADS, os.cpu_count() or 1))
    device = torch.device("cuda:0")
    if args.workload == "block":
        result = bench_block(args, torch, device)
        if args.cpu_sample_rows > 0:
            from vdn_h3_amd import synth

            result["cpu_baseline"] = cpu_baseline_block(torch, device, synth.WINDOW_FULL.layout,
                                                        result["config"]["work_per_step"], _short_conv(args),
                                                        args.cpu_sample_rows)
    elif args.workload == "stack":
        result = bench_stack(args, torch, device)
    elif args.workload == "hbm_copy":
        result = bench_hbm_copy(args, torch, device)
    elif args.workload == "branch":
        result = bench_branch(args, torch, device)
    elif args.workload.startswith("gemm_"):
        result = bench_gemm(args, torch, device)
    elif args.workload == "gdn":
        result = bench_gdn(args, torch, device)
    elif args.workload == "dit":
        result = bench_dit(args, torch, device)
    elif args.workload == "rope":
        result = bench_rope(args, torch, device)
    elif args.workload == "mfma_peak":
        result = bench_mfma_peak(args, torch, device)
    elif args.workload == "cpu_configs":
        result = bench_cpu_configs(args, torch, device)
    else:
        result = bench_window(args, torch, device)
    line = {
        "metric": result.pop("metric"),
        "value": result.pop("value"),
        "unit": result.pop("unit"),
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": result.pop("ms_per_step"),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": result.pop("dtype"),
        "data": "synthetic (seeded N(0,1) bf16 q/k/v, random-init)",
        "config": result.pop("config"),
        **result,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
