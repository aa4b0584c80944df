#!/usr/bin/env python3
"""Benchmark of the VDN-H3 hybrid attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload window]

Prints one JSON line. Workload ``window``: exact local-window softmax attention at the
full shape (512 text rows + 31 frames x 1296 tokens = 40 688 rows, 40 heads x 128,
chunk 5, radius 1, anchors both), inputs resident in HBM before timing. A step is one
call of the op (V^T pre-pass + attention kernel). ``value`` is algorithmic TFLOP/s of
the step (``4 * D * H * allowed pairs``, masked tile work and exp not counted);
``roofline`` is the attention kernel alone, timed with HIP events on the stream it
runs on; ``cpu_baseline`` times the CPU oracle on a bounded sample of query rows.
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


def _parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="window", choices=["window", "hbm_copy"],
                    help="hbm_copy: a plain 1 GiB device copy, the reference point for scaling rocprofv3's "
                         "FETCH_SIZE / WRITE_SIZE counters to bytes")
    ap.add_argument("--cpu-sample-rows", type=int, default=2048,
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
    lay = w.layout
    qkv = synth.fused_qkv(lay.seq_len, w.heads, w.head_dim, device=device, seed=0)
    q, k, v = synth.split_qkv(qkv, w.heads, w.head_dim)
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
        "roofline": {"bound": "mfma", "kernel": "window_attn_kernel<128>", "achieved": round(attn_tflops, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(attn_tflops / PEAK_BF16_TFLOPS, 4),
                     "kernel_ms": round(attn_ms, 4), "traffic": _traffic(args.traffic_json, "window_attn_kernel")},
        "breakdown_ms": {"vt_prepass": round(ms_step - attn_ms, 4), "window_attn": round(attn_ms, 4)},
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


def cpu_baseline_window(torch, qkv, w, lay, n_rows):
    """Time the CPU oracle (``oracle.window_oracle``) on ``n_rows`` query rows of the same problem."""
    from oracle import window_oracle as wo
    from vdn_h3_amd import synth

    host = qkv.cpu()
    hq, hk, hv = synth.split_qkv(host, w.heads, w.head_dim)
    seq = lay.seq_len
    rows = torch.linspace(0, seq - 1, n_rows).long().tolist()
    keys = 0
    for r in rows:
        keys += sum(b - a for a, b in wo.row_key_intervals(r, seq, lay.video_start, lay.video_end, lay.num_frames,
                                                          lay.tokens_per_frame, lay.bounds, lay.anchor_frames))
    t = time.perf_counter()
    wo.window_attention_rows(hq, hk, hv, rows, lay.video_start, lay.video_end, lay.num_frames,
                             lay.tokens_per_frame, lay.bounds, w.scale, lay.anchor_frames)
    dt = time.perf_counter() - t
    flops = 4.0 * w.head_dim * w.heads * keys
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "seconds": round(dt, 2), "cpu": platform.processor() or platform.machine(),
            "sample": f"{n_rows} evenly spaced query rows x {w.heads} heads of the 40,688-row layout, "
                      f"fp32 oracle (oracle/window_oracle.py), {keys} keys in total"}


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
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    device = torch.device("cuda:0")
    if args.workload == "hbm_copy":
        result = bench_hbm_copy(args, torch, device)
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
