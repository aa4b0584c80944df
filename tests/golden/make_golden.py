"""Write golden vectors for the branch and hybrid-block composites from the reference itself.

Run in the build container only (it reads the reference checkout, which the GPU hosts do
not have):

    python tests/golden/make_golden.py [/root/reference [NAME ...]]

(NAME: the file names below; all of them by default).

It imports ``vdn_h3`` of hyukudan/ComfyUI-Kirei-VDN-H3 v0.3.3 on the CPU and saves small
inputs / outputs as safetensors next to this script:

* ``branch_13f.safetensors``      - ``OptimizedLinearBranch.projected_delta`` (inference, skip_ends,
  text state, no short conv), and ``readout`` on the inner frames (``vdn_h3/runtime.py:545-607``);
* ``branch_13f_conv.safetensors`` - the same with the K/V short convolutions
  (``vdn_h3/runtime.py:319-341``);
* ``hybrid_13f.safetensors``      - ``make_vdn_forward`` on a windowed 13-frame layout
  (``vdn_h3/hybrid.py:409-579``): qkv, q/k RMSNorm, window attention, softmax gate,
  out-projection and the branch delta;
* ``branch_13f_sana.safetensors`` - ``projected_delta`` and ``readout`` with
  ``delta_rule="sana_scaled"`` (``SanaDelta``, ``vdn_h3/branch.py:163-177``) and the text state;
* ``branch_13f_abf16.safetensors`` - ``projected_delta`` and ``readout`` with ``a_fp32=False``
  (A from the bf16 product of ``k~ * beta`` and ``k~``, ``vdn_h3/branch.py:235-240``);
* ``dit_block.safetensors``       - ``make_fast_block_forward`` (``vdn_h3/block_kernels.py:149-240``)
  on a stand-in DiT block (RMSNorm weights, six AdaLN tables, a linear attention, a SwiGLU
  MLP) with a two-segment modulation map. The fused path only runs for device tensors; its
  torch ops are device-independent, so the input is a CPU tensor whose ``is_cuda`` reads
  True, and the state's compiler cache calls each pointwise body eagerly.

Only these composites need the reference: every other oracle function is pinned by
closed forms in the tests.
"""

from __future__ import annotations

import sys
from pathlib import Path

import torch
import torch.nn as nn
import torch.nn.functional as F
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

FRAMES, GRID, TEXT, HEADS, DIM, HIDDEN = 13, (8, 8), 16, 2, 64, 128
TPF = GRID[0] * GRID[1]


def gen(k):
    return torch.Generator().manual_seed(20261201 + k)


def branch_weights(short_conv):
    w = {
        "beta_proj.weight": torch.randn(HEADS, HIDDEN, generator=gen(101)) * 0.02,
        "alpha.down.weight": torch.randn(DIM, HIDDEN, generator=gen(102)) * 0.02,
        "alpha.up.weight": torch.randn(HEADS * DIM, DIM, generator=gen(103)) * 0.02,
        "alpha.dt_bias": torch.randn(HEADS * DIM, generator=gen(104)) * 0.5,
        "alpha.A_log": torch.randn(HEADS, generator=gen(105)) * 0.5,
        "output_gate.down.weight": torch.randn(DIM, HIDDEN, generator=gen(106)) * 0.02,
        "output_gate.up.weight": torch.randn(HEADS * DIM, DIM, generator=gen(107)) * 0.02,
        "output_gate.up.bias": torch.randn(HEADS * DIM, generator=gen(108)) * 0.5,
        "norm.weight": 1.0 + 0.1 * torch.randn(DIM, generator=gen(109)),
        "to_out_linear.weight": torch.randn(HIDDEN, HEADS * DIM, generator=gen(110)) * 0.02,
        "softmax_gate.up.weight": torch.randn(HEADS, HIDDEN, generator=gen(111)) * 0.02,
        "softmax_gate.up.bias": torch.randn(HEADS, generator=gen(112)) * 0.5,
    }
    if short_conv:
        for name in ("k", "v"):
            w[f"short_conv.{name}_sp.weight"] = torch.randn(HEADS * DIM, 1, 5, 5, generator=gen(113)) * 0.2
            w[f"short_conv.{name}_tm.weight"] = torch.randn(HEADS * DIM, 1, 5, generator=gen(114)) * 0.4
    out = {}
    for key, value in w.items():
        keep_fp32 = key in ("alpha.A_log", "alpha.dt_bias")
        out[key] = value.float() if keep_fp32 else value.to(torch.bfloat16)
    return out


def make_branch(short_conv, delta_rule="vdn_solve", a_fp32=True):
    from vdn_h3.runtime import OptimizedLinearBranch
    from vdn_h3.window import window_bounds

    weights = branch_weights(short_conv)
    seq = TEXT + FRAMES * TPF
    x = (torch.randn(seq, HIDDEN, generator=gen(1))).to(torch.bfloat16)
    qkv = torch.randn(seq, 3 * HEADS * DIM, generator=gen(2)).to(torch.bfloat16)
    q, k, v = [t.reshape(seq, HEADS, DIM) for t in qkv.split(HEADS * DIM, dim=-1)]
    bounds = window_bounds(FRAMES, 1, 5)
    conv = ("k", "v") if short_conv else ()
    branch = OptimizedLinearBranch(weights, HEADS, DIM, delta_rule=delta_rule, short_conv=conv,
                                   enable_text_state=True, kernel_backend="eager", compile_policy="off",
                                   tile_frames=0, a_fp32=a_fp32)
    va, vb = TEXT, seq
    with torch.inference_mode():
        delta = branch.projected_delta(
            weights, x[va:vb], q[va:vb], k[va:vb], v[va:vb], FRAMES, TPF, bounds, frame_size=GRID,
            text_x=x[:TEXT], text_k_raw=k[:TEXT], text_v_raw=v[:TEXT], skip_ends=True, inference=True)
        readout = branch.readout(
            weights, x[va:vb], q[va:vb], k[va:vb], v[va:vb], FRAMES, TPF, bounds, frame_size=GRID,
            text_x=x[:TEXT], text_k_raw=k[:TEXT], text_v_raw=v[:TEXT], skip_ends=True, inference=True)
    tensors = {f"w.{key}": value.contiguous() for key, value in weights.items()}
    tensors.update({"x": x, "qkv": qkv, "delta": delta.contiguous(), "readout": readout.contiguous()})
    meta = {"frames": str(FRAMES), "grid": f"{GRID[0]}x{GRID[1]}", "text": str(TEXT), "heads": str(HEADS),
            "dim": str(DIM), "hidden": str(HIDDEN), "short_conv": ",".join(conv), "radius": "1", "chunk": "5",
            "delta_rule": delta_rule, "a_fp32": str(bool(a_fp32)).lower(),
            "source": "vdn_h3.runtime.OptimizedLinearBranch.projected_delta / readout (inference, skip_ends)"}
    name = "branch_13f_conv.safetensors" if short_conv else "branch_13f.safetensors"
    if delta_rule != "vdn_solve":
        name = "branch_13f_sana.safetensors"
    if not a_fp32:
        name = "branch_13f_abf16.safetensors"
    save_file(tensors, str(HERE / name), metadata=meta)
    return name


class _RMS(nn.Module):
    def __init__(self, dim, seed):
        super().__init__()
        self.weight = nn.Parameter((1.0 + 0.1 * torch.randn(dim, generator=gen(seed))).to(torch.bfloat16))
        self.eps = 1e-6

    def forward(self, x):
        return F.rms_norm(x, (x.shape[-1],), self.weight, self.eps)


class _Attention(nn.Module):
    """The attributes make_vdn_forward reads from a MiniMax-H3 attention (vdn_h3/hybrid.py:591-597)."""

    def __init__(self):
        super().__init__()
        self.heads, self.head_dim = HEADS, DIM
        self.qkv_proj = nn.Linear(HIDDEN, 3 * HEADS * DIM, bias=False).to(torch.bfloat16)
        self.out_proj = nn.Linear(HEADS * DIM, HIDDEN, bias=False).to(torch.bfloat16)
        with torch.no_grad():
            self.qkv_proj.weight.copy_(torch.randn(3 * HEADS * DIM, HIDDEN, generator=gen(201)) * 0.1)
            self.out_proj.weight.copy_(torch.randn(HIDDEN, HEADS * DIM, generator=gen(202)) * 0.05)
        self.q_norm = _RMS(DIM, 203)
        self.k_norm = _RMS(DIM, 204)

    def forward(self, x, rope_freqs=None, transformer_options=None):  # pragma: no cover - not used with a layout
        raise AssertionError("the patched forward must not fall back to the original")


def make_hybrid():
    from vdn_h3.hybrid import VDNState, make_vdn_forward
    from vdn_h3.layout import VDNLayout, publish_layout
    from vdn_h3.runtime import OptimizedLinearBranch
    from vdn_h3.window import full_coverage, window_bounds

    weights = branch_weights(False)
    attn = _Attention()
    branch = OptimizedLinearBranch(weights, HEADS, DIM, short_conv=(), enable_text_state=True,
                                   kernel_backend="eager", compile_policy="off", tile_frames=0)
    config = {"enable_softmax_gate": True, "linear_enabled": True, "enable_text_state": True}
    state = VDNState("golden", config, [branch], HEADS, DIM, weight_mode="resident", attention_backend="grouped",
                     inference=True, kernel_backend="eager", compile_policy="off")
    seq = TEXT + FRAMES * TPF
    bounds = tuple(window_bounds(FRAMES, 1, 5))
    layout = VDNLayout(seq_len=seq, video_start=TEXT, video_end=seq, num_frames=FRAMES, tokens_per_frame=TPF,
                       frame_size=GRID, text_start=0, text_len=TEXT, bounds=bounds,
                       full_cover=full_coverage(bounds, FRAMES), anchor_frames="both")
    x = torch.randn(seq, HIDDEN, generator=gen(3)).to(torch.bfloat16)
    forward = make_vdn_forward(attn, state, 0)
    with torch.inference_mode(), publish_layout(layout):
        out = forward(x)
    tensors = {f"w.{key}": value.contiguous() for key, value in weights.items()}
    tensors.update({"x": x, "out": out.contiguous(), "attn.qkv_proj.weight": attn.qkv_proj.weight.detach(),
                    "attn.out_proj.weight": attn.out_proj.weight.detach(),
                    "attn.q_norm.weight": attn.q_norm.weight.detach(),
                    "attn.k_norm.weight": attn.k_norm.weight.detach()})
    meta = {"frames": str(FRAMES), "grid": f"{GRID[0]}x{GRID[1]}", "text": str(TEXT), "heads": str(HEADS),
            "dim": str(DIM), "hidden": str(HIDDEN), "anchor_frames": "both", "radius": "1", "chunk": "5",
            "source": "vdn_h3.hybrid.make_vdn_forward (inference, grouped attention, text state, gate on)",
            "last_attention_backend": str(state.last_attention_backend)}
    save_file(tensors, str(HERE / "hybrid_13f.safetensors"), metadata=meta)
    return "hybrid_13f.safetensors"


DIT_ROWS, DIT_HIDDEN, DIT_FFN = 96, 128, 192


class _ReportsDevice(torch.Tensor):
    """A CPU tensor whose ``is_cuda`` reads True, so ``make_fast_block_forward`` takes its fused path."""

    @property
    def is_cuda(self):
        return True


class _EagerCompiler:
    """The compiler cache ``_compiled`` calls (``vdn_h3/block_kernels.py:96-105``), running each body eagerly."""

    def call(self, name, fn, args, key, *, policy=None):
        del name, key, policy
        return fn(*args)


def make_dit_block():
    from types import SimpleNamespace

    from vdn_h3.block_kernels import make_fast_block_forward
    from vdn_h3.diagnostics import DiagnosticsRecorder

    hidden, ffn = DIT_HIDDEN, DIT_FFN
    w = {
        "norm1.weight": 1.0 + 0.1 * torch.randn(hidden, generator=gen(301)),
        "norm2.weight": 1.0 + 0.1 * torch.randn(hidden, generator=gen(302)),
        "attn.weight": 0.08 * torch.randn(hidden, hidden, generator=gen(303)),
        "fc1.weight": 0.08 * torch.randn(2 * ffn, hidden, generator=gen(304)),
        "fc2.weight": 0.08 * torch.randn(hidden, ffn, generator=gen(305)),
    }
    w = {k: v.to(torch.bfloat16) for k, v in w.items()}
    # six distinct [2, hidden] fp32 tables: a mix-up of any two changes the output
    names = ("shift_msa", "scale_msa", "gate_msa", "shift_mlp", "scale_mlp", "gate_mlp")
    mod = {n: (0.4 * torch.randn(2, hidden, generator=gen(310 + i)) + 0.1 * (i + 1)) for i, n in enumerate(names)}

    def norm(weight):
        return SimpleNamespace(weight=weight, eps=1e-6)

    attn_lin = nn.Linear(hidden, hidden, bias=False).to(torch.bfloat16)
    fc1 = nn.Linear(hidden, 2 * ffn, bias=False).to(torch.bfloat16)
    fc2 = nn.Linear(ffn, hidden, bias=False).to(torch.bfloat16)
    with torch.no_grad():
        attn_lin.weight.copy_(w["attn.weight"])
        fc1.weight.copy_(w["fc1.weight"])
        fc2.weight.copy_(w["fc2.weight"])

    def attn(h, rope_freqs=None, transformer_options=None):
        return attn_lin(h)

    block = SimpleNamespace(norm1=norm(w["norm1.weight"]), norm2=norm(w["norm2.weight"]), attn=attn,
                            mlp=SimpleNamespace(fc1=fc1, fc2=fc2),
                            adaln_proj=lambda t_emb: tuple(mod[n] for n in names),
                            forward=lambda *a, **k: (_ for _ in ()).throw(AssertionError("fallback taken")))
    state = SimpleNamespace(block_fusion=True, inference=True, weight_mode="resident", compile_policy="shared",
                            branch_runtime=SimpleNamespace(compiler=_EagerCompiler()),
                            diagnostics=DiagnosticsRecorder(False))
    x = (2.0 * torch.randn(DIT_ROWS, hidden, generator=gen(320))).to(torch.bfloat16)
    segments = [(0, 40, 0), (40, DIT_ROWS, 1)]
    forward = make_fast_block_forward(block, state, 0)
    with torch.inference_mode():
        out = forward(x.as_subclass(_ReportsDevice), torch.zeros(1), segments, None)
    out = torch.Tensor(out).as_subclass(torch.Tensor)
    tensors = {f"w.{k}": v.contiguous() for k, v in w.items()}
    tensors.update({f"mod.{n}": mod[n].contiguous() for n in names})
    tensors.update({"x": x, "out": out.contiguous()})
    meta = {"rows": str(DIT_ROWS), "hidden": str(hidden), "ffn": str(ffn), "segments": "0:40:0,40:96:1",
            "eps": "1e-6", "source": "vdn_h3.block_kernels.make_fast_block_forward (fused path, bf16 MLP)"}
    save_file(tensors, str(HERE / "dit_block.safetensors"), metadata=meta)
    return "dit_block.safetensors"


def main():
    if not (REF / "vdn_h3").is_dir():
        raise SystemExit(f"reference checkout not found at {REF}")
    sys.path.insert(0, str(REF))
    torch.set_num_threads(4)
    makers = {"branch_13f.safetensors": lambda: make_branch(False),
              "branch_13f_conv.safetensors": lambda: make_branch(True),
              "hybrid_13f.safetensors": make_hybrid,
              "branch_13f_sana.safetensors": lambda: make_branch(False, "sana_scaled"),
              "dit_block.safetensors": make_dit_block,
              "branch_13f_abf16.safetensors": lambda: make_branch(False, a_fp32=False)}
    wanted = sys.argv[2:] or list(makers)
    for name in wanted:
        print("wrote", HERE / makers[name]())


if __name__ == "__main__":
    main()
