"""The window attention with the block's q_norm / k_norm (and RoPE) fused in (GPU).

Bar: bit-identity with the separate path it replaces, the standalone q/k pass
(``vdnh3_qk_rmsnorm`` / ``_rope``, pinned against the oracle in ``test_hybrid_gpu.py``) followed by
the attention on the normalised q / k (``vdnh3_window_attn_prepared``, pinned in
``test_window_gpu.py``): the fused kernels follow the same arithmetic in the same order, so every
output bit must agree. The pre-pass's normalised keys are compared the same way, and rows past
the sequence must be zero.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import window_oracle as wo

pytestmark = pytest.mark.gpu


def _freqs(rows, rot, seed):
    g = torch.Generator().manual_seed(seed)
    theta = torch.randn(rows, rot // 2, generator=g) * 3
    c, s = torch.cos(theta), torch.sin(theta)
    return torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2).reshape(1, rows, 1, rot // 2, 2, 2)


def _inputs(seq, heads, dim, seed, device):
    from vdn_h3_amd import synth

    qkv = (3 * synth.randn((seq, 3 * heads * dim), seed)).to(torch.bfloat16).to(device)
    q, k, v = synth.split_qkv(qkv, heads, dim)
    wq = (1 + 0.1 * synth.randn((dim,), seed + 1)).to(torch.bfloat16).to(device)
    wk = (1 + 0.1 * synth.randn((dim,), seed + 2)).to(torch.bfloat16).to(device)
    return q, k, v, wq, wk


# rot: None = no RoPE; rot 48 puts the split-half partner 24 channels away (not a 16-channel step)
CASES = [(128, None, False), (64, None, False), (128, 128, False), (128, 64, True), (128, 48, False),
         (64, 64, False), (64, 32, True)]


@pytest.mark.parametrize("dim,rot,shared", CASES)
@pytest.mark.parametrize("with_queries", [False, True])
def test_qkv_prepass_matches_qk_pass(device, dim, rot, shared, with_queries):
    from vdn_h3_amd import _lib
    from vdn_h3_amd.hybrid import normalise_qk
    from vdn_h3_amd.window import rope_table

    seq, heads, q_eps, k_eps = 1000, 3, 1e-6, 1e-5
    if rot is not None:  # with RoPE the q/k pass takes one epsilon for both
        q_eps = k_eps
    print(f"case qkv_prepass D={dim} rot={rot} shared={shared} queries={with_queries}", flush=True)
    q, k, v, wq, wk = _inputs(seq, heads, dim, 300 + dim + (rot or 0), device)
    freqs = None if rot is None else _freqs(1 if shared else seq, rot, 7).to(device)
    want_q, want_k = normalise_qk(q, k, wq, wk, q_eps, rope_freqs=freqs, k_eps=k_eps)
    lib = _lib.lib()
    ws_bytes = lib.vdnh3_window_norm_workspace_bytes(seq, heads, dim, int(with_queries))
    ws = torch.full((ws_bytes,), 0x5A, dtype=torch.uint8, device=device)  # junk: the pass must write every byte
    table, f_row, rot_dim = (None, 0, 0) if freqs is None else rope_table(freqs, seq, dim, device)
    rc = lib.vdnh3_window_qkv_prepass(_lib.ptr(q) if with_queries else None, q.stride(0), q.stride(1), _lib.ptr(wq),
                                      q_eps, _lib.ptr(k), k.stride(0), k.stride(1), _lib.ptr(wk), k_eps, _lib.ptr(v),
                                      v.stride(0), v.stride(1), _lib.ptr(table), f_row, rot_dim, seq, heads, dim,
                                      _lib.ptr(ws), ws_bytes, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_window_qkv_prepass")
    region = lib.vdnh3_window_workspace_bytes(seq, heads, dim)
    vt_ref = torch.empty(region, dtype=torch.uint8, device=device)
    _lib.check(lib.vdnh3_window_vt_prepass(_lib.ptr(v), v.stride(0), v.stride(1), seq, heads, dim, _lib.ptr(vt_ref),
                                           region, _lib.stream_handle(device)), "vdnh3_window_vt_prepass")
    torch.cuda.synchronize()
    s_pad = region // (2 * heads * dim)  # the rows of each workspace region (seq padded)
    assert ws_bytes == (3 if with_queries else 2) * region
    assert torch.equal(ws[:region].cpu(), vt_ref.cpu())
    for r, want in ((1, want_k), (2, want_q))[:2 if with_queries else 1]:
        got = ws[r * region:(r + 1) * region].view(torch.bfloat16).view(heads, s_pad, dim)
        assert torch.equal(got[:, :seq].permute(1, 0, 2).cpu().view(torch.int16), want.cpu().view(torch.int16)), r
        assert not got[:, seq:].float().abs().sum().item(), r


def _geometry(frames=13, per_frame=64, text=16):
    seq = text + frames * per_frame
    return dict(seq=seq, vs=text, ve=seq, frames=frames, per_frame=per_frame,
                bounds=wo.window_bounds(frames, 1, 5))


@pytest.mark.parametrize("dim,rot,shared", CASES)
@pytest.mark.parametrize("gated", [False, True])
def test_fused_attention_matches_separate(device, dim, rot, shared, gated):
    from vdn_h3_amd import window
    from vdn_h3_amd.hybrid import normalise_qk

    geo = _geometry()
    seq, heads = geo["seq"], 3
    q_eps, k_eps = 1e-6, 1e-5 if rot is None else 1e-6
    print(f"case fused attention D={dim} rot={rot} shared={shared} gated={gated}", flush=True)
    q, k, v, wq, wk = _inputs(seq, heads, dim, 400 + dim + (rot or 0), device)
    freqs = None if rot is None else _freqs(1 if shared else seq, rot, 8).to(device)
    gate = torch.sigmoid(torch.randn(seq, heads, generator=torch.Generator().manual_seed(5))).to(
        torch.bfloat16).to(device) if gated else None
    args = (geo["vs"], geo["ve"], geo["frames"], geo["per_frame"], geo["bounds"], dim ** -0.5, "both")
    qn, kn = normalise_qk(q, k, wq, wk, q_eps, rope_freqs=freqs, k_eps=k_eps)
    want = window.window_softmax_hip(qn, kn, v, *args, gate=gate)
    got = window.window_softmax_normed(q, k, v, wq, wk, q_eps, k_eps, *args, rope_freqs=freqs, gate=gate)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got.cpu().view(torch.int16), want.cpu().view(torch.int16))


def test_fused_attention_full_shape(device):
    """The full window workload (40688 rows, 40 heads, 128 dims, RoPE on every row): the fused
    path gives the same bits as the separate q/k pass and attention."""
    from vdn_h3_amd import synth, window
    from vdn_h3_amd.hybrid import normalise_qk

    w = synth.WINDOW_FULL
    lay = w.layout
    seq, heads, dim = lay.seq_len, w.heads, w.head_dim
    print(f"case fused attention full shape S={seq} H={heads} D={dim}", flush=True)
    q, k, v, wq, wk = _inputs(seq, heads, dim, 500, device)
    freqs = _freqs(seq, dim, 9).to(device)
    cache = window.WindowAttentionCache()
    args = (lay.video_start, lay.video_end, lay.num_frames, lay.tokens_per_frame, lay.bounds, dim ** -0.5,
            lay.anchor_frames, cache)
    qn, kn = normalise_qk(q, k, wq, wk, 1e-6, rope_freqs=freqs)
    want = window.window_softmax_hip(qn, kn, v, *args)
    del qn, kn
    got = window.window_softmax_normed(q, k, v, wq, wk, 1e-6, 1e-6, *args, rope_freqs=freqs)
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_normed_rejects_bad_arguments(device):
    from vdn_h3_amd import _lib, window

    geo = _geometry(frames=3)
    seq, heads, dim = geo["seq"], 2, 128
    q, k, v, wq, wk = _inputs(seq, heads, dim, 600, device)
    args = (geo["vs"], geo["ve"], geo["frames"], geo["per_frame"], geo["bounds"], dim ** -0.5)
    with pytest.raises(ValueError, match="entries"):
        window.window_softmax_normed(q, k, v, wq[:64], wk, 1e-6, 1e-6, *args)
    with pytest.raises(ValueError, match="rot_dim"):
        window.window_softmax_normed(q, k, v, wq, wk, 1e-6, 1e-6, *args, rope_freqs=_freqs(seq, 24, 1).to(device))
    lib = _lib.lib()
    ws_bytes = lib.vdnh3_window_norm_workspace_bytes(seq, heads, dim, 0)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    sh = _lib.stream_handle(device)

    def prepass(q_ptr, ws_ptr, nbytes):
        return lib.vdnh3_window_qkv_prepass(q_ptr, q.stride(0), q.stride(1), _lib.ptr(wq), 1e-6, _lib.ptr(k),
                                            k.stride(0), k.stride(1), _lib.ptr(wk), 1e-6, _lib.ptr(v), v.stride(0),
                                            v.stride(1), None, 0, 0, seq, heads, dim, ws_ptr, nbytes, sh)

    assert prepass(None, _lib.ptr(ws), ws_bytes // 2) != 0  # holds the V^T copy only
    assert prepass(None, ctypes.c_void_p(ws.data_ptr() + 8), ws_bytes - 16) != 0  # not 16-byte aligned
    assert prepass(_lib.ptr(q), _lib.ptr(ws), ws_bytes) != 0  # no room for the queries
    assert "smaller" in _lib.last_error()
