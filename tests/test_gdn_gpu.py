"""Parity of the chunked Gated DeltaNet kernels with the float64 oracle (GPU).

Not reference parity: the reference has no token-level delta rule (its branch is per frame).
Bars (``_check``): cosine >= 0.9995 and every output within 4 bf16 ulps of its row's largest value
(8 at the full 40,688-token shape), at most 1% of outputs beyond one such ulp; q, k K^T, W, U~, P
and S^T enter the MFMAs in bf16. The final fp32 state within 1e-2 relative to its largest entry.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn_oracle as go

pytestmark = pytest.mark.gpu


def _inputs(tokens, heads, seed, decay_scale):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(tokens, heads, 128, generator=g).to(torch.bfloat16)
    k = F.normalize(torch.randn(tokens, heads, 128, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(tokens, heads, 128, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(tokens, heads, generator=g))
    lg = -F.softplus(torch.randn(tokens, heads, generator=g)) * decay_scale
    return q, k, v, beta, lg


def _check(got, want, what, row_ulps=4.0):
    """Cosine >= 0.9995, and every output within ``row_ulps`` bf16 ulps of its row's largest float64 value
    (the row: the 128 outputs of one token and head), at most 1% of them beyond one such ulp.

    The GPU forms U~, W, P, Q-hat and S^T in bf16 for its MFMAs, so an output carries an error of a few bf16
    steps of the largest term it sums, whatever its own size: an output near zero in a row of O(1) values
    is many of its own ulps off (that fraction is printed, not bounded)."""
    g32, w = got.float().cpu().double(), want.double()
    diff = (g32 - w).abs()
    cos = F.cosine_similarity(g32.flatten(), w.flatten(), dim=0).item()
    ulp_v = torch.ldexp(torch.ones_like(w), torch.frexp(w)[1] - 8).clamp_min(2.0 ** -133)
    scale = w.abs().amax(-1, keepdim=True)
    ulp_row = torch.ldexp(torch.ones_like(scale), torch.frexp(scale)[1] - 8).clamp_min(2.0 ** -133)
    sv, sr = diff / ulp_v, diff / ulp_row
    print(f"{what}: max abs {diff.max().item():.3e}, cosine {cos:.7f}; ulps of the row's largest value: max "
          f"{sr.max().item():.2f} (bar {row_ulps}), frac > 1 {(sr > 1).double().mean():.2e}; ulps of the value: "
          f"frac > 2 {(sv > 2).double().mean():.2e}, frac > 4 {(sv > 4).double().mean():.2e}", flush=True)
    assert torch.isfinite(g32).all() and cos >= 0.9995, what
    assert sr.max().item() <= row_ulps, what
    assert (sr > 1).double().mean().item() <= 1e-2, what


@pytest.mark.parametrize("tokens,heads,decay,init", [(300, 3, 0.05, True), (64, 2, 0.05, False),
                                                     (1000, 2, 1.0, False), (129, 1, 0.0, True),
                                                     (10, 2, 0.05, True), (65, 1, 0.05, False)])
def test_gdn_matches_recurrence(device, tokens, heads, decay, init):
    from vdn_h3_amd.gdn import chunk_gated_delta_rule

    print(f"case gdn T={tokens} H={heads} decay x{decay} init={init}", flush=True)
    q, k, v, beta, lg = _inputs(tokens, heads, tokens + heads, decay)
    s0 = torch.randn(heads, 128, 128, generator=torch.Generator().manual_seed(7)) * 0.1 if init else None
    want, s_want = go.recurrence(q, k, v, beta, lg, s0)
    fused = torch.cat([q, k, v], dim=-1).to(device)                  # strided q / k / v views
    dq, dk, dv = fused[..., :128], fused[..., 128:256], fused[..., 256:]
    out, s_got = chunk_gated_delta_rule(dq, dk, dv, beta.to(device), lg.to(device),
                                        initial_state=None if s0 is None else s0.to(device), output_final_state=True)
    torch.cuda.synchronize()
    _check(out, want, "gdn output")
    s_err = (s_got.cpu().double() - s_want).abs().max().item()
    assert s_err <= 1e-2 * s_want.abs().max().item(), s_err


def test_gdn_split_at_chunk_boundary_is_bit_identical(device):
    """A sequence run as two calls, the second starting at a chunk boundary from the first call's final
    state, gives the same bits as one call: the restart the library's segmented long-sequence path makes
    (a segment is an independent sequence whose initial state is the state the previous one ended with)."""
    from vdn_h3_amd.gdn import chunk_gated_delta_rule

    tokens, heads, split = 1000, 3, 384  # split at chunk 6 of 16; the tail ends in a partial chunk
    print(f"case gdn split T={tokens} H={heads} at {split}", flush=True)
    q, k, v, beta, lg = _inputs(tokens, heads, 11, 0.05)
    s0 = torch.randn(heads, 128, 128, generator=torch.Generator().manual_seed(8)) * 0.1
    dq, dk, dv, db, dg, ds0 = (t.to(device) for t in (q, k, v, beta, lg, s0))
    whole, s_whole = chunk_gated_delta_rule(dq, dk, dv, db, dg, initial_state=ds0, output_final_state=True)
    head, s_mid = chunk_gated_delta_rule(dq[:split], dk[:split], dv[:split], db[:split], dg[:split],
                                         initial_state=ds0, output_final_state=True)
    tail, s_tail = chunk_gated_delta_rule(dq[split:], dk[split:], dv[split:], db[split:], dg[split:],
                                          initial_state=s_mid, output_final_state=True)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([head, tail]).cpu(), whole.cpu())
    assert torch.equal(s_tail.cpu(), s_whole.cpu())


def test_gdn_pipelined_segments_match_chained_calls(device):
    """A sequence long enough to run in pipelined segments (the prep of segment i + 1 on the host layer's
    side stream beside the scan of segment i, through two workspace buffers, so segment 2 reuses the
    buffer of segment 0) gives the same bits as the same segments run as separate one-segment calls
    chained through their final states."""
    from vdn_h3_amd.gdn import chunk_gated_delta_rule

    tokens, heads = 64 * 70 - 17, 3  # 70 chunks: segments of 32, 32 and 6 chunks, the last one partial
    print(f"case gdn pipelined T={tokens} H={heads}", flush=True)
    q, k, v, beta, lg = _inputs(tokens, heads, 12, 0.05)
    s0 = torch.randn(heads, 128, 128, generator=torch.Generator().manual_seed(9)) * 0.1
    dq, dk, dv, db, dg, ds0 = (t.to(device) for t in (q, k, v, beta, lg, s0))
    whole, s_whole = chunk_gated_delta_rule(dq, dk, dv, db, dg, initial_state=ds0, output_final_state=True)
    parts, state = [], ds0
    for a, b in ((0, 64 * 32), (64 * 32, 64 * 64), (64 * 64, tokens)):
        o, state = chunk_gated_delta_rule(dq[a:b], dk[a:b], dv[a:b], db[a:b], dg[a:b], initial_state=state,
                                          output_final_state=True)
        parts.append(o)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat(parts).cpu(), whole.cpu())
    assert torch.equal(state.cpu(), s_whole.cpu())


def test_gdn_serial_entry_points_match_the_pipelined_call(device):
    """vdnh3_gdn_chunk_fwd (every segment's prep and scan in order on one stream) and the one-stream Python
    path give the bits of the pipelined call (preps on the side stream)."""
    from vdn_h3_amd import _lib
    from vdn_h3_amd.gdn import chunk_gated_delta_rule

    tokens, heads = 64 * 70 - 17, 3
    print(f"case gdn serial vs pipelined T={tokens} H={heads}", flush=True)
    q, k, v, beta, lg = (t.to(device) for t in _inputs(tokens, heads, 14, 0.05))
    s0 = (torch.randn(heads, 128, 128, generator=torch.Generator().manual_seed(10)) * 0.1).to(device)
    lib = _lib.lib()
    assert lib.vdnh3_gdn_segments(tokens, heads, 128) == 3
    piped, s_piped = chunk_gated_delta_rule(q, k, v, beta, lg, initial_state=s0, output_final_state=True)
    one, s_one = chunk_gated_delta_rule(q, k, v, beta, lg, initial_state=s0, output_final_state=True,
                                        pipelined=False)
    out = torch.empty_like(piped)
    s_out = torch.empty_like(s_piped)
    ws_bytes = lib.vdnh3_gdn_workspace_bytes(tokens, heads, 128)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    qb, kb, vb = (t.to(torch.bfloat16).contiguous() for t in (q, k, v))
    bf, gf = beta.float().contiguous(), lg.float().contiguous()
    rc = lib.vdnh3_gdn_chunk_fwd(_lib.ptr(qb), qb.stride(0), qb.stride(1), _lib.ptr(kb), kb.stride(0), kb.stride(1),
                                 _lib.ptr(vb), vb.stride(0), vb.stride(1), _lib.ptr(bf), bf.stride(0), _lib.ptr(gf),
                                 gf.stride(0), _lib.ptr(s0), _lib.ptr(s_out), _lib.ptr(out), out.stride(0),
                                 out.stride(1), tokens, heads, 128, _lib.ptr(ws), ws_bytes, _lib.stream_handle(device))
    _lib.check(rc, "vdnh3_gdn_chunk_fwd")
    torch.cuda.synchronize()
    for got, s_got in ((one, s_one), (out, s_out)):
        assert torch.equal(got, piped) and torch.equal(s_got, s_piped)
    with pytest.raises(ValueError, match="segment 3 of 3"):
        _lib.check(lib.vdnh3_gdn_scan(None, None, _lib.ptr(out), out.stride(0), out.stride(1), tokens, heads, 128,
                                      3, _lib.ptr(ws), ws_bytes, _lib.stream_handle(device)), "vdnh3_gdn_scan")


def test_gdn_pipelined_call_replays_in_a_graph(device):
    """The pipelined call captured in a graph (the side stream joins the capture through the call's fork
    event and is joined back by the last scan's wait) replays to the eager result, three replays with
    eager work and synchronisations between them."""
    from vdn_h3_amd.gdn import chunk_gated_delta_rule

    tokens, heads = 64 * 70, 2
    print(f"case gdn graph T={tokens} H={heads}", flush=True)
    q, k, v, beta, lg = (t.to(device) for t in _inputs(tokens, heads, 13, 0.05))
    eager, s_eager = chunk_gated_delta_rule(q, k, v, beta, lg, output_final_state=True)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, s_out = chunk_gated_delta_rule(q, k, v, beta, lg, output_final_state=True)
    for r in range(3):
        out.zero_()
        s_out.zero_()
        noise = torch.randn(1 << 20, device=device).sum()  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        assert torch.equal(out, eager), f"replay {r}: output"
        assert torch.equal(s_out, s_eager), f"replay {r}: final state"


def test_gdn_first_call_captured_in_a_fresh_process(device):
    """The per-device pipeline stream and events are made by the first pipelined call. Here that call is made
    inside a graph capture, in a fresh process with no eager call before it; three replays (eager work and
    synchronisations between them) give the bits of an eager call made afterwards."""
    import subprocess
    import sys
    import textwrap
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    script = textwrap.dedent(f"""
        import sys
        sys.path[:0] = [{str(root)!r}, {str(root / "comfyui-kirei-vdn-h3_amd")!r}]
        import torch
        import torch.nn.functional as F
        from vdn_h3_amd.gdn import chunk_gated_delta_rule
        dev = torch.device("cuda:0")
        g = torch.Generator().manual_seed(17)
        t, h = 64 * 70, 2
        q = torch.randn(t, h, 128, generator=g).to(torch.bfloat16).to(dev)
        k = F.normalize(torch.randn(t, h, 128, generator=g), dim=-1).to(torch.bfloat16).to(dev)
        v = torch.randn(t, h, 128, generator=g).to(torch.bfloat16).to(dev)
        beta = torch.sigmoid(torch.randn(t, h, generator=g)).to(dev)
        lg = (-F.softplus(torch.randn(t, h, generator=g)) * 0.05).to(dev)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out, s_out = chunk_gated_delta_rule(q, k, v, beta, lg, output_final_state=True)
        got = []
        for r in range(3):
            out.zero_()
            s_out.zero_()
            noise = torch.randn(1 << 20, device=dev).sum()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got.append((out.clone(), s_out.clone()))
        eager, s_eager = chunk_gated_delta_rule(q, k, v, beta, lg, output_final_state=True)
        torch.cuda.synchronize()
        for r, (o, s) in enumerate(got):
            assert torch.equal(o, eager), f"replay {{r}}: output"
            assert torch.equal(s, s_eager), f"replay {{r}}: final state"
        print("first call captured: 3 replays equal the eager call", flush=True)
    """)
    print("case gdn first pipelined call inside a capture (child process)", flush=True)
    proc = subprocess.run([sys.executable, "-u", "-c", script], capture_output=True, text=True, timeout=300)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    assert "3 replays equal the eager call" in proc.stdout


def test_gdn_full_shape_sampled_heads(device):
    """40,688 tokens x 40 heads (the chunk-64 benchmark shape); heads 0 and 39 against the oracle."""
    from vdn_h3_amd.gdn import chunk_gated_delta_rule

    print("case gdn full shape", flush=True)
    tokens, heads = 40688, 40
    g = torch.Generator(device=device).manual_seed(11)
    q = torch.randn(tokens, heads, 128, generator=g, device=device).to(torch.bfloat16)
    k = F.normalize(torch.randn(tokens, heads, 128, generator=g, device=device), dim=-1).to(torch.bfloat16)
    v = torch.randn(tokens, heads, 128, generator=g, device=device).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(tokens, heads, generator=g, device=device))
    lg = -F.softplus(torch.randn(tokens, heads, generator=g, device=device))
    out, _ = chunk_gated_delta_rule(q, k, v, beta, lg)
    torch.cuda.synchronize()
    sel = [0, 39]
    want, _ = go.chunked(q[:, sel].cpu(), k[:, sel].cpu(), v[:, sel].cpu(), beta[:, sel].cpu(), lg[:, sel].cpu())
    # 636 chunk steps, each through a bf16 S^T: the largest row error seen is 6.2 row-max ulps
    _check(out[:, sel], want, "gdn full shape heads 0, 39", row_ulps=8.0)


@pytest.mark.parametrize("dim", [48, 96])
def test_gdn_head_dims_below_128(device, dim):
    """Head dims below 128 run at 128 with zero channels added (exact: the state's added rows and columns stay
    zero), against the float64 recurrence at the true head dim, with an initial and a final state."""
    from vdn_h3_amd.gdn import chunk_gated_delta_rule

    tokens, heads = 300, 2
    print(f"case gdn head_dim={dim}", flush=True)
    g = torch.Generator().manual_seed(dim)
    q = torch.randn(tokens, heads, dim, generator=g).to(torch.bfloat16)
    k = F.normalize(torch.randn(tokens, heads, dim, generator=g), dim=-1).to(torch.bfloat16)
    v = torch.randn(tokens, heads, dim, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(tokens, heads, generator=g))
    lg = -F.softplus(torch.randn(tokens, heads, generator=g)) * 0.05
    s0 = torch.randn(heads, dim, dim, generator=g) * 0.1
    want, s_want = go.recurrence(q, k, v, beta, lg, s0)
    out, s_got = chunk_gated_delta_rule(q.to(device), k.to(device), v.to(device), beta.to(device), lg.to(device),
                                        initial_state=s0.to(device), output_final_state=True)
    torch.cuda.synchronize()
    assert out.shape == (tokens, heads, dim) and s_got.shape == (heads, dim, dim)
    _check(out, want, f"gdn output d={dim}")
    s_err = (s_got.cpu().double() - s_want).abs().max().item()
    assert s_err <= 1e-2 * s_want.abs().max().item(), s_err
    with pytest.raises(ValueError, match="head_dim must be 1 to 128"):
        big = torch.zeros(64, 1, 160, dtype=torch.bfloat16, device=device)
        chunk_gated_delta_rule(big, big, big, torch.zeros(64, 1, device=device), torch.zeros(64, 1, device=device))


def test_gdn_empty_sequence(device):
    """No token: an empty output and the initial state as the final state (zeros without one)."""
    from vdn_h3_amd.gdn import chunk_gated_delta_rule

    print("case gdn empty sequence", flush=True)
    for dim in (128, 48):
        x = torch.zeros(0, 2, dim, dtype=torch.bfloat16, device=device)
        z = torch.zeros(0, 2, device=device)
        s0 = torch.randn(2, dim, dim, generator=torch.Generator().manual_seed(3)).to(device)
        out, s = chunk_gated_delta_rule(x, x, x, z, z, initial_state=s0, output_final_state=True)
        assert out.shape == (0, 2, dim) and torch.equal(s, s0) and s.data_ptr() != s0.data_ptr()
        out, s = chunk_gated_delta_rule(x, x, x, z, z, output_final_state=True)
        assert out.shape == (0, 2, dim) and s.shape == (2, dim, dim) and not s.any()
