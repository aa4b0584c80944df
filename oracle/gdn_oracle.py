"""Oracle: token-level chunked Gated DeltaNet (the chunk-64 gated delta rule), CPU, float64.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

This path is NOT in hyukudan/ComfyUI-Kirei-VDN-H3: the reference's Video Delta Attention solves
its delta rule per frame (``vdn_h3/branch.py:148-160``). The token-level chunked form is the
published Gated DeltaNet recurrence (Yang, Kautz, Hatamizadeh, "Gated Delta Networks", 2024)
that the benchmark's chunk-64 workload names. Per head, with the state S (dv x dk):

    S_t = a_t S_{t-1} (I - b_t k_t k_t^T) + b_t v_t k_t^T,   o_t = S_t q_t,   a_t = exp(g_t)

``recurrence`` runs it token by token. ``chunked`` is the chunk form (chunk C): with the
in-chunk cumulative log-decay G_t = sum_{i<=t} g_i,

    A[t][j] = b_t exp(G_t - G_j) k_t.k_j  (j < t),       T = (I + A)^-1     (unit lower triangular)
    W = T diag(b exp(G)) K,   U~ = T diag(b) V,          U = U~ - W S0^T
    O = diag(exp(G)) Q S0^T + (Q K^T o D) U,             D[t][j] = exp(G_t - G_j) (j <= t)
    S_C = exp(G_C) S0 + U^T diag(exp(G_C - G)) K

Pinning (``tests/test_oracle_gdn.py``): ``chunked`` equals ``recurrence`` to float64 rounding
for chunk sizes 1, 16, 64 and ragged ends; b = 0 keeps the state a pure decay; a = 1, b = 1 with
one key makes S a projection-free write; the recurrence itself against a direct unrolled sum for
a scalar (dk = dv = 1) case.
"""

from __future__ import annotations

import torch


def recurrence(q, k, v, beta, g, initial=None):
    """Token-by-token gated delta rule. q, k: [T, H, dk]; v: [T, H, dv]; beta, g: [T, H].

    Returns (o [T, H, dv], final state [H, dv, dk]) in float64.
    """
    q, k, v, beta, g = (t.double() for t in (q, k, v, beta, g))
    steps, heads, dk = k.shape
    dv = v.shape[-1]
    s = torch.zeros(heads, dv, dk, dtype=torch.float64) if initial is None else initial.double().clone()
    out = torch.empty(steps, heads, dv, dtype=torch.float64)
    for t in range(steps):
        a = torch.exp(g[t]).view(heads, 1, 1)
        kt, vt, bt = k[t], v[t], beta[t].view(heads, 1, 1)
        sk = torch.einsum("hvk,hk->hv", s, kt)                       # S k
        s = a * s - a * bt * torch.einsum("hv,hk->hvk", sk, kt) + bt * torch.einsum("hv,hk->hvk", vt, kt)
        out[t] = torch.einsum("hvk,hk->hv", s, q[t])
    return out, s


def chunked(q, k, v, beta, g, chunk=64, initial=None):
    """The chunk form (WY representation with a per-chunk unit-triangular inverse), float64."""
    q, k, v, beta, g = (t.double() for t in (q, k, v, beta, g))
    steps, heads, dk = k.shape
    dv = v.shape[-1]
    s = torch.zeros(heads, dv, dk, dtype=torch.float64) if initial is None else initial.double().clone()
    out = torch.empty(steps, heads, dv, dtype=torch.float64)
    for c0 in range(0, steps, chunk):
        c1 = min(c0 + chunk, steps)
        n = c1 - c0
        kc, qc, vc = k[c0:c1].transpose(0, 1), q[c0:c1].transpose(0, 1), v[c0:c1].transpose(0, 1)  # [H, n, d]
        bc = beta[c0:c1].transpose(0, 1)                                                           # [H, n]
        gam = torch.cumsum(g[c0:c1].transpose(0, 1), dim=1)                                       # [H, n]
        diff = gam.unsqueeze(2) - gam.unsqueeze(1)                                                 # G_t - G_j
        lower = torch.tril(torch.ones(n, n, dtype=torch.bool), diagonal=-1)
        kk = kc @ kc.transpose(1, 2)
        a_mat = torch.where(lower, bc.unsqueeze(2) * torch.exp(diff) * kk, torch.zeros(()))
        eye = torch.eye(n, dtype=torch.float64).expand(heads, n, n)
        t_mat = torch.linalg.solve_triangular(eye + a_mat, eye, upper=False, unitriangular=True)
        w = t_mat @ ((bc * torch.exp(gam)).unsqueeze(2) * kc)
        u = t_mat @ (bc.unsqueeze(2) * vc) - w @ s.transpose(1, 2)
        incl = torch.tril(torch.ones(n, n, dtype=torch.bool))
        p = torch.where(incl, (qc @ kc.transpose(1, 2)) * torch.exp(diff), torch.zeros(()))
        o = torch.exp(gam).unsqueeze(2) * (qc @ s.transpose(1, 2)) + p @ u
        out[c0:c1] = o.transpose(0, 1)
        last = gam[:, -1:]
        s = torch.exp(last).unsqueeze(2) * s + u.transpose(1, 2) @ (torch.exp(last - gam).unsqueeze(2) * kc)
    return out, s
