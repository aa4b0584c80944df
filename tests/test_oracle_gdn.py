"""Pins of the chunked Gated DeltaNet oracle (CPU, float64)."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import gdn_oracle as go


def _inputs(steps, heads, dk, dv, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(steps, heads, dk, generator=g)
    k = F.normalize(torch.randn(steps, heads, dk, generator=g), dim=-1)
    v = torch.randn(steps, heads, dv, generator=g)
    beta = torch.sigmoid(torch.randn(steps, heads, generator=g))
    lg = -F.softplus(torch.randn(steps, heads, generator=g)) * 0.2      # mild decay: the carry matters
    return q, k, v, beta, lg


@pytest.mark.parametrize("chunk,steps", [(1, 23), (16, 70), (64, 150), (64, 64)])
def test_chunked_equals_recurrence(chunk, steps):
    q, k, v, beta, lg = _inputs(steps, 2, 16, 12, chunk + steps)
    init = torch.randn(2, 12, 16, generator=torch.Generator().manual_seed(9))
    o1, s1 = go.recurrence(q, k, v, beta, lg, init)
    o2, s2 = go.chunked(q, k, v, beta, lg, chunk, init)
    torch.testing.assert_close(o2, o1, atol=1e-9, rtol=1e-9)
    torch.testing.assert_close(s2, s1, atol=1e-9, rtol=1e-9)


def test_special_cases():
    q, k, v, beta, lg = _inputs(40, 1, 8, 8, 3)
    init = torch.randn(1, 8, 8, generator=torch.Generator().manual_seed(4))
    # beta = 0: no write, the state only decays by exp(sum g)
    _, s = go.recurrence(q, k, v, torch.zeros_like(beta), lg, init)
    torch.testing.assert_close(s, init.double() * torch.exp(lg.double().sum()), atol=1e-12, rtol=1e-12)
    # a = 1, b = 1 and one repeated unit key: S_t k = v_t (the delta rule overwrites the key's value)
    kk = F.normalize(k[:1].double(), dim=-1).expand(k.shape)             # unit to float64 rounding
    _, s = go.recurrence(q, kk, v, torch.ones_like(beta), torch.zeros_like(lg))
    torch.testing.assert_close(s[0] @ kk[0, 0], v[-1, 0].double(), atol=1e-12, rtol=1e-12)
    # dk = dv = 1: S_t = a_t (1 - b_t k_t^2) S_{t-1} + b_t v_t k_t unrolled by hand
    q1, k1, v1, b1, g1 = (t[:6, :1, :1] if t.ndim == 3 else t[:6, :1] for t in (q, k, v, beta, lg))
    k1 = torch.sign(k1) + (k1 == 0).float()                           # unit keys in one dimension: +-1
    s_ref, outs = 0.0, []
    for t in range(6):
        a, b, kv, vv = math.exp(float(g1[t, 0])), float(b1[t, 0]), float(k1[t, 0, 0]), float(v1[t, 0, 0])
        s_ref = a * (1 - b * kv * kv) * s_ref + b * vv * kv
        outs.append(s_ref * float(q1[t, 0, 0]))
    o, _ = go.recurrence(q1, k1, v1, b1, g1)
    torch.testing.assert_close(o.flatten(), torch.tensor(outs, dtype=torch.float64), atol=1e-12, rtol=1e-12)
