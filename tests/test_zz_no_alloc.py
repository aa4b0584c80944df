"""The allocation-free fp8 per-tensor quantisation (vdnh3_quant_tensor_f8_noalloc) through the C ABI
(GPU): bit-identical codes and scale to vdnh3_quant_tensor_f8 (caller workspace), on two calls in a row
on the same GPU (the library's scratch keeps the first call's partial maxima), the second smaller, and
with no device allocation made by the call."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _reference(lib, x):
    from vdn_h3_amd import _lib

    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scale = torch.empty(1, dtype=torch.float32, device=x.device)
    amax = torch.empty(1, dtype=torch.float32, device=x.device)
    rc = lib.vdnh3_quant_tensor_f8(_lib.ptr(x), x.numel(), _lib.ptr(q), _lib.ptr(scale), _lib.ptr(amax),
                                   _lib.stream_handle(x.device))
    _lib.check(rc, "vdnh3_quant_tensor_f8")
    return q, scale


def test_noalloc_fp8_tensor_quantisation_two_calls(device):
    from vdn_h3_amd import _lib, synth

    lib = _lib.lib()
    # the larger call spans many partials (its largest |x| planted in a late span), the second is smaller
    # and its maximum lies in its first span: a stale partial of the first call would raise its scale
    cases = [("large", (40688, 5120), 70, 40687 * 5120 + 77, 96.0), ("small", (333, 640), 71, 5, 64.0)]
    for name, shape, seed, spot, peak in cases:
        x = synth.randn(shape, seed, device=device, dtype=torch.bfloat16)
        x.view(-1)[spot] = peak
        print(f"case noalloc {name} {shape}", flush=True)
        want_q, want_s = _reference(lib, x)
        q = torch.empty(x.shape, dtype=torch.uint8, device=device)
        scale = torch.empty(1, dtype=torch.float32, device=device)
        torch.cuda.synchronize()
        before = torch.cuda.memory_stats(device).get("allocation.all.allocated", 0)
        rc = lib.vdnh3_quant_tensor_f8_noalloc(_lib.ptr(x), x.numel(), _lib.ptr(q), _lib.ptr(scale),
                                               _lib.stream_handle(device))
        _lib.check(rc, "vdnh3_quant_tensor_f8_noalloc")
        torch.cuda.synchronize()
        assert torch.cuda.memory_stats(device).get("allocation.all.allocated", 0) == before
        assert abs(scale.item() - peak / 448.0) <= 1e-6 * peak / 448.0
        assert torch.equal(scale.cpu(), want_s.cpu())
        assert torch.equal(q.cpu(), want_q.cpu())


def test_noalloc_wrapper_matches_quantize_tensor_fp8(device):
    from vdn_h3_amd import linear, synth

    x = synth.randn((257, 1024), 72, device=device, dtype=torch.bfloat16)
    want_q, want_s = linear.quantize_tensor_fp8(x)
    q = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=device)
    s = torch.empty((1, 1), dtype=torch.float32, device=device)
    linear.quantize_tensor_fp8_into(x, q, s)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.uint8).cpu(), want_q.view(torch.uint8).cpu())
    assert torch.equal(s.cpu(), want_s.cpu())
