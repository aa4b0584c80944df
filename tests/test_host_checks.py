"""Host-side behaviour of the product API that needs no GPU: loud failures, no CPU fallback."""

from __future__ import annotations

import pytest
import torch


def test_window_op_rejects_cpu_tensors(built_lib):
    from vdn_h3_amd import window

    q = torch.zeros(8, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        window.window_softmax_hip(q, q, q, 0, 8, 1, 8, [(0, 0)], 0.125)


def test_ops_are_forward_only_in_gradient_mode(built_lib):
    """An input that requires grad in gradient mode is an error before any device work (the HIP ops have no
    backward, so their result would silently carry no gradient); under no_grad the same call reaches the
    device check."""
    from vdn_h3_amd import gdn, linear, softmax_kernels, window
    from vdn_h3_amd.hybrid import normalise_qk

    q = torch.zeros(8, 1, 64, dtype=torch.bfloat16, requires_grad=True)
    w = torch.ones(64, dtype=torch.bfloat16)
    beta = torch.zeros(8, 1)
    calls = {
        "window_softmax_hip": lambda: window.window_softmax_hip(q, q, q, 0, 8, 1, 8, [(0, 0)], 0.125),
        "window_softmax_normed": lambda: window.window_softmax_normed(q, q, q, w, w, 1e-6, 1e-6, 0, 8, 1, 8,
                                                                      [(0, 0)], 0.125),
        "normalise_qk": lambda: normalise_qk(q, q, w, w),
        "apply_softmax_gate": lambda: softmax_kernels.apply_softmax_gate(q, beta),
        "gemm": lambda: linear.linear(q[:, 0], torch.zeros(16, 64, dtype=torch.bfloat16)),
        "chunk_gated_delta_rule": lambda: gdn.chunk_gated_delta_rule(q, q, q, beta, beta),
    }
    for what, call in calls.items():
        with pytest.raises(RuntimeError, match=f"{what} is forward-only"):
            call()
        with torch.no_grad(), pytest.raises(RuntimeError, match="no CPU fallback"):
            call()
    weight = torch.zeros(16, 64, requires_grad=True)
    with pytest.raises(RuntimeError, match="no CPU fallback"):  # the weight is a constant, not a grad input
        linear.HipLinear(weight)


def test_window_op_shape_errors(built_lib):
    from vdn_h3_amd import window

    q = torch.zeros(8, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="share shape"):
        window.window_softmax_hip(q, q[:4], q, 0, 8, 1, 8, [(0, 0)], 0.125)


def test_missing_library_is_a_hard_error(monkeypatch, tmp_path):
    from vdn_h3_amd import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libvdnh3.so")
    with pytest.raises(_lib.LibraryMissingError):
        _lib.lib()


def test_backend_resolution_is_hip():
    from vdn_h3_amd import window

    cache = window.WindowAttentionCache()
    for name in window.ATTENTION_BACKENDS:
        assert window.resolve_attention_backend(name, cache=cache) == "hip"
    with pytest.raises(ValueError):
        window.resolve_attention_backend("sage")


def test_layout_mirror_matches_reference_semantics():
    from types import SimpleNamespace

    from vdn_h3_amd.layout import current_layout, from_comfy_packed_layout, publish_layout

    # tests/test_layout.py:13-30 packed layout: 3 text rows, 2 audio rows, 2 frames of 2x2
    packed = SimpleNamespace(signature=(3, 2, 4, 4, 1), segments=((0, 3, "text"), (3, 5, "audio"), (5, 13, "video")),
                             seq_len=13)
    lay = from_comfy_packed_layout(packed, radius=1, chunk=5, anchor_frames="both")
    assert (lay.video_start, lay.video_end, lay.frame_size, lay.tokens_per_frame) == (5, 13, (2, 2), 4)
    assert lay.full_cover is True
    assert current_layout(required=False) is None
    with publish_layout(lay):
        assert current_layout() is lay
    with pytest.raises(RuntimeError):
        current_layout()


def test_c_abi_rejects_bad_arguments_before_any_launch(built_lib):
    """The C ABI validates on the host and returns VDNH3_ERR_INVALID (1) without touching a device:
    a negative or out-of-range activation code, and a Gated DeltaNet head size other than 128."""
    import ctypes

    buf = (ctypes.c_uint8 * 4096)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    gemm = lambda act: built_lib.vdnh3_gemm(0, p, 64, p, 64, p, 64, 4, 4, 64, None, 0, None, 0, 1.0, None, 0, act,  # noqa: E731
                                            0, 0, 1, None)
    assert gemm(-1) == 1 and b"activation" in built_lib.vdnh3_last_error()
    assert gemm(2 * 5 + 1) == 1                          # sigmoid on 5 leading columns of a 4-column output
    rc = built_lib.vdnh3_gdn_chunk_fwd(p, 64, 64, p, 64, 64, p, 64, 64, p, 1, p, 1, None, None, p, 64, 64, 8, 1, 64, p,
                                       4096, None)
    assert rc == 1 and b"head_dim" in built_lib.vdnh3_last_error()


def test_row_span_joins_row_slices_of_one_matrix():
    """The branch computes the text rows' beta in the video rows' GEMM only when both are row slices of
    one row-major matrix, text first, with at most a quarter of extra rows between them."""
    from vdn_h3_amd.runtime import _row_span

    x = torch.arange(100 * 8, dtype=torch.float32).view(100, 8)
    view, gap = _row_span(x[:10], x[20:90])
    assert gap == 20 and torch.equal(view, x[:90])
    assert _row_span(x[20:30], x[:10]) is None        # text after the video rows
    assert _row_span(x[:5], x[50:60]) is None         # too many rows in between
    assert _row_span(x[:10], x[5:20]) is None         # overlapping
    view, gap = _row_span(x[:10, :4], x[20:90, :4])   # column slices keep the row stride
    assert gap == 20 and torch.equal(view, x[:90, :4])
    assert _row_span(x[:10].clone(), x[20:90]) is None  # different storage
    assert _row_span(None, x[20:90]) is None


def test_segment_index_is_built_without_device_reads_and_range_checked():
    """BlockPointwiseCache turns a segment map into the per-token index (same values as the oracle's
    brute-force map), knows its range on the host for integer and CPU-tensor rows, and the pointwise
    ops reject an index outside the modulation table before any launch (ValueError, as index_select)."""
    from oracle import dit_oracle as do
    from vdn_h3_amd import block_kernels as bk

    segs = [(0, 5, 2), (5, 9, torch.tensor([0, 1, 1, 0])), (9, 12, torch.tensor(1)), (12, 12, 7)]
    idx = bk.build_segment_index(segs, 12, torch.device("cpu"))
    assert idx.ids.dtype == torch.int32 and idx.ids.tolist() == do.segment_indices(segs[:3], 12).tolist()
    assert (idx.low, idx.high) == (0, 2)
    cache = bk.BlockPointwiseCache(limit=2)
    ints = [(0, 7, 1), (7, 12, 0)]
    first = cache.index(ints, 12, "cpu")
    assert first is cache.index(ints, 12, "cpu") and (first.low, first.high) == (0, 1)
    assert cache.indices(ints, 12, "cpu").tolist() == [1] * 7 + [0] * 5
    with pytest.raises(ValueError):
        bk.build_segment_index([(0, 5, 0), (6, 12, 1)], 12, "cpu")        # a gap
    with pytest.raises(ValueError):
        bk.build_segment_index([(0, 5, 0)], 12, "cpu")                    # short of the sequence
    with pytest.raises(ValueError):
        bk.build_segment_index([(0, 12, torch.tensor([0, 1]))], 12, "cpu")  # wrong row count
    x = torch.zeros(12, 16, dtype=torch.bfloat16)
    table = torch.zeros(2, 16)
    bad = bk.build_segment_index([(0, 6, 0), (6, 12, 2)], 12, "cpu")     # row 2 of a 2-row table
    with pytest.raises(ValueError, match="out of range"):
        bk.rmsnorm_modulate(x, torch.ones(16), 1e-6, table, table, bad)
    with pytest.raises(ValueError, match="out of range"):
        bk.gated_residual(x, table, torch.tensor([0] * 11 + [-1]), x)


def test_noalloc_fp8_quantisation_rejects_oversize_tensors_on_the_host(built_lib):
    """vdnh3_quant_tensor_f8_noalloc's scratch holds 16,384 partial maxima of 16,384 elements: a larger
    tensor is rejected with VDNH3_ERR_INVALID before any device access (as are null and unaligned operands)."""
    import ctypes

    limit = built_lib.vdnh3_quant_tensor_f8_noalloc_max_elements()
    assert limit == 16384 * 16384
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.c_void_p((ctypes.addressof(buf) + 15) // 16 * 16)
    assert built_lib.vdnh3_quant_tensor_f8_noalloc(p, limit + 8, p, p, None) == 1
    assert b"exceed" in built_lib.vdnh3_last_error()
    assert built_lib.vdnh3_quant_tensor_f8_noalloc(None, 8, p, p, None) == 1
    assert built_lib.vdnh3_quant_tensor_f8_noalloc(p, 12, p, p, None) == 1


def test_tile_frames_option_checks():
    from vdn_h3_amd.hybrid import VDNState
    from vdn_h3_amd.runtime import OptimizedLinearBranch

    br = OptimizedLinearBranch({}, 2, 64)
    assert br.tile_frames == 0
    br.set_runtime(tile_frames=5, kernel_backend="ignored")
    assert br.tile_frames == 5
    for bad in (-1, True):
        with pytest.raises(ValueError, match="tile_frames"):
            br.set_runtime(tile_frames=bad)
    with pytest.raises(ValueError, match="tile_frames"):
        VDNState("t", {}, [br], 2, 64, tile_frames=-2)
    VDNState("t", {}, [br], 2, 64, tile_frames=3)
    assert br.tile_frames == 3


def test_readout_frame_range_checks():
    from vdn_h3_amd import branch

    frames, tokens, heads, dim = 4, 8, 1, 64
    q = torch.zeros(2 * tokens, heads, dim, dtype=torch.bfloat16)
    banks = torch.zeros(frames, heads, dim, dim)
    alpha = torch.ones(frames, heads, dim)
    kw = dict(num_frames=frames, tokens_per_frame=tokens, gate_hidden=torch.zeros(2 * tokens, dim),
              gate_up_weight=torch.zeros(heads * dim, dim))
    bounds = [(0, 1), (0, 2), (1, 3), (2, 3)]
    for bad in ((3, 5), (2, 2), (-1, 1)):
        with pytest.raises(ValueError, match="frame_range"):
            branch.readout_epilogue(q, banks, banks, alpha, bounds, torch.ones(dim), None, frame_range=bad, **kw)
    with pytest.raises(ValueError, match="range's frames"):
        branch.readout_epilogue(q, banks, banks, alpha, bounds, torch.ones(dim), None, frame_range=(0, 3), **kw)
