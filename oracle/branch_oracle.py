"""Oracle: the VDN (Video Delta Attention) linear branch on the CPU.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Restates the inference spelling of the branch of hyukudan/ComfyUI-Kirei-VDN-H3 v0.3.3
with the reference's dtype casts (bf16 model: features, gates and readout in bf16;
statistics, factor, scans and gather in fp32):

* ``activate``           -> ``vdn_h3/kernels.py:47-51``
* ``temporal_shift``     -> ``vdn_h3/kernels.py:59-68``
* ``conv_features``      -> ``vdn_h3/runtime.py:319-341`` / ``vdn_h3/branch.py:443-480`` (eager
  bf16 temporal sum, the reference's CPU spelling)
* ``conv_features_fused``-> the same with the fused temporal kernel of ``vdn_h3/kernels.py:100-129``
  (fp32 temporal sum, SiLU and norm; the reference's CUDA spelling)
* ``frame_statistics``   -> ``vdn_h3/branch.py:197-243``
* ``vdn_factor``         -> ``vdn_h3/branch.py:62-71``, ``:148-160`` (``VdnDelta.factor_apply``)
* ``sana_factor``        -> ``vdn_h3/branch.py:163-177``
* ``run_scans``          -> ``vdn_h3/branch.py:285-333``, ``vdn_h3/runtime.py:118-131``
* ``gather_linear_state``-> ``vdn_h3/branch.py:345-396``
* ``alpha_gate``         -> ``vdn_h3/branch.py:483-491``
* ``rms_norm`` / ``linear_epilogue`` -> ``vdn_h3/branch.py:494-505``
* ``text_state``         -> ``vdn_h3/branch.py:649-670``
* ``readout``            -> ``vdn_h3/runtime.py:361-419``
* ``projected_delta``    -> ``vdn_h3/runtime.py:545-607``

"bf16 matmul" below means: the product of the bf16 operands accumulated in fp32 and
rounded once to bf16, which is what a bf16 ``torch.matmul`` returns on the reference's
CUDA path.

Pinning (``tests/test_oracle_branch.py``):

* ``vdn_factor``: ``torch.linalg.inv(I + A)`` closed form (``tests/test_branch.py:11-23``),
  and the leading-minor index for a planted non-SPD matrix (``tests/test_cholesky.py:57-69``).
* ``frame_statistics``: ``einsum`` formulation (``tests/test_branch.py:26-36``), symmetry.
* ``run_scans``: naive ``state @ Phi + J`` loop (``tests/test_branch.py:51-76``).
* ``gather_linear_state``: the per-frame naive gather of ``tests/test_branch.py:79-97``.
* ``alpha_gate`` / ``rms_norm`` / ``activate``: closed forms (``exp(-e^A softplus)``,
  ``x / sqrt(mean x^2 + eps)``, ``silu`` then unit norm).
* ``conv_features``: unit norm and ``F.conv3d`` with a (1,kh,kw) then (kt,1,1) kernel.
* ``conv_features_fused``: ``F.conv3d`` in float64 with the bf16 rounding of the spatial output,
  then SiLU / unit norm in float64 (within one bf16 step), and the branch golden with short
  convolutions (``tests/golden/branch_13f_conv.safetensors``) end to end.
* ``readout`` / ``projected_delta`` composites: golden vectors written by
  ``tests/golden/make_golden.py`` from the reference implementation itself
  (``tests/golden/branch_*.safetensors``).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

TEXT_STATE_SCALE = 0.5  # vdn_h3/branch.py:23


def bf16_matmul(a, b):
    """Product of bf16 operands accumulated in fp32, rounded once to bf16."""
    return torch.matmul(a.float(), b.float()).to(torch.bfloat16)


def activate(tokens, l2norm):
    """SiLU then optional unit L2 norm over the last dim, eps 1e-6 (``vdn_h3/kernels.py:47-51``)."""
    out = F.silu(tokens)
    if l2norm:
        return F.normalize(out, dim=-1, eps=1e-6).to(out.dtype)
    return out


def to_fhsd(rows, num_frames, heads, head_dim):
    """``[F*T, H, D]`` -> ``[F, H, T, D]`` (``vdn_h3/kernels.py:89-94``)."""
    per_frame = rows.shape[0] // num_frames
    return rows.reshape(num_frames, per_frame, heads, head_dim).permute(0, 2, 1, 3).contiguous()


def temporal_shift(x, w, kernel):
    """Depthwise temporal conv over frames, zero padded (``vdn_h3/kernels.py:59-68``).

    ``x``: ``[F, T, C]``, ``w``: ``[C, kernel]``.
    """
    pad = kernel // 2
    xp = F.pad(x, (0, 0, 0, 0, pad, pad))
    out = None
    for dt in range(kernel):
        part = xp[dt:dt + x.shape[0]] * w[:, dt].view(1, 1, -1)
        out = part if out is None else out + part
    return out


def conv_features(tokens, spatial_weight, temporal_weight, num_frames, frame_size, l2norm):
    """Depthwise spatial conv per frame, temporal conv, activation (``vdn_h3/runtime.py:319-341``)."""
    heads, head_dim = tokens.shape[-2:]
    gh, gw = frame_size
    channels = heads * head_dim
    kh, kw = spatial_weight.shape[-2:]
    volume = tokens.reshape(num_frames, gh, gw, channels).permute(0, 3, 1, 2)
    volume = F.conv2d(volume, spatial_weight.to(volume.dtype), padding=(kh // 2, kw // 2), groups=channels)
    flat = volume.permute(0, 2, 3, 1).reshape(num_frames, gh * gw, channels)
    temporal = temporal_weight.squeeze(1).to(flat.dtype)
    raw = temporal_shift(flat, temporal, temporal.shape[-1])
    return activate(raw.reshape(-1, heads, head_dim), l2norm)


def temporal_conv_act_fused(flat, weight, heads, head_dim, l2norm):
    """The reference's fused temporal kernel (``vdn_h3/kernels.py:100-129``) on ``[F, T, C]`` bf16.

    ``acc = sum_dt x[f + dt - kt//2] * w[:, dt]`` in fp32 (zero padded over frames), then
    ``y = acc * sigmoid(acc)``, with ``l2norm`` ``y * 1/sqrt(max(sum_head y^2, 1e-12))``, one
    rounding to bf16 at the end.
    """
    frames, tokens, channels = flat.shape
    kt = weight.shape[-1]
    pad = kt // 2
    xp = F.pad(flat.float(), (0, 0, 0, 0, pad, pad))
    w = weight.reshape(channels, kt).to(flat.dtype).float()
    acc = torch.zeros((frames, tokens, channels), dtype=torch.float32)
    for dt in range(kt):
        acc = acc + xp[dt:dt + frames] * w[:, dt]
    y = acc * torch.sigmoid(acc)
    y = y.reshape(frames, tokens, heads, head_dim)
    if l2norm:
        y = y * (1.0 / torch.sqrt(torch.clamp((y * y).sum(-1, keepdim=True), min=1e-12)))
    return y.to(flat.dtype).reshape(frames * tokens, heads, head_dim)


def conv_features_fused(tokens, spatial_weight, temporal_weight, num_frames, frame_size, l2norm):
    """Short-convolution features as the reference's CUDA path computes them.

    ``vdn_h3/runtime.py:319-341``: the depthwise ``Conv2d`` output is a bf16 tensor (fp32
    accumulation, one rounding), then the fused temporal kernel (``temporal_conv_act_fused``).
    Returns ``[F*T, H, D]`` bf16.
    """
    heads, head_dim = tokens.shape[-2:]
    gh, gw = frame_size
    channels = heads * head_dim
    kh, kw = spatial_weight.shape[-2:]
    volume = tokens.reshape(num_frames, gh, gw, channels).permute(0, 3, 1, 2).float()
    sp = spatial_weight.to(tokens.dtype).float()
    volume = F.conv2d(volume, sp, padding=(kh // 2, kw // 2), groups=channels).to(tokens.dtype)
    flat = volume.permute(0, 2, 3, 1).reshape(num_frames, gh * gw, channels)
    return temporal_conv_act_fused(flat, temporal_weight, heads, head_dim, l2norm)


def frame_statistics(key_by_frame, value_by_frame, beta, a_fp32=True):
    """``A = K^T diag(beta) K`` (fp32, symmetrised) and ``B = (V*beta)^T K`` (``vdn_h3/branch.py:197-243``).

    ``key_by_frame``/``value_by_frame``: ``[F, H, T, D]`` (bf16), ``beta``: ``[F, H, T]``.
    Returns fp32 ``A, B`` of shape ``[F, H, D, D]``; ``B`` carries the bf16 rounding of the
    reference's bf16 matmul.
    """
    key16 = key_by_frame
    key32 = key16.float()
    weighted_key32 = key32 * beta.float().unsqueeze(-1)
    weighted_value = value_by_frame * beta.to(value_by_frame.dtype).unsqueeze(-1)
    if a_fp32:
        matrix_a = weighted_key32.transpose(-1, -2) @ key32
    else:
        weighted_key = key16 * beta.to(key16.dtype).unsqueeze(-1)
        matrix_a = bf16_matmul(weighted_key.transpose(-1, -2), key16).float()
    matrix_a = 0.5 * (matrix_a + matrix_a.transpose(-1, -2))
    if weighted_value.dtype == torch.bfloat16:
        matrix_b = bf16_matmul(weighted_value.transpose(-1, -2), key16).float()
    else:
        matrix_b = (weighted_value.transpose(-1, -2) @ key16).float()
    return matrix_a, matrix_b


def vdn_factor(alpha, a_raw, b_raw):
    """``L = chol(I + A)``, ``M = L^-T L^-1``, ``Phi = alpha[..., None] * M``, ``J = B M``.

    Follows ``vdn_h3/branch.py:148-160`` with the status of ``torch.linalg.cholesky_ex``
    (``vdn_h3/branch.py:68``): ``info`` is 0, or the order of the first non-positive
    leading minor. Returns ``(Phi, J, info)``.
    """
    a32, b32 = a_raw.float(), b_raw.float()
    eye = torch.eye(a32.shape[-1], dtype=torch.float32).expand_as(a32)
    chol, info = torch.linalg.cholesky_ex(a32 + eye, check_errors=False)
    inv_chol = torch.linalg.solve_triangular(chol, eye, upper=False, left=True)
    inverse = inv_chol.transpose(-1, -2) @ inv_chol
    return alpha.float().unsqueeze(-1) * inverse, b32 @ inverse, info


def sana_factor(alpha, a_raw, b_raw, tokens_per_frame):
    """``Phi = alpha * (I - A/T)``, ``J = B / sqrt(T)`` (``vdn_h3/branch.py:163-177``)."""
    inv_t = 1.0 / tokens_per_frame
    eye = torch.eye(a_raw.shape[-1], dtype=a_raw.dtype)
    return alpha.unsqueeze(-1) * (eye - inv_t * a_raw), (inv_t ** 0.5) * b_raw


def run_scans(transitions, injections, initial):
    """Bidirectional affine scans ``P_f = J_f + P_{f-1} Phi_f`` (``vdn_h3/runtime.py:118-131``)."""
    frames = transitions.shape[0]
    prefix = torch.empty((frames, *initial.shape), dtype=torch.float32)
    suffix = torch.empty_like(prefix)
    state = initial.float()
    for f in range(frames):
        state = torch.baddbmm(injections[f], state, transitions[f])
        prefix[f] = state
    state = initial.float()
    for f in range(frames - 1, -1, -1):
        state = torch.baddbmm(injections[f], state, transitions[f])
        suffix[f] = state
    return prefix, suffix


def gather_indices(bounds, num_frames):
    """Index tables of ``vdn_h3/branch.py:345-369``."""
    last_before = torch.tensor([lo for lo, _ in bounds], dtype=torch.long) - 1
    first_after = torch.tensor([hi for _, hi in bounds], dtype=torch.long) + 1
    return {
        "before_idx": last_before.clamp(0, num_frames - 1),
        "after_idx": first_after.clamp(0, num_frames - 1),
        "has_before": last_before >= 0,
        "has_after": first_after < num_frames,
        "bridge_before": (last_before + 1).clamp(0, num_frames),
        "bridge_after": first_after.clamp(0, num_frames),
        "frames": torch.arange(num_frames, dtype=torch.long),
    }


def gather_linear_state(prefix, suffix, alpha, bounds, bridge="alpha", text_state=None, out_dtype=None):
    """Complementary-window state per frame (``vdn_h3/branch.py:372-396``)."""
    frames = prefix.shape[0]
    idx = gather_indices(bounds, frames)
    before = prefix[idx["before_idx"]]
    after = suffix[idx["after_idx"]]
    shape = (frames, 1, 1, 1)
    if text_state is not None:
        text = text_state.to(before.dtype)
        before = torch.where(idx["has_before"].view(shape), before, text)
        after = torch.where(idx["has_after"].view(shape), after, text)
    if bridge == "alpha":
        log_alpha = alpha.clamp_min(1e-12).log()
        log_prefix = torch.cat((torch.zeros_like(log_alpha[:1]), log_alpha.cumsum(0)))
        decay_before = torch.exp(log_prefix[idx["frames"] + 1] - log_prefix[idx["bridge_before"]])
        decay_after = torch.exp(log_prefix[idx["bridge_after"]] - log_prefix[idx["frames"]])
        before = before * decay_before.unsqueeze(2)
        after = after * decay_after.unsqueeze(2)
    if text_state is None:
        result = before * idx["has_before"].view(shape) + after * idx["has_after"].view(shape)
    else:
        result = before + after
    return result if out_dtype is None else result.to(out_dtype)


def alpha_gate(frame_mean, weight_down, weight_up, dt_bias, a_log, num_heads, head_dim):
    """Per-frame key-channel decay ``exp(-e^{A_log} softplus(W_up W_down m + dt))`` (``branch.py:483-491``)."""
    delta = F.linear(frame_mean.float(), weight_down.float())
    delta = F.linear(delta, weight_up.float()) + dt_bias.float()
    decay_scale = torch.exp(a_log.float()).reshape(num_heads, 1)
    delta = delta.reshape(-1, num_heads, head_dim)
    return torch.exp(-decay_scale * F.softplus(delta))


def rms_norm(x, weight, eps=1e-6):
    """``x * rsqrt(mean(x^2) + eps).to(x.dtype) * w`` with an fp32 norm (``vdn_h3/branch.py:494-498``)."""
    ms = torch.linalg.vector_norm(x, dim=-1, keepdim=True, dtype=torch.float32).square() / x.shape[-1]
    return x * torch.rsqrt(ms + eps).to(x.dtype) * weight.to(x.dtype)


def linear_epilogue(readout_fhsd, norm_weight, gate, eps=1e-6):
    """RMSNorm, FHSD -> rows, times the output gate (``vdn_h3/branch.py:501-505``)."""
    normalized = rms_norm(readout_fhsd, norm_weight, eps)
    frames, heads, tokens, head_dim = normalized.shape
    rows = frames * tokens
    return normalized.permute(0, 2, 1, 3).reshape(rows, heads * head_dim) * gate.reshape(rows, heads * head_dim)


def linear_bf16(x, weight, bias=None):
    """``F.linear`` in the activation dtype (bf16 GEMM, fp32 accumulate, one rounding)."""
    y = torch.matmul(x.float(), weight.float().t())
    if bias is not None:
        y = y + bias.float()
    return y.to(x.dtype)


def text_state(weights, text_x, text_k_raw, text_v_raw, num_heads, head_dim, delta_rule="vdn_solve",
               a_fp32=True, stats=None):
    """``0.5 * B_text (I + A_text)^-1`` over all text rows as one frame (``vdn_h3/branch.py:649-670``).

    ``stats``: ``(A_text, B_text)`` ``[1, H, D, D]`` to use instead of computing them (a test hook that
    isolates everything after the statistics)."""
    length = text_x.shape[0]
    if stats is None:
        key = activate(text_k_raw, True).reshape(1, length, num_heads, head_dim).permute(0, 2, 1, 3)
        value = activate(text_v_raw, False).reshape(1, length, num_heads, head_dim).permute(0, 2, 1, 3)
        beta = torch.sigmoid(linear_bf16(text_x, weights["beta_proj.weight"]))
        beta = beta.reshape(1, length, num_heads).permute(0, 2, 1)
        matrix_a, matrix_b = frame_statistics(key, value, beta, a_fp32)
    else:
        matrix_a, matrix_b = (t.float() for t in stats)
    ones = torch.ones(1, num_heads, head_dim, dtype=matrix_a.dtype)
    if delta_rule == "vdn_solve":
        _, injection, info = vdn_factor(ones, matrix_a, matrix_b)
    else:
        _, injection = sana_factor(ones, matrix_a, matrix_b, length)
        info = torch.zeros(1, num_heads, dtype=torch.int32)
    return TEXT_STATE_SCALE * injection[0], info


def features(weights, q_raw, k_raw, v_raw, num_frames, frame_size, short_conv=(), fused_conv=False):
    """q, k, v features in FHSD layout (``vdn_h3/runtime.py:311-359``).

    ``fused_conv`` selects the CUDA spelling of the short convolutions (``conv_features_fused``).
    """
    heads, head_dim = q_raw.shape[-2:]
    out = []
    conv = conv_features_fused if fused_conv else conv_features
    for name, raw in (("q", q_raw), ("k", k_raw), ("v", v_raw)):
        l2 = name != "v"
        if name in short_conv:
            rows = conv(raw, weights[f"short_conv.{name}_sp.weight"],
                        weights[f"short_conv.{name}_tm.weight"], num_frames, frame_size, l2)
        else:
            rows = activate(raw, l2)
        out.append(to_fhsd(rows, num_frames, heads, head_dim))
    return out


def readout(weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds, *, frame_size=None,
            text_x=None, text_k_raw=None, text_v_raw=None, short_conv=(), delta_rule="vdn_solve",
            bridge="alpha", a_fp32=True, return_parts=False, fused_conv=False, stats=None, text_stats=None,
            gate_hidden=None):
    """Inference readout before ``to_out_linear`` (``vdn_h3/runtime.py:361-419``).

    Returns ``[F*T, H*D]`` in the activation dtype (and the intermediate tensors with
    ``return_parts=True``). Test hooks: ``stats`` / ``text_stats`` = ``(A, B)`` of the frames / the text
    rows and ``gate_hidden`` = the output gate's down-projection ``[F*T, D]`` replace the values this
    function would compute, so a comparison can start after the bf16 roundings they contain.
    """
    heads, head_dim = q_raw.shape[-2:]
    rows = num_frames * tokens_per_frame
    qf, kf, vf = features(weights, q_raw, k_raw, v_raw, num_frames, frame_size, short_conv, fused_conv)
    beta = torch.sigmoid(linear_bf16(xv, weights["beta_proj.weight"]))
    beta = beta.reshape(num_frames, tokens_per_frame, heads).permute(0, 2, 1)
    if stats is None:
        matrix_a, matrix_b = frame_statistics(kf, vf, beta, a_fp32)
    else:
        matrix_a, matrix_b = (t.float() for t in stats)
    frame_mean = xv.reshape(num_frames, tokens_per_frame, -1).mean(dim=1, dtype=torch.float32)
    alpha = alpha_gate(frame_mean, weights["alpha.down.weight"], weights["alpha.up.weight"],
                       weights["alpha.dt_bias"], weights["alpha.A_log"], heads, head_dim)
    tstate, tinfo = (None, None)
    if text_x is not None:
        tstate, tinfo = text_state(weights, text_x, text_k_raw, text_v_raw, heads, head_dim, delta_rule, a_fp32,
                                   stats=text_stats)
    if delta_rule == "vdn_solve":
        phi, jay, info = vdn_factor(alpha, matrix_a, matrix_b)
    else:
        phi, jay = sana_factor(alpha, matrix_a, matrix_b, tokens_per_frame)
        info = torch.zeros(num_frames, heads, dtype=torch.int32)
    initial = torch.zeros_like(jay[0]) if tstate is None else tstate
    prefix, suffix = run_scans(phi, jay, initial)
    hidden = linear_bf16(xv, weights["output_gate.down.weight"]) if gate_hidden is None else gate_hidden
    gate = torch.sigmoid(linear_bf16(hidden, weights["output_gate.up.weight"], weights.get("output_gate.up.bias")))
    state = gather_linear_state(prefix, suffix, alpha, bounds, bridge=bridge, text_state=tstate,
                                out_dtype=gate.dtype)
    read = bf16_matmul(qf, state.transpose(-1, -2)) if qf.dtype == torch.bfloat16 else qf @ state.transpose(-1, -2)
    flat = linear_epilogue(read, weights["norm.weight"], gate, 1e-6).reshape(rows, heads * head_dim)
    if return_parts:
        return flat, dict(qf=qf, kf=kf, vf=vf, beta=beta, A=matrix_a, B=matrix_b, alpha=alpha, phi=phi,
                          jay=jay, info=info, text_state=tstate, text_info=tinfo, prefix=prefix,
                          suffix=suffix, gate=gate, state=state, readout=read)
    return flat


def projected_delta(weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds, *,
                    frame_size=None, text_x=None, text_k_raw=None, text_v_raw=None, skip_ends=False,
                    projector=None, **kwargs):
    """Branch output after ``to_out_linear`` with anchor rows zeroed (``vdn_h3/runtime.py:545-607``)."""
    if projector is None:
        weight = weights["to_out_linear.weight"]
        projector = lambda value: linear_bf16(value, weight)  # noqa: E731
    original_rows = num_frames * tokens_per_frame
    row_offset = 0
    if skip_ends:
        if num_frames <= 2:
            return xv.new_zeros(original_rows, int(weights["to_out_linear.weight"].shape[0]))
        row_offset = tokens_per_frame
        inner = slice(row_offset, (num_frames - 1) * tokens_per_frame)
        xv = xv[inner]
        q_raw, k_raw, v_raw = q_raw[inner], k_raw[inner], v_raw[inner]
        num_frames -= 2
        bounds = [(lo - 1, hi - 1) for lo, hi in bounds[1:-1]]
    flat = readout(weights, xv, q_raw, k_raw, v_raw, num_frames, tokens_per_frame, bounds,
                   frame_size=frame_size, text_x=text_x, text_k_raw=text_k_raw, text_v_raw=text_v_raw, **kwargs)
    active = projector(flat.to(dtype=xv.dtype))
    if not skip_ends:
        return active
    out = active.new_zeros(original_rows, active.shape[-1])
    out[row_offset:row_offset + active.shape[0]] = active
    return out
