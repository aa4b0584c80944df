"""Packed VDN-H3 sequence geometry and its request-local publication.

Mirrors ``vdn_h3/layout.py`` (VDNLayout ``:19-41``, ``CURRENT_LAYOUT`` / ``current_layout`` /
``publish_layout`` ``:44-69``, ``from_comfy_packed_layout`` ``:106-159``,
``layout_from_payload`` ``:162-196``, ``with_window`` ``:199-202``): same fields, same
validation and the same exception types, so a caller written against the reference
works unchanged.
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass, replace
from typing import Any, Iterator, Sequence

from .window import full_coverage, window_bounds

_ANCHOR_MODES = frozenset({"none", "columns", "rows", "both"})


@dataclass(frozen=True, slots=True)
class VDNLayout:
    """Geometry of one packed sequence: text/global rows plus ``num_frames`` video frames."""

    seq_len: int
    video_start: int
    video_end: int
    num_frames: int
    tokens_per_frame: int
    frame_size: tuple[int, int]
    text_start: int
    text_len: int
    bounds: tuple[tuple[int, int], ...] = ()
    full_cover: bool = False
    anchor_frames: str = "both"

    @property
    def frame_height(self) -> int:
        return self.frame_size[0]

    @property
    def frame_width(self) -> int:
        return self.frame_size[1]


CURRENT_LAYOUT: ContextVar[VDNLayout | None] = ContextVar("vdn_h3_amd_layout", default=None)


def current_layout(*, required: bool = True) -> VDNLayout | None:
    """This execution context's layout (``RuntimeError`` if required and absent)."""
    layout = CURRENT_LAYOUT.get()
    if required and layout is None:
        raise RuntimeError(
            "VDN-H3 attention ran without a packed layout. Apply the model through the VDN-H3 node "
            "and do not invoke a patched attention block directly.")
    return layout


@contextmanager
def publish_layout(layout: VDNLayout) -> Iterator[VDNLayout]:
    """Publish ``layout`` for one forward; nested publications restore the outer one."""
    if not isinstance(layout, VDNLayout):
        raise TypeError(f"expected VDNLayout, got {type(layout).__name__}")
    token = CURRENT_LAYOUT.set(layout)
    try:
        yield layout
    finally:
        CURRENT_LAYOUT.reset(token)


def _one_segment(segments: Sequence[Any], kind: str) -> tuple[int, int]:
    found = []
    for segment in segments:
        if not isinstance(segment, (tuple, list)) or len(segment) < 3:
            raise TypeError(f"invalid PackedLayout segment {segment!r}")
        start, stop, value = segment[:3]
        if value == kind:
            found.append((int(start), int(stop)))
    if len(found) != 1:
        raise ValueError(f"expected exactly one {kind!r} segment, got {len(found)}")
    start, stop = found[0]
    if start < 0 or stop <= start:
        raise ValueError(f"invalid {kind!r} segment [{start}, {stop})")
    return start, stop


def _geometry(num_frames: int, radius: int, chunk: int):
    bounds = tuple((int(lo), int(hi)) for lo, hi in window_bounds(num_frames, radius, chunk))
    return bounds, bool(full_coverage(bounds, num_frames))


def from_comfy_packed_layout(packed: Any, *, radius: int = 1, chunk: int = 5,
                             anchor_frames: str = "both") -> VDNLayout:
    """Adapt a ComfyUI MiniMax-H3 ``PackedLayout`` (signature + segments) strictly."""
    if isinstance(radius, bool) or not isinstance(radius, int) or radius < 0:
        raise ValueError(f"window radius must be a non-negative integer, got {radius!r}")
    if isinstance(chunk, bool) or not isinstance(chunk, int) or chunk < 0:
        raise ValueError(f"window chunk must be a non-negative integer, got {chunk!r}")
    if anchor_frames not in _ANCHOR_MODES:
        raise ValueError(f"anchor_frames must be one of {sorted(_ANCHOR_MODES)}, got {anchor_frames!r}")
    try:
        signature = tuple(map(int, packed.signature))
        segments = tuple(packed.segments)
        seq_len = int(packed.seq_len)
    except (AttributeError, TypeError, ValueError) as exc:
        raise TypeError("not a compatible ComfyUI MiniMax-H3 PackedLayout") from exc
    if len(signature) != 5:
        raise ValueError("PackedLayout.signature must be (text_len, latent_t, latent_h, latent_w, audio_t), "
                         f"got {signature!r}")
    text_len, latent_t, latent_h, latent_w, _audio_t = signature
    if min(seq_len, text_len, latent_t, latent_h, latent_w) <= 0:
        raise ValueError(f"invalid PackedLayout signature/length: {signature!r}, seq={seq_len}")
    text_start, text_end = _one_segment(segments, "text")
    video_start, video_end = _one_segment(segments, "video")
    if text_end - text_start != text_len:
        raise ValueError("text segment length disagrees with PackedLayout.signature: "
                         f"{text_end - text_start} != {text_len}")
    if video_end > seq_len or text_end > seq_len:
        raise ValueError("a PackedLayout segment extends past the packed sequence")
    rows = video_end - video_start
    if rows % latent_t:
        raise ValueError(f"{rows} video rows are not divisible by {latent_t} latent frames")
    tokens_per_frame = rows // latent_t
    frame_size = ((latent_h + 1) // 2, (latent_w + 1) // 2)
    if frame_size[0] * frame_size[1] != tokens_per_frame:
        raise ValueError(f"patched grid {frame_size[0]}x{frame_size[1]} does not match "
                         f"{tokens_per_frame} video tokens per frame")
    bounds, full_cover = _geometry(latent_t, radius, chunk)
    return VDNLayout(seq_len=seq_len, video_start=video_start, video_end=video_end, num_frames=latent_t,
                     tokens_per_frame=tokens_per_frame, frame_size=frame_size, text_start=text_start,
                     text_len=text_len, bounds=bounds, full_cover=full_cover, anchor_frames=anchor_frames)


def layout_from_payload(payload: dict[str, Any] | None, x: Any, context: Any, config: dict[str, Any]) -> VDNLayout:
    """Use the payload's ``PackedLayout`` when it matches the input shapes.

    Rebuilding a missing layout needs ComfyUI's ``PackedLayout``; without ComfyUI this
    raises ``RuntimeError`` exactly as the reference does.
    """
    payload = payload or {}
    packed = payload.get("layout")
    try:
        video, audio = x[0], x[1]
        text_len = int(context.shape[1])
        latent_t, latent_h, latent_w = int(video.shape[2]), int(video.shape[3]), int(video.shape[4])
        audio_t = int(audio.shape[-1])
    except (IndexError, AttributeError, TypeError, ValueError) as exc:
        raise TypeError("VDN-H3 expected x=(video[B,C,T,H,W], audio[...,T]) and context[B,text,hidden]") from exc
    signature = (text_len, latent_t, (latent_h + 1) // 2 * 2, (latent_w + 1) // 2 * 2, audio_t)
    if packed is None or tuple(getattr(packed, "signature", ())) != signature:
        try:
            from comfy.ldm.minimax.model import PackedLayout  # noqa: PLC0415
        except ImportError as exc:
            raise RuntimeError("minimax_payload has no layout matching this input and ComfyUI's "
                               "MiniMax-H3 PackedLayout is unavailable") from exc
        packed = PackedLayout(*signature, keyframes=payload.get("keyframes"), refs=payload.get("refs"))
    return from_comfy_packed_layout(packed, radius=int(config.get("radius", 1)), chunk=int(config.get("chunk", 5)),
                                    anchor_frames=str(config.get("anchor_frames", "both")))


def with_window(layout: VDNLayout, *, radius: int, chunk: int) -> VDNLayout:
    """The same layout with recomputed window bounds and full-cover flag."""
    bounds, full_cover = _geometry(layout.num_frames, radius, chunk)
    return replace(layout, bounds=bounds, full_cover=full_cover)


def text_first_layout(text_len: int, num_frames: int, frame_size: tuple[int, int], *, radius: int = 1,
                      chunk: int = 5, anchor_frames: str = "both") -> VDNLayout:
    """Layout of a text-first packed sequence (``text_len`` rows, then the video frames)."""
    tokens = frame_size[0] * frame_size[1]
    bounds, full_cover = _geometry(num_frames, radius, chunk)
    return VDNLayout(seq_len=text_len + num_frames * tokens, video_start=text_len,
                     video_end=text_len + num_frames * tokens, num_frames=num_frames, tokens_per_frame=tokens,
                     frame_size=tuple(frame_size), text_start=0, text_len=text_len, bounds=bounds,
                     full_cover=full_cover, anchor_frames=anchor_frames)


__all__ = ["CURRENT_LAYOUT", "VDNLayout", "current_layout", "from_comfy_packed_layout", "layout_from_payload",
           "publish_layout", "text_first_layout", "with_window"]
