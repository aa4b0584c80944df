"""Packed VDN-H3 sequence geometry and its request-local publication.

Interface of ``vdn_h3/layout.py``: ``VDNLayout`` (``:19-41``), ``CURRENT_LAYOUT`` /
``current_layout`` / ``publish_layout`` (``:44-69``), ``from_comfy_packed_layout``
(``:106-159``), ``layout_from_payload`` (``:162-196``) and ``with_window`` (``:199-202``) keep
their names, fields, argument meaning and exception types (``TypeError`` for an object that
is not a PackedLayout, ``ValueError`` for inconsistent geometry, ``RuntimeError`` when no
layout is published or ComfyUI is needed and absent).

A ComfyUI ``PackedLayout`` is read once into a ``_PackedView``: the five signature numbers by
name and the segment spans grouped by kind. The checks then run over that record, and the
frame grid and window geometry are derived from it.
"""

from __future__ import annotations

from collections import defaultdict
from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass, replace
from typing import Any, Iterator, NamedTuple

from .window import ANCHOR_FRAME_MODES, full_coverage, window_bounds


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
    """The layout published in this execution context; ``RuntimeError`` if one is required and none is."""
    found = CURRENT_LAYOUT.get()
    if found is None and required:
        raise RuntimeError("no VDN-H3 packed layout is published for this forward: a patched attention "
                           "block must run inside the VDN-H3 model wrapper (publish_layout), not on its own")
    return found


@contextmanager
def publish_layout(layout: VDNLayout) -> Iterator[VDNLayout]:
    """Make ``layout`` the current one for the ``with`` body; the previous value comes back on exit."""
    if not isinstance(layout, VDNLayout):
        raise TypeError(f"publish_layout needs a VDNLayout, not {type(layout).__name__}")
    token = CURRENT_LAYOUT.set(layout)
    try:
        yield layout
    finally:
        CURRENT_LAYOUT.reset(token)


class _PackedView(NamedTuple):
    """The parts of a ComfyUI MiniMax-H3 ``PackedLayout`` this module reads."""

    seq_len: int
    text_len: int
    latent_t: int
    latent_h: int
    latent_w: int
    audio_t: int
    spans: dict  # segment kind -> list of (start, stop)

    def span(self, kind: str) -> tuple[int, int]:
        spans = self.spans.get(kind, ())
        if len(spans) != 1:
            raise ValueError(f"a PackedLayout needs one {kind!r} segment, it has {len(spans)}")
        start, stop = spans[0]
        if not 0 <= start < stop:
            raise ValueError(f"{kind!r} segment [{start}, {stop}) is empty or negative")
        return start, stop


def _read_packed(packed: Any) -> _PackedView:
    try:
        numbers = [int(v) for v in packed.signature]
        entries = list(packed.segments)
        seq_len = int(packed.seq_len)
    except (AttributeError, TypeError, ValueError) as exc:
        raise TypeError("expected a ComfyUI MiniMax-H3 PackedLayout with signature, segments and seq_len") from exc
    if len(numbers) != 5:
        raise ValueError("PackedLayout.signature has five entries (text_len, latent_t, latent_h, latent_w, "
                         f"audio_t); got {tuple(numbers)!r}")
    spans: dict[Any, list[tuple[int, int]]] = defaultdict(list)
    for entry in entries:
        if not isinstance(entry, (tuple, list)) or len(entry) < 3:
            raise TypeError(f"PackedLayout segment {entry!r} is not a (start, stop, kind, ...) sequence")
        spans[entry[2]].append((int(entry[0]), int(entry[1])))
    view = _PackedView(seq_len, *numbers, spans=dict(spans))
    if min(view.seq_len, view.text_len, view.latent_t, view.latent_h, view.latent_w) <= 0:
        raise ValueError(f"PackedLayout sizes must be positive: signature {tuple(numbers)!r}, seq_len {seq_len}")
    return view


def _check_window_args(radius: Any, chunk: Any, anchor_frames: Any) -> None:
    for name, value in (("radius", radius), ("chunk", chunk)):
        if isinstance(value, bool) or not isinstance(value, int) or value < 0:
            raise ValueError(f"window {name} must be an int >= 0, got {value!r}")
    if anchor_frames not in ANCHOR_FRAME_MODES:
        raise ValueError(f"anchor_frames {anchor_frames!r} is not one of {list(ANCHOR_FRAME_MODES)}")


def _window(num_frames: int, radius: int, chunk: int) -> tuple[tuple[tuple[int, int], ...], bool]:
    bounds = tuple((int(lo), int(hi)) for lo, hi in window_bounds(num_frames, radius, chunk))
    return bounds, bool(full_coverage(bounds, num_frames))


def _patched_grid(latent_h: int, latent_w: int) -> tuple[int, int]:
    """Token grid of one frame after MiniMax-H3's 2x2 patchify (odd sizes round up)."""
    return (latent_h + 1) // 2, (latent_w + 1) // 2


def from_comfy_packed_layout(packed: Any, *, radius: int = 1, chunk: int = 5,
                             anchor_frames: str = "both") -> VDNLayout:
    """The ``VDNLayout`` of a ComfyUI MiniMax-H3 ``PackedLayout``; every inconsistency raises."""
    _check_window_args(radius, chunk, anchor_frames)
    view = _read_packed(packed)
    text = view.span("text")
    video = view.span("video")
    if text[1] - text[0] != view.text_len:
        raise ValueError(f"the text segment holds {text[1] - text[0]} rows but the signature says {view.text_len}")
    if max(text[1], video[1]) > view.seq_len:
        raise ValueError(f"a segment ends past seq_len {view.seq_len}")
    tokens, remainder = divmod(video[1] - video[0], view.latent_t)
    if remainder:
        raise ValueError(f"{video[1] - video[0]} video rows do not split into {view.latent_t} equal frames")
    grid = _patched_grid(view.latent_h, view.latent_w)
    if grid[0] * grid[1] != tokens:
        raise ValueError(f"a {grid[0]}x{grid[1]} patch grid has {grid[0] * grid[1]} tokens, "
                         f"the video segment has {tokens} per frame")
    bounds, full_cover = _window(view.latent_t, radius, chunk)
    return VDNLayout(seq_len=view.seq_len, video_start=video[0], video_end=video[1], num_frames=view.latent_t,
                     tokens_per_frame=tokens, frame_size=grid, text_start=text[0], text_len=view.text_len,
                     bounds=bounds, full_cover=full_cover, anchor_frames=anchor_frames)


def _input_signature(x: Any, context: Any) -> tuple[int, int, int, int, int]:
    """``(text_len, latent_t, padded_h, padded_w, audio_t)`` of a model call's inputs."""
    try:
        video, audio = x[0], x[1]
        t, h, w = (int(n) for n in tuple(video.shape)[2:5])
        return int(context.shape[1]), t, 2 * ((h + 1) // 2), 2 * ((w + 1) // 2), int(audio.shape[-1])
    except (IndexError, AttributeError, TypeError, ValueError) as exc:
        raise TypeError("VDN-H3 needs x = (video [B, C, T, H, W], audio [..., T]) and context "
                        "[B, text, hidden]") from exc


def layout_from_payload(payload: dict[str, Any] | None, x: Any, context: Any, config: dict[str, Any]) -> VDNLayout:
    """The layout of one model call: the payload's ``PackedLayout`` when its signature matches the
    inputs, else a new one built with ComfyUI's ``PackedLayout`` (``RuntimeError`` without ComfyUI)."""
    payload = payload or {}
    signature = _input_signature(x, context)
    packed = payload.get("layout")
    if packed is None or tuple(getattr(packed, "signature", ())) != signature:
        try:
            from comfy.ldm.minimax.model import PackedLayout  # noqa: PLC0415
        except ImportError as exc:
            raise RuntimeError("no PackedLayout in the payload matches these inputs, and ComfyUI's MiniMax-H3 "
                               "PackedLayout cannot be imported to build one") from exc
        packed = PackedLayout(*signature, keyframes=payload.get("keyframes"), refs=payload.get("refs"))
    settings = {"radius": 1, "chunk": 5, "anchor_frames": "both"}
    settings.update({key: config[key] for key in settings if key in config})
    return from_comfy_packed_layout(packed, radius=int(settings["radius"]), chunk=int(settings["chunk"]),
                                    anchor_frames=str(settings["anchor_frames"]))


def with_window(layout: VDNLayout, *, radius: int, chunk: int) -> VDNLayout:
    """``layout`` with its window bounds and full-cover flag recomputed for ``radius`` / ``chunk``."""
    bounds, full_cover = _window(layout.num_frames, radius, chunk)
    return replace(layout, bounds=bounds, full_cover=full_cover)


def text_first_layout(text_len: int, num_frames: int, frame_size: tuple[int, int], *, radius: int = 1,
                      chunk: int = 5, anchor_frames: str = "both") -> VDNLayout:
    """Layout of a text-first packed sequence (``text_len`` rows, then the video frames)."""
    _check_window_args(radius, chunk, anchor_frames)
    tokens = frame_size[0] * frame_size[1]
    bounds, full_cover = _window(num_frames, radius, chunk)
    return VDNLayout(seq_len=text_len + num_frames * tokens, video_start=text_len,
                     video_end=text_len + num_frames * tokens, num_frames=num_frames, tokens_per_frame=tokens,
                     frame_size=tuple(frame_size), text_start=0, text_len=text_len, bounds=bounds,
                     full_cover=full_cover, anchor_frames=anchor_frames)


__all__ = ["ANCHOR_FRAME_MODES", "CURRENT_LAYOUT", "VDNLayout", "current_layout", "from_comfy_packed_layout",
           "layout_from_payload", "publish_layout", "text_first_layout", "with_window"]
