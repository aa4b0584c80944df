"""Stage timing of the hybrid block with HIP events (no synchronisation inside a forward).

Mirrors the role of ``DiagnosticsRecorder`` (``vdn_h3/diagnostics.py:26-174``): a disabled
recorder costs nothing; an enabled one records a start / end event pair on the current
stream around each named scope and resolves all pending pairs with one device
synchronisation in ``flush`` / ``snapshot``. Stage names follow the reference
(``attention.qkv``, ``attention.softmax``, ``attention.out_proj``, ``attention.linear_branch``;
the reference's ``attention.rope_norm`` runs inside ``attention.softmax`` here, whose
``attention.softmax.qkv_prepass`` / ``.kernel`` sub-stages time its two kernels).
"""

from __future__ import annotations

from contextlib import contextmanager

import torch


class DiagnosticsRecorder:
    def __init__(self, enabled: bool = False):
        self.enabled = bool(enabled)
        self._pending: list[tuple[str, torch.cuda.Event, torch.cuda.Event, torch.device]] = []
        self._stats: dict[str, list[float]] = {}

    @contextmanager
    def scope(self, name: str, device=None):
        if not self.enabled or device is None or torch.device(device).type != "cuda":
            yield
            return
        device = torch.device(device)
        stream = torch.cuda.current_stream(device)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        try:
            yield
        finally:
            end.record(stream)
            self._pending.append((name, start, end, device))

    def flush(self) -> None:
        if not self._pending:
            return
        for device in {d for *_, d in self._pending}:
            torch.cuda.synchronize(device)
        pending, self._pending = self._pending, []
        for name, start, end, _ in pending:
            entry = self._stats.setdefault(name, [0, 0.0, 0.0])
            ms = float(start.elapsed_time(end))
            entry[0] += 1
            entry[1] += ms
            entry[2] = max(entry[2], ms)

    def snapshot(self, *, flush: bool = True) -> dict:
        if flush:
            self.flush()
        stages = {name: {"count": c, "total_ms": t, "mean_ms": t / c, "max_ms": m}
                  for name, (c, t, m) in sorted(self._stats.items())}
        return {"enabled": self.enabled, "pending_samples": len(self._pending), "stages": stages}

    def clear(self) -> None:
        self._pending.clear()
        self._stats.clear()


__all__ = ["DiagnosticsRecorder"]
