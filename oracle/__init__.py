"""CPU oracle for the VDN-H3 hybrid attention hot path.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU and in fp32 (integer
GEMMs in exact int64), the algorithm of hyukudan/ComfyUI-Kirei-VDN-H3 v0.3.3 for the
hybrid attention block. Each function cites the reference ``file:line`` it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline. The
product path (``vdn_h3_amd``) never imports it and has no CPU fallback.

Pinning (how each function is checked independently of its own formula) is listed in
the header of each module; a function with no independent check says
"parity unpinned" there.
"""
