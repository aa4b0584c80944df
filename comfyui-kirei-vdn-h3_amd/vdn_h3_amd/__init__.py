"""MI355X-native (gfx950) VDN-H3 hybrid attention hot path.

Python mirror of the hot-path API of hyukudan/ComfyUI-Kirei-VDN-H3 (``vdn_h3``):
``layout``, ``window``, ``branch``/``runtime``, ``softmax_kernels``, ``fp8``/``projection``
and ``hybrid``, each calling hand-written HIP kernels through the C ABI of
``libvdnh3.so`` (``include/vdnh3.h``).
"""

__version__ = "0.1.0"

from .layout import VDNLayout, current_layout, from_comfy_packed_layout, publish_layout  # noqa: E402

__all__ = ["__version__", "VDNLayout", "current_layout", "from_comfy_packed_layout", "publish_layout"]
