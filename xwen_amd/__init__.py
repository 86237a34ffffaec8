"""xwen_amd: MI355X-native (gfx950, HIP) token sampling for xwen.

The kernels and the C ABI live in xwen_amd/csrc (built into xwen_amd/libxsamp.so);
xwen_amd.sampler mirrors the reference's Sampler interface over that ABI.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
