"""MI355X (gfx950) execution provider for OxiONNX's dense-contraction hot path.

libohip.so (C ABI, include/ohip.h) holds every kernel and the provider's host
logic; this package is its Python binding.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
