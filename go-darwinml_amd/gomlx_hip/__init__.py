"""gomlx_hip — host side of the MI355X GoMLX backend.

Layout:
  _lib    ctypes binding of include/gomlx_hip.h (libgomlx_hip.so)
  ops     direct op entry points on device tensors (import gomlx_hip.ops; needs torch)
  synth   seeded synthetic inputs
"""
from . import _lib, synth  # noqa: F401
from ._lib import BackendError  # noqa: F401

__all__ = ["BackendError", "synth", "load_library"]


def load_library():
    return _lib.load()
