"""velox_amd -- MI355X-native (gfx950) decode backend for Velox's generated LLM runners.

The product is the HIP library behind include/velox_hip.h (velox_amd/csrc, built into
velox_amd/lib/libvelox_hip.so). This package holds its ctypes bindings (_lib), the host-side
mirror of the reference engine interface (engine.HipDecodeEngine) and the build script.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib", "engine", "build"]
