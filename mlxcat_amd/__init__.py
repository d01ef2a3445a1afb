"""MI355X (gfx950) n-gram speculative-decode step behind a C ABI (include/mlxcat_hip.h).

The compute path is libmlxcat_hip.so (hand-written HIP kernels); importing a
submodule that needs it raises if the library has not been built.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
