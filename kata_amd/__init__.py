"""kata_amd — MI355X (gfx950) ternary-matmul hot path of the Kata engine.

The compute path is the HIP library kata_amd/libkata_amd.so (C ABI: include/kata_amd.h);
this package is its host-side mirror: ctypes bindings (`kata_amd.capi`), torch-tensor
wrappers (`kata_amd.ops`) and the engine-style dispatcher (`kata_amd.engine`).
Importing never falls back to a CPU path: a missing library raises.
"""
from .capi import KataError, lib, library_path  # noqa: F401

__all__ = ["KataError", "lib", "library_path"]
