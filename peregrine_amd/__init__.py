"""peregrine_amd — MI355X (gfx950) decode path for the Qwen3.5-9B-shaped 4-bit
token loop of XiaoConstantine/peregrine.

The product is libperegrine_hip.so (hand-written HIP kernels + a C++ host layer
behind the C ABI in include/peregrine_hip.h). This package binds that library
with ctypes; it contains no compute of its own and no fallback path.
"""
from ._lib import LIB_PATH, PrgError, declared_symbols, lib  # noqa: F401

__all__ = ["LIB_PATH", "PrgError", "declared_symbols", "lib"]
