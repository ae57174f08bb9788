"""exact_amd: the exact integer forward path of exact-llm on AMD MI355X (gfx950).

Host side of the C ABI in include/exact_hip.h (libexact_hip.so, built in this directory).
"""
from ._lib import ExactError, LIB_PATH, load  # noqa: F401

__all__ = ["ExactError", "LIB_PATH", "load"]
