"""physllm_amd — MI355X (gfx950) MXFP4 MoE expert path behind PhysLLM's kernel ABI.

The product is libphysllm_moe.so (hand-written HIP in physllm_amd/csrc, C ABI in
include/physllm_moe.h). This package holds its build script, the ctypes binding,
the host operator layer mirroring crates/rocm-backend/src/ops.rs, and the seeded
synthetic-input generator used by the bench and the tests.
"""
from .capi import LIB_PATH, BackendError, lib  # noqa: F401

__all__ = ["LIB_PATH", "BackendError", "lib"]
