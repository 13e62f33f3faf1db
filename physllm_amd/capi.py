"""ctypes binding of libphysllm_moe.so (the C ABI in include/physllm_moe.h).

Loading fails loudly when the library has not been built: there is no CPU or
PyTorch fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libphysllm_moe.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "physllm_moe.h")

PHYSLLM_MOE_OK = 0
PHYSLLM_MOE_EINVAL = -1
PHYSLLM_MOE_EWORKSPACE = -2
PHYSLLM_MOE_ELAUNCH = -3


class MoEConfig(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("intermediate", ctypes.c_int),
                ("num_experts", ctypes.c_int), ("top_k", ctypes.c_int),
                ("swiglu_alpha", ctypes.c_float), ("swiglu_limit", ctypes.c_float),
                ("max_chunk_tokens", ctypes.c_int)]


class MoEWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "router_w", "router_b", "gate_up_blocks", "gate_up_scales", "gate_up_bias",
        "down_blocks", "down_scales", "down_bias")]


_lib = None


def header_symbols() -> list:
    """Names of the functions include/physllm_moe.h declares."""
    text = open(HEADER_PATH).read()
    return re.findall(r"PHYSLLM_MOE_API\s+[\w\s\*]+?\b(\w+)\s*\(", text)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run `python -m physllm_amd.build` "
                           "(there is no fallback path)")
    L = ctypes.CDLL(LIB_PATH)
    P, I, I64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    sig = {
        "physllm_moe_last_error": ([], I),
        "physllm_moe_last_error_message": ([], ctypes.c_char_p),
        "launch_moe_router": ([P, P, P, P, I, I, I, I, P], None),
        "launch_moe_expert_silu": ([P, P, P, P, I, I, P], None),
        "launch_moe_expert_down": ([P, P, P, I, I, P], None),
        "launch_moe_combine": ([P, P, P, I, I, P], None),
        "launch_mxfp4_dequant": ([P, P, P, I, I, P], None),
        "launch_rms_norm": ([P, P, P, I, I, ctypes.c_float, P], None),
        "launch_residual_add": ([P, P, I, P], None),
        "physllm_moe_workspace_bytes": ([ctypes.POINTER(MoEConfig), I], SZ),
        "physllm_moe_layer_forward": ([ctypes.POINTER(MoEConfig), ctypes.POINTER(MoEWeights), P, I, P,
                                       P, P, P, SZ, P], I),
        "physllm_moe_layer_forward_noalloc": ([ctypes.POINTER(MoEConfig), ctypes.POINTER(MoEWeights), P, I, P,
                                               P, P, P], I),
        "physllm_moe_block_workspace_bytes": ([ctypes.POINTER(MoEConfig), I], SZ),
        "physllm_moe_block_forward": ([ctypes.POINTER(MoEConfig), ctypes.POINTER(MoEWeights), P, P,
                                       ctypes.c_float, I, P, P, P, P, SZ, P], I),
        "physllm_moe_stage_route": ([ctypes.POINTER(MoEConfig), ctypes.POINTER(MoEWeights), P, I, P, P, P,
                                     SZ, P], I),
        "physllm_moe_stage_gate_up": ([ctypes.POINTER(MoEConfig), ctypes.POINTER(MoEWeights), P, I, P, SZ,
                                       P], I),
        "physllm_moe_stage_down": ([ctypes.POINTER(MoEConfig), ctypes.POINTER(MoEWeights), I, P, SZ, P], I),
        "physllm_moe_stage_combine": ([ctypes.POINTER(MoEConfig), I, P, P, P, SZ, P], I),
        "physllm_moe_stage_batch1": ([ctypes.POINTER(MoEConfig), ctypes.POINTER(MoEWeights), P, I, I, P, P, SZ,
                                      P], I),
        "physllm_moe_route_topk": ([P, P, P, I, I, I, I, P, P, P], I),
        "physllm_moe_bucket": ([P, I, I, I, P, P, P, P, P], I),
        "physllm_moe_mxfp4_dequant": ([P, P, P, I64, P], I),
        "physllm_moe_mxfp4_dequant_transpose": ([P, P, P, I, I, I, I, P], I),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes, f.restype = args, res
    _lib = L
    return L


class BackendError(RuntimeError):
    """Raised when an entry point reports an error (mirrors rocm-backend's BackendError)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"physllm_moe error {code}: {msg}")
        self.code = code


def last_error():
    L = lib()
    return int(L.physllm_moe_last_error()), (L.physllm_moe_last_error_message() or b"").decode()


def check(rc=None):
    """Raise BackendError if rc (or, for void entry points, the last error) is nonzero."""
    code, msg = last_error()
    if rc is None:
        rc = code
    if rc != 0:
        raise BackendError(rc, msg)
