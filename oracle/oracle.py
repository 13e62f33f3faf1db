"""ctypes binding of the C oracle (oracle/moe_oracle.c) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
module, and only as the checker / the CPU baseline. Arrays are numpy; 16-bit
activations and weights are bf16 bit patterns stored as uint16.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build(force: bool = False) -> str:
    """Compile oracle/liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", _HERE], check=True)
    return _LIB_PATH


class _Cfg(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("intermediate", ctypes.c_int),
                ("num_experts", ctypes.c_int), ("top_k", ctypes.c_int),
                ("alpha", ctypes.c_float), ("limit", ctypes.c_float)]


class _W(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "router_w", "router_b", "gate_up_blocks", "gate_up_scales", "gate_up_bias",
        "down_blocks", "down_scales", "down_bias")]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I, I64, F, D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double
        L.or_bf16_to_f32.argtypes, L.or_bf16_to_f32.restype = [ctypes.c_uint16], F
        L.or_f32_to_bf16.argtypes, L.or_f32_to_bf16.restype = [F], ctypes.c_uint16
        L.or_e2m1_value.argtypes, L.or_e2m1_value.restype = [I], F
        L.or_mxfp4_value_bf16.argtypes, L.or_mxfp4_value_bf16.restype = [I, I], ctypes.c_uint16
        L.or_mxfp4_dequant.argtypes, L.or_mxfp4_dequant.restype = [P, P, P, I64, I, I], None
        L.or_router.argtypes, L.or_router.restype = [P, P, P, I, I, I, I, P, P, P, I], None
        L.or_router_logits_fp32_serial.argtypes = [P, P, I, I, I, P]
        L.or_router_logits_fp32_serial.restype = None
        L.or_topk_softmax.argtypes, L.or_topk_softmax.restype = [P, I, I, P, P], None
        L.or_bucket.argtypes, L.or_bucket.restype = [P, I, I, I, P, P, P, P], None
        L.or_swiglu.argtypes, L.or_swiglu.restype = [F, F, F, F], F
        L.or_moe_layer.argtypes = [ctypes.POINTER(_Cfg), ctypes.POINTER(_W), P, I, P, P, P, P, P, I]
        L.or_moe_layer.restype = I
        L.or_moe_experts.argtypes = [ctypes.POINTER(_Cfg), ctypes.POINTER(_W), P, I, P, P, P, P, P, I]
        L.or_moe_experts.restype = I
        L.or_legacy_expert_silu.argtypes, L.or_legacy_expert_silu.restype = [P, P, P, P, I, I], None
        L.or_legacy_expert_down.argtypes, L.or_legacy_expert_down.restype = [P, P, P, I, I], None
        L.or_legacy_combine.argtypes, L.or_legacy_combine.restype = [P, P, P, I, I], None
        L.or_rms_norm.argtypes, L.or_rms_norm.restype = [P, P, P, I, I, F], None
        L.or_residual_add.argtypes, L.or_residual_add.restype = [P, P, ctypes.c_size_t], None
        L.or_moe_block.argtypes = [ctypes.POINTER(_Cfg), ctypes.POINTER(_W), P, P, F, I, P, P, P, I]
        L.or_moe_block.restype = I
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    a = np.ascontiguousarray(a)
    assert a.dtype == dtype, (a.dtype, dtype)
    return a


def default_threads() -> int:
    return max(1, len(os.sched_getaffinity(0)))


def f32_to_bf16(f: float) -> int:
    return int(lib().or_f32_to_bf16(float(f)))


def mxfp4_value_bf16(code: int, scale: int) -> int:
    return int(lib().or_mxfp4_value_bf16(int(code), int(scale)))


def mxfp4_dequant(packed, scales, numel: int, block_size: int = 32, nthreads: int = 0):
    packed = _c(packed, np.uint8)
    scales = _c(scales, np.uint8)
    out = np.empty(numel, dtype=np.uint16)
    lib().or_mxfp4_dequant(_p(packed), _p(scales), _p(out), int(numel), int(block_size),
                           nthreads or default_threads())
    return out


def router(x, w, bias, K: int, nthreads: int = 0, return_logits: bool = False):
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    B, H = x.shape
    E = w.shape[0]
    bias = None if bias is None else _c(bias, np.uint16)
    idx = np.empty((B, K), dtype=np.int32)
    wts = np.empty((B, K), dtype=np.float32)
    logits = np.empty((B, E), dtype=np.float64) if return_logits else None
    lib().or_router(_p(x), _p(w), _p(bias), B, H, E, K, _p(idx), _p(wts), _p(logits),
                    nthreads or default_threads())
    return (idx, wts, logits) if return_logits else (idx, wts)


def router_logits_fp32_serial(x, w):
    x = _c(x, np.uint16)
    w = _c(w, np.uint16)
    B, H = x.shape
    E = w.shape[0]
    out = np.empty((B, E), dtype=np.float32)
    lib().or_router_logits_fp32_serial(_p(x), _p(w), B, H, E, _p(out))
    return out


def topk_softmax(logits, K: int):
    lg = _c(np.asarray(logits, dtype=np.float64), np.float64)
    idx = np.empty(K, dtype=np.int32)
    wts = np.empty(K, dtype=np.float32)
    lib().or_topk_softmax(_p(lg), lg.shape[-1], K, _p(idx), _p(wts))
    return idx, wts


def bucket(idx, E: int):
    idx = _c(idx, np.int32)
    B, K = idx.shape
    N = B * K
    counts = np.empty(E, dtype=np.int32)
    offsets = np.empty(E + 1, dtype=np.int32)
    perm = np.empty(N, dtype=np.int32)
    pos = np.empty(N, dtype=np.int32)
    lib().or_bucket(_p(idx), B, K, E, _p(counts), _p(offsets), _p(perm), _p(pos))
    return counts, offsets, perm, pos


def swiglu(g: float, u: float, alpha: float = 1.702, limit: float = 7.0) -> float:
    return float(lib().or_swiglu(float(g), float(u), float(alpha), float(limit)))


def _cfg_w(layer):
    cfg = _Cfg(layer.hidden, layer.intermediate, layer.num_experts, layer.top_k,
               layer.alpha, layer.limit)
    keep = {}
    vals = {}
    for n, dt in (("router_w", np.uint16), ("router_b", np.uint16),
                  ("gate_up_blocks", np.uint8), ("gate_up_scales", np.uint8),
                  ("gate_up_bias", np.uint16), ("down_blocks", np.uint8),
                  ("down_scales", np.uint8), ("down_bias", np.uint16)):
        a = getattr(layer, n)
        if a is None:
            vals[n] = None
        else:
            keep[n] = _c(a, dt)
            vals[n] = keep[n].ctypes.data
    return cfg, _W(**vals), keep


def moe_layer(layer, x, nthreads: int = 0, want_pairs: bool = False):
    """Full layer on the CPU. `layer` is a physllm_amd.synthetic.MoELayer-like object.
    Returns dict(out, idx, wts[, h_pairs, y_pairs])."""
    x = _c(x, np.uint16)
    B = x.shape[0]
    cfg, w, keep = _cfg_w(layer)
    K, H, I = layer.top_k, layer.hidden, layer.intermediate
    out = np.empty((B, H), dtype=np.uint16)
    idx = np.empty((B, K), dtype=np.int32)
    wts = np.empty((B, K), dtype=np.float32)
    hp = np.empty((B * K, I), dtype=np.uint16) if want_pairs else None
    yp = np.empty((B * K, H), dtype=np.float32) if want_pairs else None
    rc = lib().or_moe_layer(ctypes.byref(cfg), ctypes.byref(w), _p(x), B, _p(out), _p(idx),
                            _p(wts), _p(hp), _p(yp), nthreads or default_threads())
    if rc != 0:
        raise ValueError(f"or_moe_layer rc={rc}")
    r = dict(out=out, idx=idx, wts=wts)
    if want_pairs:
        r.update(h_pairs=hp, y_pairs=yp)
    return r


def moe_experts(layer, x, idx, wts, nthreads: int = 0, want_pairs: bool = False):
    x = _c(x, np.uint16)
    idx = _c(idx, np.int32)
    wts = _c(wts, np.float32)
    B = x.shape[0]
    cfg, w, keep = _cfg_w(layer)
    K, H, I = layer.top_k, layer.hidden, layer.intermediate
    out = np.empty((B, H), dtype=np.uint16)
    hp = np.empty((B * K, I), dtype=np.uint16) if want_pairs else None
    yp = np.empty((B * K, H), dtype=np.float32) if want_pairs else None
    rc = lib().or_moe_experts(ctypes.byref(cfg), ctypes.byref(w), _p(x), B, _p(idx), _p(wts),
                              _p(out), _p(hp), _p(yp), nthreads or default_threads())
    if rc != 0:
        raise ValueError(f"or_moe_experts rc={rc}")
    r = dict(out=out)
    if want_pairs:
        r.update(h_pairs=hp, y_pairs=yp)
    return r


def legacy_expert_silu(x, wg, wu):
    x, wg, wu = _c(x, np.uint16), _c(wg, np.uint16), _c(wu, np.uint16)
    I, H = wg.shape
    out = np.empty(I, dtype=np.uint16)
    lib().or_legacy_expert_silu(_p(x), _p(wg), _p(wu), _p(out), H, I)
    return out


def legacy_expert_down(inter, wd):
    inter, wd = _c(inter, np.uint16), _c(wd, np.uint16)
    H, I = wd.shape
    out = np.empty(H, dtype=np.uint16)
    lib().or_legacy_expert_down(_p(inter), _p(wd), _p(out), H, I)
    return out


def legacy_combine(y, w):
    y, w = _c(y, np.uint16), _c(w, np.float32)
    K, H = y.shape
    out = np.empty(H, dtype=np.uint16)
    lib().or_legacy_combine(_p(y), _p(w), _p(out), H, K)
    return out


def rms_norm(x, weight, eps: float):
    """kernels/rms_norm_gpu.hip:4-31 with bf16 data: x [B,H], weight [H] bf16 bits."""
    x, weight = _c(x, np.uint16), _c(weight, np.uint16)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    B, H = x.shape
    out = np.empty((B, H), dtype=np.uint16)
    lib().or_rms_norm(_p(x), _p(weight), _p(out), B, H, float(eps))
    return out


def residual_add(out, res):
    """kernels/residual_add.hip:4-10 with bf16 data: returns bf16(out + res)."""
    o = _c(out, np.uint16).copy()
    r = _c(res, np.uint16)
    lib().or_residual_add(_p(o), _p(r), o.size)
    return o


def moe_block(layer, x, norm_w, eps: float, nthreads: int = 0):
    """crates/llm-core/src/moe.rs:238-313: rms_norm -> MoE layer -> residual add.
    Returns dict(out, idx, wts)."""
    x = _c(x, np.uint16)
    norm_w = _c(norm_w, np.uint16)
    B = x.shape[0]
    cfg, w, keep = _cfg_w(layer)
    K, H = layer.top_k, layer.hidden
    out = np.empty((B, H), dtype=np.uint16)
    idx = np.empty((B, K), dtype=np.int32)
    wts = np.empty((B, K), dtype=np.float32)
    rc = lib().or_moe_block(ctypes.byref(cfg), ctypes.byref(w), _p(x), _p(norm_w), float(eps), B, _p(out),
                            _p(idx), _p(wts), nthreads or default_threads())
    if rc != 0:
        raise ValueError(f"or_moe_block rc={rc}")
    return dict(out=out, idx=idx, wts=wts)
