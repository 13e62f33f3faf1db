"""Independent reference mathematics used to pin the C oracle.

Nothing here reuses the oracle's formulas: e2m1 values come from the OCP MX
bit-level definition with exact rationals, bf16 encodings from exact
round-to-nearest-even on rationals, and layer maths from float64 numpy with
weights decoded by that rational decoder.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np


def e2m1_fraction(code: int):
    """(value, negative) of a 4-bit e2m1 code per the OCP MX v1.0 definition:
    1 sign bit, 2 exponent bits (bias 1), 1 mantissa bit, subnormal when e == 0."""
    s, e, m = (code >> 3) & 1, (code >> 1) & 3, code & 1
    mag = Fraction(m, 2) if e == 0 else Fraction(2) ** (e - 1) * (1 + Fraction(m, 2))
    return (-mag if s else mag), bool(s)


def bf16_bits_of_fraction(v: Fraction, negative: bool) -> int:
    """Exact round-to-nearest-even of a rational to bf16 bits (1-8-7, bias 127)."""
    sign = 0x8000 if negative else 0
    a = abs(Fraction(v))
    if a == 0:
        return sign
    E = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** E > a:
        E -= 1
    normal = E >= -126
    quantum = Fraction(2) ** (E - 7) if normal else Fraction(2) ** -133
    q = a / quantum
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    if not normal:
        return sign | n  # n == 128 encodes the smallest normal, as it should
    if n == 256:
        n, E = 128, E + 1
    if E > 127:
        return sign | 0x7F80
    return sign | ((E + 127) << 7) | (n - 128)


def mxfp4_kat():
    """uint16 [256 scales, 16 codes] of bf16(e2m1(code) * 2^(s-127)); s = 255 -> NaN."""
    out = np.zeros((256, 16), dtype=np.uint16)
    for s in range(256):
        for c in range(16):
            if s == 255:
                out[s, c] = 0x7FC0
                continue
            v, neg = e2m1_fraction(c)
            out[s, c] = bf16_bits_of_fraction(v * Fraction(2) ** (s - 127), neg)
    return out


def decode_table_f64():
    """float64 [256, 16] exact values (NaN for s = 255)."""
    t = np.zeros((256, 16), dtype=np.float64)
    for s in range(256):
        for c in range(16):
            v, _ = e2m1_fraction(c)
            t[s, c] = np.nan if s == 255 else float(v * Fraction(2) ** (s - 127))
    t[:, 8] = -0.0
    return t


_TAB = None


def decode_rows_f64(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """[..., R, C/2] u8 codes + [..., R, C/32] E8M0 -> float64 [..., R, C]."""
    global _TAB
    if _TAB is None:
        _TAB = decode_table_f64()
    lo = blocks & 15
    hi = blocks >> 4
    codes = np.stack([lo, hi], axis=-1).reshape(*blocks.shape[:-1], blocks.shape[-1] * 2)
    sc = np.repeat(scales, 32, axis=-1)
    return _TAB[sc, codes]


def bf16_bits_to_f64(u) -> np.ndarray:
    return (np.asarray(u, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def round_bf16_f64(a: np.ndarray) -> np.ndarray:
    """Round float64 values to bf16 (via float32) and return them as float64."""
    f = np.asarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def topk_desc_stable(logits: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest per row, descending, ties -> lower index (lexsort)."""
    E = logits.shape[-1]
    out = np.empty(logits.shape[:-1] + (k,), dtype=np.int64)
    for r in range(logits.shape[0]):
        key = np.where(np.isnan(logits[r]), -np.inf, logits[r])
        order = np.lexsort((np.arange(E), -key))
        out[r] = order[:k]
    return out


def swiglu_f64(g, u, alpha=1.702, limit=7.0):
    g = np.minimum(g, limit)
    u = np.clip(u, -limit, limit)
    return g / (1.0 + np.exp(-alpha * g)) * (u + 1.0)


def moe_layer_f64(layer, x_bits: np.ndarray, round_h: bool = True):
    """Float64 brute force of the MoE layer. Returns (out f64 [B,H], idx [B,K], w [B,K])."""
    x = bf16_bits_to_f64(x_bits)
    E, K = layer.num_experts, layer.top_k
    Wr = bf16_bits_to_f64(layer.router_w)
    br = bf16_bits_to_f64(layer.router_b) if layer.router_b is not None else np.zeros(E)
    logits = x @ Wr.T + br
    idx = topk_desc_stable(logits, K)
    sel = np.take_along_axis(logits, idx, axis=1)
    ex = np.exp(sel - sel.max(axis=1, keepdims=True))
    w = ex / ex.sum(axis=1, keepdims=True)
    Wgu = decode_rows_f64(layer.gate_up_blocks, layer.gate_up_scales)
    Wd = decode_rows_f64(layer.down_blocks, layer.down_scales)
    bgu = bf16_bits_to_f64(layer.gate_up_bias) if layer.gate_up_bias is not None else np.zeros(Wgu.shape[:2])
    bd = bf16_bits_to_f64(layer.down_bias) if layer.down_bias is not None else np.zeros(Wd.shape[:2])
    B = x.shape[0]
    out = np.zeros((B, layer.hidden))
    for t in range(B):
        for j in range(K):
            e = idx[t, j]
            gu = Wgu[e] @ x[t] + bgu[e]
            h = swiglu_f64(gu[0::2], gu[1::2], layer.alpha, layer.limit)
            if round_h:
                h = round_bf16_f64(h)
            y = Wd[e] @ h + bd[e]
            out[t] += w[t, j] * y
    return out, idx, w


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
