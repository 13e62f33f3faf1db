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


def rms_norm_f64(x_bits: np.ndarray, w_bits: np.ndarray, eps: float) -> np.ndarray:
    """Float64 RMSNorm: x / sqrt(mean(x^2) + eps) * w, per row (no rounding)."""
    x = bf16_bits_to_f64(x_bits)
    w = bf16_bits_to_f64(w_bits)
    rms = np.sqrt((x * x).mean(axis=-1, keepdims=True) + np.float64(np.float32(eps)))
    return x / rms * w


def bf16_ulp_distance(a_bits, b_bits) -> np.ndarray:
    """Distance in representable bf16 steps between finite bf16 values (sign aware)."""
    def key(u):
        u = np.asarray(u, dtype=np.uint16).astype(np.int64)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return np.abs(key(a_bits) - key(b_bits))


def f32_of_bits(u) -> np.ndarray:
    return (np.asarray(u, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bits_of_f32_rne(f) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (finite inputs)."""
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def sum_sq_f32(v: np.ndarray, order: str):
    """Sum of squares of a float32 row in float32, in one of two orders:
    'tree' = kernels/rms_norm_gpu.hip:11-21 (256 strided partials, then
    p[:s] += p[s:2s] for s = 128..1), written as array operations;
    'serial' = left to right (a plausible mistake)."""
    sq = v * v  # exact for bf16 inputs of normal magnitude
    if order == "serial":
        t = np.float32(0)
        for q in sq:
            t = np.float32(t + q)
        return t
    n = -(-v.size // 256) * 256
    cols = np.zeros(n, dtype=np.float32)
    cols[: v.size] = sq
    p = np.zeros(256, dtype=np.float32)
    for r in cols.reshape(-1, 256):
        p = p + r
    s = 128
    while s:
        p[:s] = p[:s] + p[s:2 * s]
        s //= 2
    return p[0]


def rms_order_sensitive_row(H: int, seed: int):
    """A bf16 row x and weights w (all 1.0 but w[i]) for which RMSNorm (eps = 0) gives
    a different output bit at i when the sum of squares is taken left to right
    instead of in the tree order. Returns (x, w, i, bits_tree, bits_serial)."""
    rng = np.random.default_rng(seed)
    wall = np.arange(0x0080, 0x7000, dtype=np.uint16)  # positive normal bf16 below 2^97
    wf = f32_of_bits(wall)
    for _ in range(50):
        x = bits_of_f32_rne(rng.standard_normal(H).astype(np.float32))
        v = f32_of_bits(x)
        r_tree = np.sqrt(np.float32(sum_sq_f32(v, "tree") / np.float32(H)))
        r_ser = np.sqrt(np.float32(sum_sq_f32(v, "serial") / np.float32(H)))
        if r_tree == r_ser:
            continue
        for i in range(H):
            b1 = bits_of_f32_rne((v[i] / r_tree) * wf)
            b2 = bits_of_f32_rne((v[i] / r_ser) * wf)
            hit = np.flatnonzero(b1 != b2)
            if hit.size:
                w = np.full(H, 0x3F80, dtype=np.uint16)
                w[i] = wall[hit[0]]
                return x, w, i, b1[hit[0]], b2[hit[0]]
    raise RuntimeError("no order-sensitive row found")


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))
