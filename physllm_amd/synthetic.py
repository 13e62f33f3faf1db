"""Seeded synthetic inputs for the MXFP4 MoE layer (host side, numpy).

Every tensor of a configuration comes from one 64-bit seed (numpy SeedSequence ->
one PCG64 stream per tensor, in a fixed order), so the GPU path and the CPU
oracle see identical bytes. Distributions follow the benchmark configurations:

* packed e2m1 bytes uniform over 0..255 (both nibbles uniform over 0..15);
* E8M0 scales 127 + U{-8..-4};
* expert biases, router weight and router bias bf16 from N(0, 0.02);
* activations x bf16 from N(0, 1);
* optional Zipf(1.1) router skew: bias_e += ln p_e - mean(ln p), p_e ~ r_e^-1.1 for a
  seeded permutation r of 1..E.

Weight layout (the extension ABI's layout, shared with the GPT-OSS checkpoints):
gate_up_blocks [E, 2I, H/2] u8 with row 2i = gate_i and row 2i+1 = up_i, byte b of a
row holding element 2b in its low nibble and 2b+1 in its high nibble;
gate_up_scales [E, 2I, H/32] u8; gate_up_bias [E, 2I] bf16; down_blocks [E, H, I/2];
down_scales [E, H, I/32]; down_bias [E, H]; router_w [E, H]; router_b [E].
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

GPT_OSS_HIDDEN = 2880
GPT_OSS_INTERMEDIATE = 2880
SWIGLU_ALPHA = 1.702
SWIGLU_LIMIT = 7.0


def bf16_from_f32(a) -> np.ndarray:
    """Round float32 to bf16 (nearest-even); returns the uint16 bit patterns."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_to_f32(u) -> np.ndarray:
    u = np.ascontiguousarray(u, dtype=np.uint16)
    return (u.astype(np.uint32) << 16).view(np.float32)


@dataclass
class MoELayer:
    hidden: int
    intermediate: int
    num_experts: int
    top_k: int
    router_w: np.ndarray
    router_b: Optional[np.ndarray]
    gate_up_blocks: np.ndarray
    gate_up_scales: np.ndarray
    gate_up_bias: Optional[np.ndarray]
    down_blocks: np.ndarray
    down_scales: np.ndarray
    down_bias: Optional[np.ndarray]
    alpha: float = SWIGLU_ALPHA
    limit: float = SWIGLU_LIMIT

    @property
    def expert_bytes(self) -> int:
        """Algorithmic HBM bytes of one expert: packed codes + scales + biases."""
        H, I = self.hidden, self.intermediate
        return (2 * I * H // 2 + H * I // 2) + (2 * I * H // 32 + H * I // 32) + 2 * (2 * I + H)

    @property
    def weight_bytes(self) -> int:
        return sum(a.nbytes for a in (self.router_w, self.router_b, self.gate_up_blocks,
                                      self.gate_up_scales, self.gate_up_bias,
                                      self.down_blocks, self.down_scales, self.down_bias)
                   if a is not None)


def _rngs(seed: int, n: int):
    ss = np.random.SeedSequence(int(seed))
    return [np.random.Generator(np.random.PCG64(s)) for s in ss.spawn(n)]


def _normal_bf16(rng, shape, sigma: float) -> np.ndarray:
    return bf16_from_f32(rng.standard_normal(size=shape, dtype=np.float32) * np.float32(sigma))


def _bytes(rng, shape) -> np.ndarray:
    n = int(np.prod(shape))
    return np.frombuffer(rng.bytes(n), dtype=np.uint8).reshape(shape).copy()


def make_layer(num_experts: int, hidden: int = GPT_OSS_HIDDEN,
               intermediate: int = GPT_OSS_INTERMEDIATE, top_k: int = 4, seed: int = 0,
               scale_exp_lo: int = -8, scale_exp_hi: int = -4, bias_sigma: float = 0.02,
               router_sigma: float = 0.02, zipf: Optional[float] = None,
               with_bias: bool = True) -> MoELayer:
    E, H, I = num_experts, hidden, intermediate
    if H % 32 or I % 32:
        raise ValueError("hidden and intermediate must be multiples of 32")
    r = _rngs(seed, 10)
    gub = _bytes(r[0], (E, 2 * I, H // 2))
    gus = (127 + r[1].integers(scale_exp_lo, scale_exp_hi + 1, size=(E, 2 * I, H // 32))).astype(np.uint8)
    db = _bytes(r[2], (E, H, I // 2))
    ds = (127 + r[3].integers(scale_exp_lo, scale_exp_hi + 1, size=(E, H, I // 32))).astype(np.uint8)
    gbias = _normal_bf16(r[4], (E, 2 * I), bias_sigma) if with_bias else None
    dbias = _normal_bf16(r[5], (E, H), bias_sigma) if with_bias else None
    rw = _normal_bf16(r[6], (E, H), router_sigma)
    rb = _normal_bf16(r[7], (E,), router_sigma) if with_bias else None
    if zipf is not None:
        ranks = r[8].permutation(E).astype(np.float64) + 1.0
        lnp = -zipf * np.log(ranks)
        skew = (lnp - lnp.mean()).astype(np.float32)
        base = bf16_to_f32(rb) if rb is not None else np.zeros(E, np.float32)
        rb = bf16_from_f32(base + skew)
    return MoELayer(H, I, E, top_k, rw, rb, gub, gus, gbias, db, ds, dbias)


def make_x(batch: int, hidden: int = GPT_OSS_HIDDEN, seed: int = 0, sigma: float = 1.0) -> np.ndarray:
    """Activations [B, H] bf16 from N(0, sigma); the stream is distinct from the layer's."""
    rng = _rngs(int(seed) ^ 0x5EED_0000_7A11_0001, 1)[0]
    return _normal_bf16(rng, (batch, hidden), sigma)


# The benchmark configurations (one seed each).
CONFIGS = {
    0: dict(workload="gpt-oss-20b MoE layer, decode B=1", num_experts=32, batch=1, zipf=None, seed=1000),
    1: dict(workload="MXFP4->bf16 dequant [32,5760,2880]", num_experts=32, batch=0, zipf=None, seed=1001),
    2: dict(workload="gpt-oss-20b MoE layer, decode B=64, Zipf(1.1) router skew", num_experts=32,
            batch=64, zipf=1.1, seed=1002),
    3: dict(workload="gpt-oss-20b MoE layer, prefill 4096 tokens", num_experts=32, batch=4096,
            zipf=None, seed=1003),
    4: dict(workload="gpt-oss-120b-shape MoE layer, decode B=256", num_experts=128, batch=256,
            zipf=None, seed=1004),
}


def make_config(index: int, hidden: int = GPT_OSS_HIDDEN, intermediate: int = GPT_OSS_INTERMEDIATE):
    c = CONFIGS[index]
    layer = make_layer(c["num_experts"], hidden, intermediate, 4, seed=c["seed"], zipf=c["zipf"])
    x = make_x(max(c["batch"], 1), hidden, seed=c["seed"])
    return layer, x


def make_dequant_input(shape=(32, 5760, 2880), seed: int = 1001, block_size: int = 32):
    """Config 1: packed [numel/2] u8 and E8M0 scales [numel/block_size] u8."""
    numel = int(np.prod(shape))
    r = _rngs(seed, 2)
    packed = _bytes(r[0], (numel // 2,))
    scales = (127 + r[1].integers(-8, -3, size=(numel // block_size,))).astype(np.uint8)
    return packed, scales, numel
