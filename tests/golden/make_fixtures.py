"""Writes the committed fixtures under tests/golden/ (run from the repository root:
`python -m tests.golden.make_fixtures`). They freeze independently derived answers so
that a change to the oracle or to the reference mathematics of tests/refmath.py shows
up as a fixture mismatch:
  mxfp4_kat.npy   bf16 bits of e2m1(code) * 2^(s - 127) for all 256 scales x 16 codes,
                  from exact rational round-to-nearest-even (refmath.mxfp4_kat);
  tiny_layer.npz  a seeded 4-expert layer (H = I = 64, k = 2), 3 tokens, and the float64
                  brute-force layer (refmath.moe_layer_f64): out, top-k indices, weights.
Nothing here runs the reference or the oracle.
"""
import os

import numpy as np

from physllm_amd import synthetic as syn
from tests import refmath

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    np.save(os.path.join(HERE, "mxfp4_kat.npy"), refmath.mxfp4_kat())
    layer = syn.make_layer(4, 64, 64, 2, seed=3)
    x = syn.make_x(3, 64, seed=11)
    out, idx, w = refmath.moe_layer_f64(layer, x)
    np.savez_compressed(
        os.path.join(HERE, "tiny_layer.npz"),
        router_w=layer.router_w, router_b=layer.router_b, gate_up_blocks=layer.gate_up_blocks,
        gate_up_scales=layer.gate_up_scales, gate_up_bias=layer.gate_up_bias, down_blocks=layer.down_blocks,
        down_scales=layer.down_scales, down_bias=layer.down_bias, x=x, out_f64=out, idx=idx, w=w,
        shape=np.array([4, 64, 64, 2]))
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
