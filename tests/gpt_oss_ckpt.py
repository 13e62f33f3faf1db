"""Writes small synthetic GPT-OSS MXFP4 checkpoints for the loader tests.

Files are written by the `safetensors` package (an independent implementation of
the format), with the tensor names of either published convention. No real
checkpoint is available offline, so the names are the external convention as
documented in physllm_amd/host/gpt_oss_checkpoint.hpp ("parity unpinned" for the
names themselves; the bytes and layouts are checked end to end).
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch
from safetensors.torch import save_file


def _bf16(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def _f32_of_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy((a.astype(np.uint32) << 16).view(np.float32).copy())


def layer_tensors(layer, i: int, norm_w: np.ndarray, naming: str = "hf", blocks_4d: bool = True,
                  f32_router: bool = False) -> dict:
    """Checkpoint tensors of MoE layer i from a physllm_amd.synthetic.MoELayer."""
    E, H, I = layer.num_experts, layer.hidden, layer.intermediate

    def blocks(b, R, C):
        t = torch.from_numpy(np.ascontiguousarray(b))
        return t.reshape(E, R, C // 32, 16) if blocks_4d else t.reshape(E, R, C // 2)

    rw = _f32_of_bits(layer.router_w) if f32_router else _bf16(layer.router_w)
    t = {
        "router_w": rw,
        "router_b": _bf16(layer.router_b) if layer.router_b is not None else None,
        "gu_blocks": blocks(layer.gate_up_blocks, 2 * I, H),
        "gu_scales": torch.from_numpy(np.ascontiguousarray(layer.gate_up_scales)),
        "gu_bias": _bf16(layer.gate_up_bias) if layer.gate_up_bias is not None else None,
        "dn_blocks": blocks(layer.down_blocks, H, I),
        "dn_scales": torch.from_numpy(np.ascontiguousarray(layer.down_scales)),
        "dn_bias": _bf16(layer.down_bias) if layer.down_bias is not None else None,
        "norm": _f32_of_bits(norm_w) if f32_router else _bf16(norm_w),
    }
    if naming == "hf":
        m = f"model.layers.{i}.mlp."
        names = {"router_w": m + "router.weight", "router_b": m + "router.bias",
                 "gu_blocks": m + "experts.gate_up_proj_blocks", "gu_scales": m + "experts.gate_up_proj_scales",
                 "gu_bias": m + "experts.gate_up_proj_bias", "dn_blocks": m + "experts.down_proj_blocks",
                 "dn_scales": m + "experts.down_proj_scales", "dn_bias": m + "experts.down_proj_bias",
                 "norm": f"model.layers.{i}.post_attention_layernorm.weight"}
    else:
        m = f"block.{i}.mlp."
        names = {"router_w": m + "gate.weight", "router_b": m + "gate.bias",
                 "gu_blocks": m + "mlp1_weight.blocks", "gu_scales": m + "mlp1_weight.scales",
                 "gu_bias": m + "mlp1_bias", "dn_blocks": m + "mlp2_weight.blocks",
                 "dn_scales": m + "mlp2_weight.scales", "dn_bias": m + "mlp2_bias", "norm": m + "norm.scale"}
    return {names[k]: v.contiguous() for k, v in t.items() if v is not None}


def write_checkpoint(d: str, layers: list, norms: list, top_k: int, naming: str = "hf", shards: int = 2,
                     blocks_4d: bool = True, f32_router: bool = False, eps: float = 1e-5,
                     extra: dict | None = None) -> str:
    """Layers [(MoELayer)], norm weights [H] per layer; tensors spread round-robin over
    `shards` files model-0000k-of-0000n.safetensors, plus config.json."""
    os.makedirs(d, exist_ok=True)
    allt = {}
    for i, (layer, nw) in enumerate(zip(layers, norms)):
        allt.update(layer_tensors(layer, i, nw, naming, blocks_4d, f32_router))
    if extra:
        allt.update(extra)
    names = sorted(allt)
    for s in range(shards):
        part = {n: allt[n] for n in names[s::shards]}
        save_file(part, os.path.join(d, f"model-{s + 1:05d}-of-{shards:05d}.safetensors"),
                  metadata={"format": "pt", "shard": str(s)})
    L0 = layers[0]
    if naming == "hf":
        cfg = {"hidden_size": L0.hidden, "intermediate_size": L0.intermediate,
               "num_local_experts": L0.num_experts, "num_experts_per_tok": top_k,
               "num_hidden_layers": len(layers), "rms_norm_eps": eps, "swiglu_limit": 7.0,
               "model_type": "gpt_oss"}
    else:
        cfg = {"hidden_size": L0.hidden, "intermediate_size": L0.intermediate, "num_experts": L0.num_experts,
               "experts_per_token": top_k, "num_hidden_layers": len(layers), "swiglu_limit": 7.0}
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)
    return d
