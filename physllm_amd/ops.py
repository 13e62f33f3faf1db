"""Host-side operator layer over the C ABI, mirroring crates/rocm-backend/src/ops.rs.

The reference's Rust wrappers (ops.rs:597-696) derive sizes from the tensors,
launch on the device's stream and then call dev.synchronise(), turning HIP
errors into BackendError. The functions here keep those names, argument
meanings and error behaviour; PyTorch supplies device memory and the stream
(plumbing only — every computation runs in libphysllm_moe.so).

Tensors holding bf16 data may be torch.bfloat16 or torch.int16 (raw bits).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import capi
from .capi import BackendError, MoEConfig, MoEWeights, check, lib


class GpuDevice:
    """One HIP device and its stream (crates/rocm-backend/src/device.rs:24-27)."""

    def __init__(self, idx: int = 0, stream: Optional[torch.cuda.Stream] = None):
        if not torch.cuda.is_available():
            raise BackendError(capi.PHYSLLM_MOE_ELAUNCH, "no HIP device available")
        self.device = torch.device("cuda", idx)
        self.stream = stream if stream is not None else torch.cuda.current_stream(self.device)

    def raw_stream(self) -> int:
        return self.stream.cuda_stream

    def synchronise(self) -> None:
        self.stream.synchronize()


def _ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if not t.is_cuda or not t.is_contiguous():
        raise BackendError(capi.PHYSLLM_MOE_EINVAL, "tensor must be a contiguous device tensor")
    return t.data_ptr()


def _rows_cols(t: torch.Tensor):
    rows = t.shape[-2] if t.dim() >= 2 else 1
    return rows, t.shape[-1]


# ---- legacy wrappers (ops.rs:597-696) -------------------------------------------

def moe_router_gpu(dev: GpuDevice, hidden, router_weight, expert_indices, expert_weights,
                   num_experts: int, top_k: int) -> None:
    """ops.rs:597-618: batch = hidden.rows(), hidden_dim = hidden.cols()."""
    batch, hidden_dim = _rows_cols(hidden)
    lib().launch_moe_router(_ptr(hidden), _ptr(router_weight), _ptr(expert_indices),
                            _ptr(expert_weights), batch, hidden_dim, num_experts, top_k,
                            dev.raw_stream())
    check()
    dev.synchronise()


def moe_expert_forward_gpu(dev: GpuDevice, inp, w_gate, w_up, w_down, intermediate, output,
                           hidden_dim: int, intermediate_dim: int) -> None:
    """ops.rs:621-652: SiLU(gate)*up -> intermediate, then the down projection."""
    L = lib()
    L.launch_moe_expert_silu(_ptr(inp), _ptr(w_gate), _ptr(w_up), _ptr(intermediate), hidden_dim,
                             intermediate_dim, dev.raw_stream())
    check()
    L.launch_moe_expert_down(_ptr(intermediate), _ptr(w_down), _ptr(output), hidden_dim,
                             intermediate_dim, dev.raw_stream())
    check()
    dev.synchronise()


def moe_combine_gpu(dev: GpuDevice, expert_outputs, expert_weights, output, top_k: int) -> None:
    """ops.rs:655-674: hidden_dim = output.numel()."""
    lib().launch_moe_combine(_ptr(expert_outputs), _ptr(expert_weights), _ptr(output),
                             output.numel(), top_k, dev.raw_stream())
    check()
    dev.synchronise()


def mxfp4_dequant_gpu(dev: GpuDevice, packed, scales, output, block_size: int) -> None:
    """ops.rs:677-696: numel = output.numel(); scales are E8M0 bytes, output bf16."""
    lib().launch_mxfp4_dequant(_ptr(packed), _ptr(scales), _ptr(output), output.numel(), block_size,
                               dev.raw_stream())
    check()
    dev.synchronise()


def rms_norm_gpu(dev: GpuDevice, inp, weight, output, eps: float) -> None:
    """ops.rs:366-384: batch = input.rows(), hidden_dim = input.cols()."""
    batch, hidden_dim = _rows_cols(inp)
    lib().launch_rms_norm(_ptr(inp), _ptr(weight), _ptr(output), batch, hidden_dim, float(eps),
                          dev.raw_stream())
    check()
    dev.synchronise()


def residual_add_gpu(dev: GpuDevice, output, residual) -> None:
    """ops.rs:421-435: output += residual over output.numel() elements."""
    lib().launch_residual_add(_ptr(output), _ptr(residual), output.numel(), dev.raw_stream())
    check()
    dev.synchronise()


# ---- extension wrappers ----------------------------------------------------------

def mxfp4_dequant(packed, scales, output, stream: int = 0) -> None:
    rc = lib().physllm_moe_mxfp4_dequant(_ptr(packed), _ptr(scales), _ptr(output), output.numel(), stream)
    check(rc)


def route_topk(x, router_w, router_b, idx, w, top_k: int, stream: int = 0) -> None:
    B, H = x.shape
    E = router_w.shape[0]
    rc = lib().physllm_moe_route_topk(_ptr(x), _ptr(router_w), _ptr(router_b), B, H, E, top_k,
                                      _ptr(idx), _ptr(w), stream)
    check(rc)


def bucket(idx, num_experts: int, counts, offsets, perm, pos, stream: int = 0) -> None:
    B, K = idx.shape
    rc = lib().physllm_moe_bucket(_ptr(idx), B, K, num_experts, _ptr(counts), _ptr(offsets),
                                  _ptr(perm), _ptr(pos), stream)
    check(rc)


def _dev_bits(a: Optional[np.ndarray], device) -> Optional[torch.Tensor]:
    if a is None:
        return None
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


@dataclass
class DeviceMoELayer:
    """A MoE layer's weights resident in device memory plus the ABI structs."""
    cfg: MoEConfig
    tensors: dict
    weights: MoEWeights

    @property
    def hidden(self):
        return self.cfg.hidden

    @property
    def top_k(self):
        return self.cfg.top_k

    @classmethod
    def from_host(cls, layer, device="cuda") -> "DeviceMoELayer":
        names = ("router_w", "router_b", "gate_up_blocks", "gate_up_scales", "gate_up_bias",
                 "down_blocks", "down_scales", "down_bias")
        t = {n: _dev_bits(getattr(layer, n), device) for n in names}
        return cls.from_tensors(layer.hidden, layer.intermediate, layer.num_experts, layer.top_k,
                                t, layer.alpha, layer.limit)

    @classmethod
    def from_tensors(cls, hidden, intermediate, num_experts, top_k, t: dict, alpha=1.702,
                     limit=7.0) -> "DeviceMoELayer":
        cfg = MoEConfig(hidden, intermediate, num_experts, top_k, alpha, limit)
        w = MoEWeights(**{n: (v.data_ptr() if v is not None else None) for n, v in t.items()})
        return cls(cfg, t, w)

    def workspace_bytes(self, batch: int) -> int:
        n = lib().physllm_moe_workspace_bytes(ctypes.byref(self.cfg), batch)
        if n == 0 and batch > 0:
            check(capi.last_error()[0] or capi.PHYSLLM_MOE_EINVAL)
        return int(n)

    def forward(self, x: torch.Tensor, out: torch.Tensor, workspace: torch.Tensor,
                topk_idx: Optional[torch.Tensor] = None, topk_w: Optional[torch.Tensor] = None,
                stream: Optional[int] = None) -> None:
        B = x.shape[0]
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        rc = lib().physllm_moe_layer_forward(ctypes.byref(self.cfg), ctypes.byref(self.weights),
                                             _ptr(x), B, _ptr(out), _ptr(topk_idx), _ptr(topk_w),
                                             _ptr(workspace), workspace.numel() * workspace.element_size(), s)
        check(rc)


    def block_workspace_bytes(self, batch: int) -> int:
        n = lib().physllm_moe_block_workspace_bytes(ctypes.byref(self.cfg), batch)
        if n == 0 and batch > 0:
            check(capi.last_error()[0] or capi.PHYSLLM_MOE_EINVAL)
        return int(n)

    def block_forward(self, x: torch.Tensor, norm_w: torch.Tensor, eps: float, out: torch.Tensor,
                      workspace: torch.Tensor, topk_idx: Optional[torch.Tensor] = None,
                      topk_w: Optional[torch.Tensor] = None, stream: Optional[int] = None) -> None:
        """moe.rs:238-313: out = x + layer(rms_norm(x)); out may be x itself."""
        B = x.shape[0]
        s = torch.cuda.current_stream().cuda_stream if stream is None else stream
        rc = lib().physllm_moe_block_forward(ctypes.byref(self.cfg), ctypes.byref(self.weights), _ptr(x),
                                             _ptr(norm_w), float(eps), B, _ptr(out), _ptr(topk_idx),
                                             _ptr(topk_w), _ptr(workspace),
                                             workspace.numel() * workspace.element_size(), s)
        check(rc)


def moe_block_forward(dlayer: DeviceMoELayer, x: torch.Tensor, norm_w: torch.Tensor, eps: float,
                      return_routing: bool = False):
    """Allocating convenience wrapper of the block: returns out [B,H] (int16 bf16 bits) [, idx, w]."""
    B = x.shape[0]
    out = torch.empty((B, dlayer.hidden), dtype=torch.int16, device=x.device)
    ws = torch.empty(max(dlayer.block_workspace_bytes(B), 1), dtype=torch.uint8, device=x.device)
    idx = torch.empty((B, dlayer.top_k), dtype=torch.int32, device=x.device) if return_routing else None
    w = torch.empty((B, dlayer.top_k), dtype=torch.float32, device=x.device) if return_routing else None
    dlayer.block_forward(x, norm_w, eps, out, ws, idx, w)
    return (out, idx, w) if return_routing else out


def moe_layer_forward(dlayer: DeviceMoELayer, x: torch.Tensor, return_routing: bool = False):
    """Allocating convenience wrapper: returns out [B,H] (int16 bf16 bits) [, idx, w]."""
    B = x.shape[0]
    out = torch.empty((B, dlayer.hidden), dtype=torch.int16, device=x.device)
    ws = torch.empty(max(dlayer.workspace_bytes(B), 1), dtype=torch.uint8, device=x.device)
    idx = torch.empty((B, dlayer.top_k), dtype=torch.int32, device=x.device) if return_routing else None
    w = torch.empty((B, dlayer.top_k), dtype=torch.float32, device=x.device) if return_routing else None
    dlayer.forward(x, out, ws, idx, w)
    return (out, idx, w) if return_routing else out
