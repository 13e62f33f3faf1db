"""physllm_moe_layer_forward_noalloc: the layer with the library's own 64 MiB device
array in place of a caller workspace (for callers that cannot allocate). Every call
goes through the C ABI and is compared with physllm_moe_layer_forward on a torch
workspace: the same kernels run, so outputs, indices and routing weights must be
bit-identical, on consecutive calls whose sizes shrink (the array keeps the previous
call's contents)."""
import ctypes

import numpy as np
import pytest
import torch

from physllm_amd import capi, ops
from physllm_amd import synthetic as syn

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def noalloc(dl, x, out, idx, w):
    rc = capi.lib().physllm_moe_layer_forward_noalloc(
        ctypes.byref(dl.cfg), ctypes.byref(dl.weights), x.data_ptr(), x.shape[0], out.data_ptr(),
        idx.data_ptr(), w.data_ptr(), torch.cuda.current_stream().cuda_stream)
    capi.check(rc)


def check_against_workspace_entry(dl, x, label):
    ref = ops.moe_layer_forward(dl, x, return_routing=True)
    B, K = x.shape[0], dl.top_k
    out = torch.full((B, dl.hidden), 0x7fc0, dtype=torch.int16, device="cuda")  # NaN bits
    idx = torch.full((B, K), -7, dtype=torch.int32, device="cuda")
    w = torch.full((B, K), float("nan"), dtype=torch.float32, device="cuda")
    noalloc(dl, x, out, idx, w)
    torch.cuda.synchronize()
    assert torch.equal(out, ref[0]), f"{label}: outputs differ"
    assert torch.equal(idx, ref[1]), f"{label}: indices differ"
    assert torch.equal(w, ref[2]), f"{label}: routing weights differ"
    print(f"{label}: identical", flush=True)


def test_noalloc_equals_workspace_entry_on_shrinking_calls():
    """GPT-OSS-20B shape: decode B = 64 (streaming GEMV), then B = 8, 4, 2 and 1 (smaller
    inputs into the same array; 4 runs the down projection and the combine as one
    launch, 2 and 1 take the three-launch path), then B = 64 again."""
    layer = syn.make_layer(32, 2880, 2880, 4, seed=71)
    dl = ops.DeviceMoELayer.from_host(layer)
    for B, seed in ((64, 1), (8, 2), (4, 6), (2, 5), (1, 3), (64, 4)):
        x = torch.from_numpy(syn.make_x(B, 2880, seed=seed).view(np.int16)).cuda()
        assert dl.workspace_bytes(B) <= SCRATCH_BYTES
        check_against_workspace_entry(dl, x, f"noalloc B={B}")


def test_noalloc_prefill_in_chunks_and_size_limit():
    """A 2048-token prefill needs more than the array at the default chunk size and is
    refused before any launch; with max_chunk_tokens = 512 it runs in 4 grouped-GEMM
    chunks, bit-identical to the workspace entry point under the same limit; then a
    smaller prefill (600 tokens: chunks of 300) into the same array."""
    layer = syn.make_layer(8, 2880, 2880, 4, seed=72)
    dl = ops.DeviceMoELayer.from_host(layer)
    x = torch.from_numpy(syn.make_x(2048, 2880, seed=5).view(np.int16)).cuda()
    assert dl.workspace_bytes(2048) > SCRATCH_BYTES
    out = torch.empty((2048, 2880), dtype=torch.int16, device="cuda")
    idx = torch.empty((2048, 4), dtype=torch.int32, device="cuda")
    w = torch.empty((2048, 4), dtype=torch.float32, device="cuda")
    with pytest.raises(capi.BackendError) as ei:
        noalloc(dl, x, out, idx, w)
    assert ei.value.code == capi.PHYSLLM_MOE_EINVAL and "scratch" in str(ei.value)
    dc = dl.with_chunk_limit(512)
    assert dc.workspace_bytes(2048) <= SCRATCH_BYTES
    check_against_workspace_entry(dc, x, "noalloc prefill 2048 in chunks of 512")
    check_against_workspace_entry(dl.with_chunk_limit(300), x[:600], "noalloc prefill 600 in chunks of 300")


def test_noalloc_under_hip_graph_capture():
    """After one warm-up call on the device (the array's address lookup and the kernels'
    attributes happen on a device's first call, outside any capture), the noalloc layer
    is captured into a HIP graph. Each replay, after new tokens are copied into the
    captured x buffer, equals the workspace entry point's output, indices and weights on
    those tokens, with eager work and synchronisations between the replays."""
    layer = syn.make_layer(32, 2880, 2880, 4, seed=74)
    dl = ops.DeviceMoELayer.from_host(layer)
    B, K = 64, 4
    x = torch.from_numpy(syn.make_x(B, 2880, seed=10).view(np.int16)).cuda()
    out = torch.empty((B, 2880), dtype=torch.int16, device="cuda")
    idx = torch.empty((B, K), dtype=torch.int32, device="cuda")
    w = torch.empty((B, K), dtype=torch.float32, device="cuda")
    noalloc(dl, x, out, idx, w)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        noalloc(dl, x, out, idx, w)
    torch.cuda.synchronize()
    for seed in (11, 12, 13, 11):
        x.copy_(torch.from_numpy(syn.make_x(B, 2880, seed=seed).view(np.int16)).cuda())
        g.replay()
        torch.cuda.synchronize()
        ref = ops.moe_layer_forward(dl, x, return_routing=True)
        torch.cuda.synchronize()
        assert torch.equal(out, ref[0]), f"graph replay (x seed {seed}): outputs differ"
        assert torch.equal(idx, ref[1]), f"graph replay (x seed {seed}): indices differ"
        assert torch.equal(w, ref[2]), f"graph replay (x seed {seed}): routing weights differ"
        print(f"noalloc graph replay, x seed {seed}: identical", flush=True)
