"""GPU test of the GPT-OSS checkpoint loader (physllm_amd/host/gpt_oss_loader.hpp):
synthetic MXFP4 checkpoints written by the `safetensors` package in either naming
convention are loaded by tests/cpp/gpt_oss_block, which runs the block
(rms_norm -> layer -> residual add) on the device. The result must be
bit-identical to the same block run through the C ABI on weights uploaded
directly from the arrays the checkpoint was written from (so the loader delivered
the same bytes in the same layout), with top-k identical to the oracle block and
the output within the layer tolerance of it.
"""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from physllm_amd import ops
from physllm_amd import synthetic as syn
from tests import gpt_oss_ckpt, refmath

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "gpt_oss_block")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("naming,blocks_4d,f32,E,H,I,K,B", [
    ("hf", True, False, 8, 256, 128, 2, 5),
    ("orig", False, True, 8, 256, 128, 2, 5),
    ("hf", True, False, 32, 2880, 2880, 4, 3),
])
def test_loaded_layer_runs_the_block(oracle, tmp_path, naming, blocks_4d, f32, E, H, I, K, B):
    assert os.path.exists(BIN), "tests/cpp/gpt_oss_block not built (run __graft_entry__.build())"
    say(f"gpt-oss checkpoint {naming} E={E} H={H} I={I} B={B}")
    layers = [syn.make_layer(E, H, I, K, seed=s) for s in (11, 12)]
    norms = [syn.bf16_from_f32(np.random.default_rng(s).standard_normal(H).astype(np.float32) * 0.5 + 1)
             for s in (13, 14)]
    eps = 1e-5
    d = gpt_oss_ckpt.write_checkpoint(str(tmp_path / "ck"), layers, norms, top_k=K, naming=naming,
                                      blocks_4d=blocks_4d, f32_router=f32, eps=eps)
    x = syn.make_x(B, H, seed=15)
    xp, op = str(tmp_path / "x.bin"), str(tmp_path / "out.bin")
    x.tofile(xp)
    r = subprocess.run([BIN, d, "1", xp, str(B), op], capture_output=True, text=True, timeout=120)
    say(r.stdout.strip())
    assert r.returncode == 0, r.stdout + r.stderr
    raw = np.fromfile(op, dtype=np.uint8)
    out = raw[: B * H * 2].view(np.uint16).reshape(B, H)
    idx = raw[B * H * 2: B * H * 2 + B * K * 4].view(np.int32).reshape(B, K)
    wts = raw[B * H * 2 + B * K * 4:].view(np.float32).reshape(B, K)

    # the same block on weights uploaded straight from the arrays (layer 1)
    dl = ops.DeviceMoELayer.from_host(layers[1])
    xt = torch.from_numpy(x.view(np.int16)).cuda()
    nw = torch.from_numpy(norms[1].view(np.int16)).cuda()
    ref_out, ref_idx, ref_w = ops.moe_block_forward(dl, xt, nw, eps, return_routing=True)
    torch.cuda.synchronize()
    assert np.array_equal(out, ref_out.cpu().numpy().view(np.uint16)), "loaded layer differs from direct upload"
    assert np.array_equal(idx, ref_idx.cpu().numpy())
    assert np.array_equal(wts, ref_w.cpu().numpy())

    e = oracle.moe_block(layers[1], x, norms[1], eps)
    assert np.array_equal(idx, e["idx"])
    err = refmath.rel_l2(refmath.bf16_bits_to_f64(out), refmath.bf16_bits_to_f64(e["out"]))
    say(f"  rel L2 vs oracle block = {err:.3e}")
    assert err < 1e-2


def test_loader_reports_bad_checkpoint(tmp_path):
    assert os.path.exists(BIN)
    layer = syn.make_layer(4, 64, 96, 2, seed=1)
    d = gpt_oss_ckpt.write_checkpoint(str(tmp_path / "ck"), [layer], [syn.make_x(1, 64, seed=2)[0]], top_k=2)
    x = str(tmp_path / "x.bin")
    syn.make_x(1, 64, seed=3).tofile(x)
    r = subprocess.run([BIN, d, "5", x, "1", str(tmp_path / "o.bin")], capture_output=True, text=True, timeout=60)
    assert r.returncode == 3 and "layer 5" in r.stdout
