"""GPU parity of the steps either side of the MoE layer (crates/llm-core/src/moe.rs:238-313):
RMSNorm before the router, the residual add after the combine, and the fused block
entry point, all through the C ABI against the CPU oracle.

Bars: RMSNorm and the residual add bit-exact for finite inputs (same summation order,
correctly rounded fp32 division and square root); non-finite inputs give NaN/inf at
the same places. The block's routing indices are bit-exact (its normalised activations
are), its output is bit-identical to the separate calls rms_norm -> layer -> residual
add, and within the layer tolerance of the oracle block.
"""
import ctypes
import sys

import numpy as np
import pytest
import torch

from physllm_amd import capi, ops
from physllm_amd import synthetic as syn
from tests import refmath

pytestmark = pytest.mark.gpu

LAYER_TOL = 1e-2


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "gpu tests need a HIP device"
    capi.lib()
    yield
    torch.cuda.synchronize()


def dev(a: np.ndarray, pad: int = 0) -> torch.Tensor:
    """Device copy of a; with pad > 0 the data starts `pad` elements into the buffer."""
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    a = np.ascontiguousarray(a).reshape(-1)
    t = torch.zeros(a.size + pad, dtype=torch.from_numpy(a[:0]).dtype, device="cuda")
    t[pad:] = torch.from_numpy(a).cuda()
    return t


def host(t: torch.Tensor, dtype=None) -> np.ndarray:
    a = t.cpu().numpy()
    return a.view(dtype) if dtype is not None else a


def bits(rng, shape, sigma):
    return syn.bf16_from_f32(rng.standard_normal(shape, dtype=np.float32) * np.float32(sigma))


def _rms_gpu(x, w, eps, pad=0, inplace=False):
    B, H = x.shape
    xt = dev(x, pad)
    wt = dev(w, pad)
    out = xt if inplace else torch.zeros(B * H + pad, dtype=torch.int16, device="cuda")
    capi.lib().launch_rms_norm(xt.data_ptr() + 2 * pad, wt.data_ptr() + 2 * pad, out.data_ptr() + 2 * pad, B, H,
                               float(eps), torch.cuda.current_stream().cuda_stream)
    capi.check()
    torch.cuda.synchronize()
    return host(out, np.uint16)[pad:].reshape(B, H)


@pytest.mark.parametrize("B,H,eps,sigma,pad", [(1, 2880, 1e-5, 1.0, 0), (7, 2880, 1e-6, 3.0, 0),
                                               (64, 2880, 1e-5, 0.05, 0), (3, 300, 0.5, 0.3, 0),
                                               (2, 64, 1e-5, 1.0, 0), (5, 2888, 1e-5, 1.0, 0),
                                               (4, 2880, 1e-5, 1.0, 1), (2, 1, 1e-5, 1.0, 0),
                                               (3, 9000, 1e-5, 1.0, 0), (4096, 2880, 1e-5, 1.0, 0)])
def test_rms_norm_bit_exact(oracle, B, H, eps, sigma, pad):
    """Vector path (H % 8 == 0 and 16-byte aligned pointers, up to H = 9000) and
    element path (H = 300 and H = 1, and pad = 1, which puts every pointer 2 bytes
    off 16-byte alignment)."""
    say(f"rms_norm B={B} H={H} eps={eps} pad={pad}")
    rng = np.random.default_rng(B * 7 + H)
    x = bits(rng, (B, H), sigma)
    w = bits(rng, (H,), 1.0)
    got = _rms_gpu(x, w, eps, pad)
    exp = oracle.rms_norm(x, w, eps)
    bad = np.argwhere(got != exp)
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:4].tolist()}"


def test_rms_norm_in_place_and_order_sensitive_row(oracle):
    say("rms_norm in place + order-sensitive row")
    x, w, i, want_tree, want_serial = refmath.rms_order_sensitive_row(2880, seed=77)
    xb = np.stack([x, x[::-1].copy()])
    exp = oracle.rms_norm(xb, w, 0.0)
    assert exp[0, i] == want_tree != want_serial
    got = _rms_gpu(xb, w, 0.0, inplace=True)
    assert np.array_equal(got, exp)


def test_rms_norm_closed_forms_and_specials(oracle):
    say("rms_norm closed forms + specials")
    H = 2880
    x = np.full((4, H), 0x3FC0, dtype=np.uint16)   # 1.5 -> every output 1.0
    x[1] = 0
    x[1, 17] = 0xC2F6                                # a single -123 in a row of zeros
    x[2, 5] = 0x7FC0                                 # NaN
    x[3, 9] = 0x7F80                                 # +inf -> sum inf -> inf/inf = NaN, finite/inf = 0
    w = np.full(H, 0x3F80, dtype=np.uint16)
    got = _rms_gpu(x, w, 0.0)
    exp = oracle.rms_norm(x, w, 0.0)
    assert np.all(got[0] == 0x3F80)
    fin = (exp & 0x7FFF) <= 0x7F80
    assert np.array_equal(fin, (got & 0x7FFF) <= 0x7F80), "NaN positions differ"
    assert np.array_equal(got[fin], exp[fin])
    # zero-size batch is a no-op
    capi.lib().launch_rms_norm(None, None, None, 0, H, 1e-5, None)
    assert capi.last_error()[0] == 0


@pytest.mark.parametrize("n,pad", [(1, 0), (7, 0), (8, 0), (4097, 0), (2880 * 64, 0), (2880 * 4096 + 3, 0),
                                   (1000, 1)])
def test_residual_add_bit_exact(oracle, n, pad):
    say(f"residual_add n={n} pad={pad}")
    rng = np.random.default_rng(n)
    a = bits(rng, (n,), 1.0)
    b = bits(rng, (n,), 0.05)
    b[: min(n, 50)] = bits(rng, (min(n, 50),), 1e4)
    if n >= 8:
        a[:6] = [0x7F80, 0x8000, 0x0000, 0x7F7F, 0x3F80, 0x3F81]
        b[:6] = [0xFF80, 0x8000, 0x8000, 0x7F7F, 0x3B80, 0x3B80]
    at, bt = dev(a, pad), dev(b, pad)
    dv = ops.GpuDevice()
    capi.lib().launch_residual_add(at.data_ptr() + 2 * pad, bt.data_ptr() + 2 * pad, n, dv.raw_stream())
    capi.check()
    torch.cuda.synchronize()
    got = host(at, np.uint16)[pad:]
    exp = oracle.residual_add(a, b)
    fin = (exp & 0x7FFF) <= 0x7F80
    assert np.array_equal(fin, (got & 0x7FFF) <= 0x7F80)
    assert np.array_equal(got[fin], exp[fin])


def test_legacy_wrappers(oracle):
    """ops.rs:366-384 / :421-435 mirrors: sizes from the tensors, errors raised."""
    say("rms_norm_gpu / residual_add_gpu wrappers")
    rng = np.random.default_rng(3)
    x, w = bits(rng, (5, 2880), 1.0), bits(rng, (2880,), 1.0)
    dv = ops.GpuDevice()
    xt = dev(x).view(5, 2880)
    out = torch.empty_like(xt)
    ops.rms_norm_gpu(dv, xt, dev(w), out, 1e-5)
    assert np.array_equal(host(out, np.uint16), oracle.rms_norm(x, w, 1e-5))
    r = bits(rng, (5, 2880), 1.0)
    ops.residual_add_gpu(dv, out, dev(r).view(5, 2880))
    assert np.array_equal(host(out, np.uint16), oracle.residual_add(oracle.rms_norm(x, w, 1e-5), r))
    with pytest.raises(capi.BackendError):
        ops.rms_norm_gpu(dv, xt, None, out, 1e-5)


# ---- the fused block entry -----------------------------------------------------------

def _block_gpu(layer, x, nw, eps, inplace=False):
    dl = ops.DeviceMoELayer.from_host(layer)
    B = x.shape[0]
    xt = dev(x).view(B, -1)
    out = xt if inplace else torch.empty_like(xt)
    ws = torch.empty(max(dl.block_workspace_bytes(B), 1), dtype=torch.uint8, device="cuda")
    idx = torch.empty((B, layer.top_k), dtype=torch.int32, device="cuda")
    wk = torch.empty((B, layer.top_k), dtype=torch.float32, device="cuda")
    dl.block_forward(xt, dev(nw), eps, out, ws, idx, wk)
    torch.cuda.synchronize()
    return host(out, np.uint16), host(idx), host(wk), dl


def _separate_calls(dl, x, nw, eps):
    """rms_norm -> layer -> residual add as three calls (moe.rs:239-244, :246-307, :310-311)."""
    B, H = x.shape
    dv = ops.GpuDevice()
    xt = dev(x).view(B, H)
    h = torch.empty_like(xt)
    ops.rms_norm_gpu(dv, xt, dev(nw), h, eps)
    m = ops.moe_layer_forward(dl, h)
    ops.residual_add_gpu(dv, m, xt)
    return host(m, np.uint16)


@pytest.mark.parametrize("E,H,I,K,B", [(4, 64, 64, 2, 3), (32, 2880, 2880, 4, 4), (32, 2880, 2880, 4, 6), (8, 256, 128, 3, 20),
                                       (32, 2880, 2880, 4, 1),
                                       (8, 256, 128, 3, 1), (200, 96, 64, 5, 1), (32, 2880, 2880, 4, 2),
                                       (4, 64, 64, 2, 2), (128, 2880, 2880, 4, 2),
                                       (32, 2880, 2880, 4, 64), (4, 256, 128, 2, 512), (128, 256, 128, 4, 2048)])
def test_block_forward(oracle, E, H, I, K, B):
    """Batch 1 and 2 (the norm runs inside the logits launch), 3, 4 and 6 (the residual
    add inside the fused down + combine launch), decode GEMV, grouped GEMM (512 tokens on 4
    experts) and the two-pass router (2048 tokens, 128 experts)."""
    say(f"block E={E} H={H} I={I} K={K} B={B}")
    layer = syn.make_layer(E, H, I, K, seed=E + B)
    x = syn.make_x(B, H, seed=B + 1)
    rng = np.random.default_rng(B)
    nw = bits(rng, (H,), 0.5)
    eps = 1e-5
    got, gidx, gw, dl = _block_gpu(layer, x, nw, eps)
    rows = slice(None) if B <= 64 else np.sort(rng.choice(B, 48, replace=False))
    r = oracle.moe_block(layer, x[rows], nw, eps)
    assert np.array_equal(gidx[rows], r["idx"]), "top-k indices differ"
    assert np.allclose(gw[rows], r["wts"], rtol=1e-6, atol=1e-7)
    err = refmath.rel_l2(refmath.bf16_bits_to_f64(got[rows]), refmath.bf16_bits_to_f64(r["out"]))
    say(f"  rel L2 vs oracle block = {err:.3e}")
    assert err < LAYER_TOL
    assert np.array_equal(got, _separate_calls(dl, x, nw, eps)), "fused block differs from separate calls"
    inplace, _, _, _ = _block_gpu(layer, x, nw, eps, inplace=True)
    assert np.array_equal(inplace, got), "in-place block differs"


def test_block_errors_on_device_path():
    say("block error reporting")
    layer = syn.make_layer(8, 256, 128, 2, seed=1)
    dl = ops.DeviceMoELayer.from_host(layer)
    x = dev(syn.make_x(4, 256, seed=1)).view(4, 256)
    nw = dev(np.full(256, 0x3F80, dtype=np.uint16))
    out = torch.empty_like(x)
    small = torch.empty(dl.workspace_bytes(4), dtype=torch.uint8, device="cuda")   # layer-sized: too small
    with pytest.raises(capi.BackendError) as ei:
        dl.block_forward(x, nw, 1e-5, out, small)
    assert ei.value.code == capi.PHYSLLM_MOE_EWORKSPACE
    ws = torch.empty(dl.block_workspace_bytes(4), dtype=torch.uint8, device="cuda")
    dl.block_forward(x, nw, 1e-5, out, ws)
    torch.cuda.synchronize()
    assert capi.last_error()[0] == 0


@pytest.mark.parametrize("E,H,I,K,B", [(32, 2880, 2880, 4, 1), (32, 2880, 2880, 4, 64), (4, 256, 128, 2, 512),
                                       (8, 256, 256, 4, 1024)])
def test_layer_and_block_replay_in_hip_graph(oracle, E, H, I, K, B):
    """Layer and block captured once in a HIP graph (no host syncs, no memset nodes),
    replayed three times with eager work and synchronisation between replays; every
    replay must equal the eager result. The last shape (4,096 pairs) takes the
    multi-workgroup bucketing and the grouped GEMM."""
    say(f"hip graph replay E={E} B={B}")
    layer = syn.make_layer(E, H, I, K, seed=B + 5)
    x = syn.make_x(B, H, seed=B + 6)
    nw = bits(np.random.default_rng(B), (H,), 0.5)
    dl = ops.DeviceMoELayer.from_host(layer)
    xt, nwt = dev(x).view(B, H), dev(nw)
    out_l, out_b = torch.empty_like(xt), torch.empty_like(xt)
    ws_l = torch.empty(dl.workspace_bytes(B), dtype=torch.uint8, device="cuda")
    ws_b = torch.empty(dl.block_workspace_bytes(B), dtype=torch.uint8, device="cuda")
    dl.forward(xt, out_l, ws_l)
    dl.block_forward(xt, nwt, 1e-5, out_b, ws_b)
    torch.cuda.synchronize()
    ref_l, ref_b = out_l.clone(), out_b.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dl.forward(xt, out_l, ws_l)
        dl.block_forward(xt, nwt, 1e-5, out_b, ws_b)
    other = dev(syn.make_x(B, H, seed=B + 7)).view(B, H)
    for rep in range(3):
        out_l.fill_(0)
        out_b.fill_(0)
        dl.forward(other, torch.empty_like(other), ws_l)     # eager work on the same workspace
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_l, ref_l), f"layer replay {rep} differs"
        assert torch.equal(out_b, ref_b), f"block replay {rep} differs"


@pytest.mark.parametrize("B", [1, 2])
def test_batch1_successive_tokens_and_graph_replays(oracle, B):
    """The batch-1 layer's launches (one or two tokens) hand the logits and the
    selection on through the workspace. Successive calls on one workspace with different
    tokens, and replays of one captured call with the tokens changed in place between
    replays, must each give the result of their own tokens computed on a fresh
    workspace, through the layer and through the block (norm inside the logits launch)."""
    E, H, I, K = 32, 2880, 2880, 4
    layer = syn.make_layer(E, H, I, K, seed=91)
    dl = ops.DeviceMoELayer.from_host(layer)
    nwt = dev(bits(np.random.default_rng(92), (H,), 0.5))
    xs = [syn.make_x(B, H, seed=100 + i) for i in range(4)]
    toks = [dev(x).view(B, H) for x in xs]
    ref_l, ref_b, routes = [], [], []
    for x, t in zip(xs, toks):
        o, idx, _ = ops.moe_layer_forward(dl, t, return_routing=True)
        ref_l.append(o.clone())
        routes.append(tuple(host(idx).reshape(-1).tolist()))
        ob = torch.empty_like(t)
        dl.block_forward(t, nwt, 1e-5, ob, torch.empty(dl.block_workspace_bytes(B), dtype=torch.uint8, device="cuda"))
        ref_b.append(ob)
    torch.cuda.synchronize()
    assert len(set(routes)) > 1, "the tokens should route differently"
    r = oracle.moe_layer(layer, xs[0])
    assert tuple(np.asarray(r["idx"]).reshape(-1).tolist()) == routes[0]

    ws_l = torch.empty(dl.workspace_bytes(B), dtype=torch.uint8, device="cuda")
    ws_b = torch.empty(dl.block_workspace_bytes(B), dtype=torch.uint8, device="cuda")
    for i in [0, 1, 2, 3, 2, 0, 3, 1]:
        ol, ob = torch.empty_like(toks[i]), torch.empty_like(toks[i])
        dl.forward(toks[i], ol, ws_l)
        dl.block_forward(toks[i], nwt, 1e-5, ob, ws_b)
        torch.cuda.synchronize()
        assert torch.equal(ol, ref_l[i]), f"layer call on token {i} differs"
        assert torch.equal(ob, ref_b[i]), f"block call on token {i} differs"

    xt = toks[0].clone()
    out_l, out_b = torch.empty_like(xt), torch.empty_like(xt)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dl.forward(xt, out_l, ws_l)
        dl.block_forward(xt, nwt, 1e-5, out_b, ws_b)
    for i in [1, 2, 3, 0, 2, 2]:
        xt.copy_(toks[i])
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_l, ref_l[i]), f"layer replay on token {i} differs"
        assert torch.equal(out_b, ref_b[i]), f"block replay on token {i} differs"
