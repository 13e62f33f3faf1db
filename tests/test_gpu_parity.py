"""GPU parity tests: libphysllm_moe.so (HIP, gfx950) against the CPU oracle.

Every call goes through the C ABI; torch only supplies device memory and the
stream. Bars: dequantized values and top-k indices bit-exact; routing weights
within 1e-6 relative (fp64 exp on both sides, rounded to fp32); layer outputs
within 1e-2 relative L2 of the oracle (bf16 storage, fp32 accumulation).
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

LAYER_TOL = 1e-2  # relative L2 of the layer output (benchmark contract)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "gpu tests need a HIP device"
    capi.lib()
    yield
    torch.cuda.synchronize()


def dev(a: np.ndarray) -> torch.Tensor:
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor, dtype=None) -> np.ndarray:
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def stream():
    return torch.cuda.current_stream().cuda_stream


# ---- dequant --------------------------------------------------------------------

def _dequant_gpu(packed, scales, numel, block_size=32, out_offset_elems=0):
    p = dev(packed)
    s = dev(scales)
    out = torch.zeros(numel + out_offset_elems, dtype=torch.int16, device="cuda")
    optr = out.data_ptr() + 2 * out_offset_elems
    capi.lib().launch_mxfp4_dequant(p.data_ptr(), s.data_ptr(), optr, numel, block_size, stream())
    capi.check()
    torch.cuda.synchronize()
    return host(out, np.uint16)[out_offset_elems:]


def test_dequant_kat_every_byte_every_scale(oracle):
    say("dequant KAT 256 bytes x 256 scales")
    kat = refmath.mxfp4_kat()
    packed = np.tile(np.arange(256, dtype=np.uint8), 256)
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16)
    got = _dequant_gpu(packed, scales, packed.size * 2)
    s_of_byte = np.repeat(np.arange(256), 256)
    b = packed.astype(np.int64)
    exp = np.stack([kat[s_of_byte, b & 15], kat[s_of_byte, b >> 4]], axis=1).reshape(-1)
    bad = np.flatnonzero(got != exp)
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:5]}: got {got[bad[:5]]} exp {exp[bad[:5]]}"


@pytest.mark.parametrize("numel,bs,off", [(6, 3, 0), (1001, 32, 0), (4096, 64, 0), (4096, 32, 1), (7, 1, 0)])
def test_dequant_generic_shapes(oracle, numel, bs, off):
    rng = np.random.default_rng(numel + bs)
    packed = rng.integers(0, 256, (numel + 1) // 2, dtype=np.uint8)
    scales = rng.integers(0, 256, -(-numel // bs), dtype=np.uint8)
    got = _dequant_gpu(packed, scales, numel, bs, off)
    exp = oracle.mxfp4_dequant(packed, scales, numel, bs)
    assert np.array_equal(got, exp)


def test_dequant_config1_bit_exact(oracle):
    say("dequant config 1 [32,5760,2880]")
    packed, scales, numel = syn.make_dequant_input()
    p, s = dev(packed), dev(scales)
    out = torch.empty(numel, dtype=torch.int16, device="cuda")
    rc = capi.lib().physllm_moe_mxfp4_dequant(p.data_ptr(), s.data_ptr(), out.data_ptr(), numel, stream())
    capi.check(rc)
    got = host(out, np.uint16)
    exp = oracle.mxfp4_dequant(packed, scales, numel)
    assert np.array_equal(got, exp)


def _dequant_t_gpu(packed, scales, E, rows, cols, bs=32, out_offset_elems=0, codes_offset_bytes=0):
    p = dev(np.concatenate([np.zeros(codes_offset_bytes, np.uint8), packed]))
    s = dev(scales)
    n = E * rows * cols
    out = torch.full((n + out_offset_elems,), 0x5555, dtype=torch.int16, device="cuda")
    optr = out.data_ptr() + 2 * out_offset_elems
    rc = capi.lib().physllm_moe_mxfp4_dequant_transpose(p.data_ptr() + codes_offset_bytes, s.data_ptr(), optr, E,
                                                        rows, cols, bs, stream())
    capi.check(rc)
    torch.cuda.synchronize()
    return host(out, np.uint16)[out_offset_elems:].reshape(E, cols, rows)


# (E, out_dim, in_dim, block_size, output offset in elements): the first five take the
# LDS-tiled kernel (partial tiles in both dimensions among them), the rest the
# per-element one (odd dims, odd block size, rows % 8 != 0, misaligned output).
@pytest.mark.parametrize("E,rows,cols,bs,off", [(3, 200, 352, 32, 0), (2, 128, 128, 32, 0), (1, 8, 32, 32, 0),
                                                (4, 136, 2880, 32, 0), (1, 256, 96, 32, 8),
                                                (2, 7, 45, 32, 0), (2, 3, 5, 3, 0), (1, 12, 64, 32, 0),
                                                (2, 64, 64, 32, 1), (3, 40, 64, 64, 0)])
def test_dequant_transpose_bit_exact(oracle, E, rows, cols, bs, off):
    say(f"dequant transpose E={E} out_dim={rows} in_dim={cols} bs={bs} off={off}")
    rng = np.random.default_rng(E * 7919 + rows * 31 + cols + bs)
    n = E * rows * cols
    packed = rng.integers(0, 256, (n + 1) // 2, dtype=np.uint8)
    scales = rng.integers(0, 256, -(-n // bs), dtype=np.uint8)
    got = _dequant_t_gpu(packed, scales, E, rows, cols, bs, off)
    exp = oracle.mxfp4_dequant_transpose(packed, scales, E, rows, cols, bs)
    bad = np.argwhere(got != exp)
    assert bad.size == 0, f"{len(bad)} mismatches, first [e, in, out] {bad[:4].tolist()}"


def test_dequant_transpose_codes_not_16_byte_aligned(oracle):
    """Codes 4 bytes past a 16-byte boundary take the per-element kernel (the tiled one
    loads whole 16-byte code blocks); the result is the same."""
    rng = np.random.default_rng(404)
    E, rows, cols = 2, 64, 256
    packed = rng.integers(0, 256, E * rows * cols // 2, dtype=np.uint8)
    scales = rng.integers(0, 256, E * rows * cols // 32, dtype=np.uint8)
    got = _dequant_t_gpu(packed, scales, E, rows, cols, 32, 0, 4)
    assert np.array_equal(got, oracle.mxfp4_dequant_transpose(packed, scales, E, rows, cols, 32))


def test_dequant_transpose_config1_equals_flat_transposed():
    """At the [32, 5760, 2880] config-1 tensor: the transposing dequant equals the flat
    dequant (bit-exact against the oracle at this size in the test above) turned around
    on the device, every element."""
    say("dequant transpose config 1 [32,5760,2880] vs flat dequant transposed")
    packed, scales, numel = syn.make_dequant_input()
    E, rows, cols = 32, 5760, 2880
    assert numel == E * rows * cols
    p, s = dev(packed), dev(scales)
    flat = torch.empty(numel, dtype=torch.int16, device="cuda")
    capi.check(capi.lib().physllm_moe_mxfp4_dequant(p.data_ptr(), s.data_ptr(), flat.data_ptr(), numel,
                                                    stream()))
    tr = torch.empty(numel, dtype=torch.int16, device="cuda")
    capi.check(capi.lib().physllm_moe_mxfp4_dequant_transpose(p.data_ptr(), s.data_ptr(), tr.data_ptr(), E, rows,
                                                              cols, 32, stream()))
    exp = flat.view(E, rows, cols).transpose(1, 2).contiguous().view(-1)
    n_bad = int((tr != exp).sum().item())
    assert n_bad == 0, f"{n_bad} mismatches"


# ---- router / bucketing ---------------------------------------------------------------

@pytest.mark.parametrize("B,E,bias", [(1, 32, True), (64, 32, True), (256, 128, True), (4096, 32, True),
                                      (33, 32, False), (5, 1024, True)])
def test_router_bit_exact_indices(oracle, B, E, bias):
    say(f"router B={B} E={E} bias={bias}")
    rng = np.random.default_rng(B * 7 + E)
    H, K = 2880, 4
    x = syn.bf16_from_f32(rng.standard_normal((B, H), dtype=np.float32))
    w = syn.bf16_from_f32(rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02))
    b = syn.bf16_from_f32(rng.standard_normal(E, dtype=np.float32) * np.float32(0.02)) if bias else None
    idx = torch.empty((B, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((B, K), dtype=torch.float32, device="cuda")
    if bias:
        ops.route_topk(dev(x), dev(w), dev(b), idx, wt, K, stream())
    else:
        dv = ops.GpuDevice()
        ops.moe_router_gpu(dv, dev(x), dev(w), idx, wt, E, K)
    torch.cuda.synchronize()
    eidx, ew = oracle.router(x, w, b, K)
    assert np.array_equal(host(idx), eidx)
    assert np.allclose(host(wt), ew, rtol=1e-6, atol=1e-7)


def test_router_ties_and_nan(oracle):
    H, E, K = 64, 8, 4
    x = syn.bf16_from_f32(np.ones((3, H), np.float32))
    w = np.zeros((E, H), np.uint16)
    w[[1, 4, 6]] = syn.bf16_from_f32(np.full(H, 0.5, np.float32))   # three equal maxima
    x[2, 5] = 0x7FC0                                                  # token 2: NaN logits
    idx = torch.empty((3, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((3, K), dtype=torch.float32, device="cuda")
    ops.route_topk(dev(x), dev(w), None, idx, wt, K, stream())
    torch.cuda.synchronize()
    eidx, ew = oracle.router(x, w, None, K)
    assert host(idx)[0].tolist() == [1, 4, 6, 0]
    assert np.array_equal(host(idx), eidx)
    gw = host(wt)
    assert np.allclose(gw[:2], ew[:2], rtol=1e-6)
    assert np.array_equal(np.isnan(gw), np.isnan(ew))


def _router_case(oracle, x, w, b, K):
    B = x.shape[0]
    idx = torch.empty((B, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((B, K), dtype=torch.float32, device="cuda")
    ops.route_topk(dev(x), dev(w), None if b is None else dev(b), idx, wt, K, stream())
    torch.cuda.synchronize()
    eidx, ew = oracle.router(x, w, b, K)
    assert np.array_equal(host(idx), eidx)
    assert np.allclose(host(wt), ew, rtol=1e-6, atol=1e-7, equal_nan=True)
    return host(idx)


@pytest.mark.parametrize("B", [48, 160])
def test_router_near_ties_decided_in_fp64(oracle, B):
    """Experts whose logits differ by one bf16 ulp of one weight (far below the
    fp32 matrix-core error bound of the two-pass router, which B = 160 takes):
    the order comes from the exact fp64 logits. Experts 3 and 7 lead every token;
    10, 11 and 12 compete for the 4th pick."""
    say(f"router near ties B={B}")
    rng = np.random.default_rng(5)
    H, E, K = 2880, 32, 4
    xf = rng.standard_normal((B, H), dtype=np.float32)
    xf[:, 100] = np.abs(xf[:, 100]) + 0.5          # d = 100 has x > 0 for every token
    x = syn.bf16_from_f32(xf)
    w = syn.bf16_from_f32(rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02))
    w[7] = w[3]
    w[7, 100] += 1                                   # +1 ulp (same sign as the value's magnitude step)
    w[11] = w[10]
    w[12] = w[10]
    w[12, 100] -= 1
    bf = np.zeros(E, np.float32)
    bf[[3, 7]] = 16.0                                # logits are ~N(0, 1): gaps of >= 5 sigma
    bf[[10, 11, 12]] = 8.0
    b = syn.bf16_from_f32(bf)
    got = _router_case(oracle, x, w, b, K)
    assert set(got[:, :2].ravel()) <= {3, 7}


@pytest.mark.parametrize("B", [20, 144])
@pytest.mark.parametrize("scale", [2.0 ** 66, 2.0 ** -70])
def test_router_fp32_overflow_and_subnormal_products(oracle, scale, B):
    """Products beyond the fp32 range (x, w ~ 2^66) or below its normal range
    (~2^-140) keep the fp32-product semantics. In the two-pass router (B = 144)
    the matrix-core sums are non-finite or flushed, so every affected expert
    becomes a candidate and the exact pass ranks them."""
    say(f"router fp32 range B={B} scale={scale}")
    rng = np.random.default_rng(6)
    H, E, K = 2880, 32, 4
    x = syn.bf16_from_f32((rng.standard_normal((B, H)) * scale).astype(np.float32))
    w = syn.bf16_from_f32((rng.standard_normal((E, H)) * scale).astype(np.float32))
    _router_case(oracle, x, w, None, K)


@pytest.mark.parametrize("scale", [1.0, 2.0 ** 66, 2.0 ** -70])
def test_route_stage_tiled_two_pass_e128(oracle, scale):
    """Inside the layer (a workspace holds the bounds), E > 64 and B >= 128 route by
    the tiled two-pass router. At scale 1 one token carries a 2^70 activation (its
    matrix-core sums overflow fp32, so all its experts become candidates); at 2^66
    and 2^-70 every product leaves fp32's normal range. The indices equal the
    oracle's and the weights are within 1e-6."""
    say(f"route stage tiled two-pass scale={scale}")
    E, H, I, K, B = 128, 2880, 64, 4, 144
    layer = syn.make_layer(E, H, I, K, seed=77)
    rng = np.random.default_rng(78)
    layer.router_w = syn.bf16_from_f32((rng.standard_normal((E, H)) * scale * 0.05).astype(np.float32))
    x = syn.bf16_from_f32((rng.standard_normal((B, H)) * scale).astype(np.float32))
    if scale == 1.0:
        x[20, 5] = syn.bf16_from_f32(np.array([2.0 ** 70], np.float32))[0]
    dl = ops.DeviceMoELayer.from_host(layer)
    L, s = capi.lib(), stream()
    ws = torch.empty(dl.workspace_bytes(B), dtype=torch.uint8, device="cuda")
    idx = torch.empty((B, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((B, K), dtype=torch.float32, device="cuda")
    assert L.physllm_moe_stage_route(ctypes.byref(dl.cfg), ctypes.byref(dl.weights), dev(x).data_ptr(), B,
                                     idx.data_ptr(), wts.data_ptr(), ws.data_ptr(), ws.numel(), s) == 0
    torch.cuda.synchronize()
    eidx, ew = oracle.router(x, layer.router_w, layer.router_b, K)
    assert np.array_equal(host(idx), eidx)
    assert np.allclose(host(wts), ew, rtol=1e-6, atol=1e-7, equal_nan=True)


@pytest.mark.parametrize("E,H,K", [(8, 64, 4), (40, 2880, 4), (128, 2880, 8), (17, 96, 1), (128, 3072, 4)])
def test_router_two_pass_ties_nan_and_shapes(oracle, E, H, K):
    """The two-pass router (B >= 128) on expert counts that are not multiples of
    16, short and maximal rows, k = 1 and 8: random logits, experts with identical
    rows (exact ties: the lower index wins), tokens with a NaN activation (NaN
    logits rank last) and tokens whose logits are all equal."""
    say(f"router two-pass E={E} H={H} K={K}")
    rng = np.random.default_rng(E * 31 + H + K)
    B = 137 if E <= 64 else 2048        # above 64 experts the two-pass router needs B * E >= 2^18
    x = syn.bf16_from_f32(rng.standard_normal((B, H), dtype=np.float32))
    w = syn.bf16_from_f32(rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.05))
    w[E - 1] = w[0]                      # tie between the first and last expert
    if E > 4:
        w[3] = w[2]
    x[5, 7] = 0x7FC0                     # NaN activation
    x[9] = 0                             # all logits equal (zero, no bias)
    b = None if E % 2 else syn.bf16_from_f32(rng.standard_normal(E, dtype=np.float32) * np.float32(0.05))
    if b is not None:
        b[E - 1] = b[0]
        if E > 4:
            b[3] = b[2]
    _router_case(oracle, x, w, b, K)


@pytest.mark.parametrize("B,K,E,skew", [(1, 4, 32, False), (64, 4, 32, True), (4096, 4, 32, False),
                                        (256, 4, 128, False), (3000, 1, 3, True), (200, 4, 256, True),
                                        (100, 2, 200, False), (30, 3, 65, True)])
def test_bucket_matches_oracle(oracle, B, K, E, skew):
    rng = np.random.default_rng(B + K + E)
    if skew:
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        idx = np.stack([rng.choice(E, K, replace=False, p=p / p.sum()) for _ in range(B)]).astype(np.int32)
    else:
        idx = np.stack([rng.permutation(E)[:K] for _ in range(B)]).astype(np.int32)
    N = B * K
    c = torch.empty(E, dtype=torch.int32, device="cuda")
    o = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    pm = torch.empty(N, dtype=torch.int32, device="cuda")
    ps = torch.empty(N, dtype=torch.int32, device="cuda")
    ops.bucket(dev(idx), E, c, o, pm, ps, stream())
    torch.cuda.synchronize()
    ec, eo, ep, eps = oracle.bucket(idx, E)
    assert np.array_equal(host(c), ec) and np.array_equal(host(o), eo)
    assert np.array_equal(host(pm), ep) and np.array_equal(host(ps), eps)


# ---- whole layer ------------------------------------------------------------------

def _run_layer(layer, x, return_routing=True):
    dl = ops.DeviceMoELayer.from_host(layer)
    out, idx, w = ops.moe_layer_forward(dl, dev(x), return_routing=True)
    torch.cuda.synchronize()
    return host(out, np.uint16), host(idx), host(w), dl


def _check_layer(oracle, layer, x, label, rows=None):
    got, gidx, gw, _ = _run_layer(layer, x)
    xs = x if rows is None else x[rows]
    r = oracle.moe_layer(layer, xs)
    if rows is not None:
        got, gidx, gw = got[rows], gidx[rows], gw[rows]
    assert np.array_equal(gidx, r["idx"]), f"{label}: top-k indices differ"
    assert np.allclose(gw, r["wts"], rtol=1e-6, atol=1e-7), f"{label}: routing weights differ"
    err = refmath.rel_l2(refmath.bf16_bits_to_f64(got), refmath.bf16_bits_to_f64(r["out"]))
    say(f"{label}: rel L2 = {err:.3e}")
    assert err < LAYER_TOL, f"{label}: rel L2 {err}"
    return err


def test_layer_tiny_against_oracle_and_float64(oracle):
    layer = syn.make_layer(4, 64, 64, 2, seed=3)
    x = syn.make_x(3, 64, seed=11)
    _check_layer(oracle, layer, x, "tiny E=4 H=I=64")
    got, _, _, _ = _run_layer(layer, x)
    ref, _, _ = refmath.moe_layer_f64(layer, x)
    assert refmath.rel_l2(refmath.bf16_bits_to_f64(got), ref) < 4e-3


@pytest.mark.parametrize("E,H,I,K,zipf,bias", [(32, 2880, 2880, 4, 1.1, True), (8, 256, 128, 3, None, True),
                                               (64, 2880, 2880, 1, None, True), (16, 512, 1024, 4, None, False),
                                               (128, 2880, 2880, 4, None, True), (256, 256, 128, 4, None, True)])
def test_layer_two_tokens(oracle, E, H, I, K, zipf, bias):
    """Two decode tokens take the three-launch batch-1 layer (selection inside the
    gate_up launch, one tile per distinct expert with a column per token, down waves
    per routed pair, combine per token): indices bit-exact, layer within tolerance."""
    layer = syn.make_layer(E, H, I, K, seed=E + K, zipf=zipf, with_bias=bias)
    x = syn.make_x(2, H, seed=E + 2)
    _check_layer(oracle, layer, x, f"two tokens E={E} H={H} I={I} K={K}")


def test_layer_two_tokens_equals_stage_entry_points():
    """At the GPT-OSS-20B shape (where the per-stage down projection does not split K)
    the two-token layer gives the bits of the four stage entry points run one by one."""
    layer = syn.make_layer(32, 2880, 2880, 4, seed=1002, zipf=1.1)
    x = syn.make_x(2, 2880, seed=5)
    got, _, _, dl = _run_layer(layer, x)
    L = capi.lib()
    B, xd = 2, dev(x)
    ws = torch.zeros(dl.workspace_bytes(B), dtype=torch.uint8, device="cuda")
    out = torch.empty((B, 2880), dtype=torch.int16, device="cuda")
    cfg, w, n, s = ctypes.byref(dl.cfg), ctypes.byref(dl.weights), ws.numel(), None
    # routing into the workspace, where the combine stage reads its weights
    capi.check(L.physllm_moe_stage_route(cfg, w, xd.data_ptr(), B, None, None, ws.data_ptr(), n, s))
    capi.check(L.physllm_moe_stage_gate_up(cfg, w, xd.data_ptr(), B, ws.data_ptr(), n, s))
    capi.check(L.physllm_moe_stage_down(cfg, w, B, ws.data_ptr(), n, s))
    capi.check(L.physllm_moe_stage_combine(cfg, B, out.data_ptr(), None, ws.data_ptr(), n, s))
    torch.cuda.synchronize()
    assert np.array_equal(host(out, np.uint16), got), "two-token layer differs from the stage entry points"


@pytest.mark.parametrize("E,H,I,K,B", [(8, 256, 128, 3, 20), (16, 512, 1024, 4, 40), (3, 96, 160, 1, 37),
                                       (8, 256, 4096, 2, 1), (8, 128, 3200, 2, 3), (5, 160, 4096, 3, 3),
                                       (8, 160, 4096, 3, 8)])
def test_layer_odd_shapes(oracle, E, H, I, K, B):
    """Includes down projections whose reduction (I = 4096, 3200) is split over
    several K ranges at small batch: 128 and 100 scale blocks per row; and with H = 160
    rows, a last 64-row group in which only two of the four waves have a tile (the other
    two still stage their share of the activations)."""
    layer = syn.make_layer(E, H, I, K, seed=E + B)
    x = syn.make_x(B, H, seed=B)
    _check_layer(oracle, layer, x, f"E={E} H={H} I={I} K={K} B={B}")


@pytest.mark.parametrize("E,H,I,K,B", [(4, 256, 128, 2, 512), (3, 224, 96, 1, 300), (8, 2880, 2880, 4, 1024),
                                       (2, 160, 160, 2, 700)])
def test_layer_grouped_gemm_path(oracle, E, H, I, K, B):
    """Shapes with >= 64 routed tokens per touched expert take the grouped-GEMM
    (prefill) kernels: partial 128-row tiles (R = 192, 160), partial 128-token
    tiles, and K ranges that end inside a 128-element step (H = 224, 160)."""
    layer = syn.make_layer(E, H, I, K, seed=E * 100 + B)
    x = syn.make_x(B, H, seed=B)
    _check_layer(oracle, layer, x, f"gemm E={E} H={H} I={I} K={K} B={B}")


@pytest.mark.parametrize("E,H,I,K,B,bias", [(16, 2880, 1440, 4, 2048, True), (6, 352, 416, 2, 900, False),
                                            (5, 4096, 320, 3, 700, True)])
def test_layer_lds_staged_gemm(oracle, E, H, I, K, B, bias):
    """The LDS-staged grouped GEMM (384-row gate_up and 320-row down tiles, both operands,
    the tile's scale block and biases copied into LDS): row counts that end inside a tile
    (2I = 2880, 832, 640; H = 352), odd and non-multiple-of-4 block counts (K = 1440, 416, 320:
    45, 13, 10 blocks), several tiles per workgroup (the next tile's pair ids and first step
    copied during the current one), no biases, and K = 4096 (128 blocks: the older 128-row
    kernel)."""
    layer = syn.make_layer(E, H, I, K, seed=E * 7 + B, with_bias=bias)
    x = syn.make_x(B, H, seed=B + 1)
    _check_layer(oracle, layer, x, f"lds gemm E={E} H={H} I={I} K={K} B={B} bias={bias}")


@pytest.mark.parametrize("E,H,I,K,B", [(128, 256, 256, 4, 600), (1000, 64, 64, 2, 700), (32, 128, 96, 4, 5000)])
def test_layer_bucketing_many_blocks(oracle, E, H, I, K, B):
    """More than 1024 routed pairs are bucketed by many workgroups (block counts, one scan
    that writes the tables, one scatter per block): decode-path shapes whose pass table
    comes from the scan (E = 128; E = 1000, one scan thread per expert) and a
    20,000-pair prefill (20 blocks of 1024 pairs)."""
    layer = syn.make_layer(E, H, I, K, seed=E + 3 * B)
    x = syn.make_x(B, H, seed=B + 7)
    _check_layer(oracle, layer, x, f"bucket blocks E={E} H={H} I={I} K={K} B={B}")


def test_layer_gemm_unaligned_scales_fall_back(oracle):
    """Scale and bias arrays that are not 16-byte aligned cannot be copied in 16-byte units:
    the layer takes the register-staged GEMM instead, with the same results."""
    layer = syn.make_layer(8, 2880, 2880, 4, seed=77)
    x = syn.make_x(1024, 2880, seed=77)
    dl = ops.DeviceMoELayer.from_host(layer)
    t = dict(dl.tensors)
    keep = []
    for name in ("gate_up_scales", "down_scales", "gate_up_bias", "down_bias"):
        v = t[name]
        # the same bytes one element further into a larger buffer: 1 (scales) or 2 (bias) bytes off
        big = torch.empty(v.numel() + 16, dtype=v.dtype, device="cuda")
        big[1:1 + v.numel()] = v.reshape(-1)
        keep.append(big)
        t[name] = big[1:1 + v.numel()].view(v.shape)
    du = ops.DeviceMoELayer.from_tensors(layer.hidden, layer.intermediate, layer.num_experts, layer.top_k, t,
                                         layer.alpha, layer.limit)
    assert du.tensors["gate_up_scales"].data_ptr() % 16 == 1
    xd = dev(x)
    got = ops.moe_layer_forward(du, xd, return_routing=True)
    ref = ops.moe_layer_forward(dl, xd, return_routing=True)
    torch.cuda.synchronize()
    assert torch.equal(got[1], ref[1])
    r = oracle.moe_layer(layer, x[:256])
    err = refmath.rel_l2(refmath.bf16_bits_to_f64(host(got[0], np.uint16)[:256]),
                         refmath.bf16_bits_to_f64(r["out"]))
    say(f"unaligned scales (fallback GEMM): rel L2 = {err:.3e}")
    assert err < LAYER_TOL


@pytest.mark.parametrize("E,H,I,K,B,hot,bias", [(128, 288, 352, 4, 100, None, True),
                                                (128, 288, 352, 4, 100, 3, True),
                                                (128, 288, 352, 4, 100, None, False),
                                                (64, 2880, 2880, 4, 16, None, True)])
def test_layer_streaming_gemv(oracle, E, H, I, K, B, hot, bias):
    """Decode batches touching many experts (>= 2 work items per CU) take the
    persistent streaming GEMV: K ranges ending inside a 4-block step (9 and 11
    blocks), weight rows not a multiple of 128 (704, 288), an expert holding every
    token (100 tokens: 7 pass-table entries, restaged activations), no biases."""
    layer = syn.make_layer(E, H, I, K, seed=E + H + B, with_bias=bias)
    if hot is not None:
        rb = syn.bf16_to_f32(layer.router_b).copy()
        rb[hot] = 50.0
        layer.router_b = syn.bf16_from_f32(rb)
    x = syn.make_x(B, H, seed=B + 1)
    _check_layer(oracle, layer, x, f"stream E={E} H={H} I={I} K={K} B={B} hot={hot} bias={bias}")


@pytest.mark.parametrize("E,H,I,K,bias", [(32, 2880, 2880, 4, True), (256, 256, 128, 8, True),
                                          (128, 4096, 256, 4, True), (4, 64, 64, 4, True), (7, 96, 64, 1, True),
                                          (300, 64, 96, 3, True), (32, 2880, 2880, 4, False),
                                          (16, 160, 2944, 2, True)])
def test_layer_batch1_fused_route(oracle, E, H, I, K, bias):
    """Batch 1 routes in one launch (router, top-k, softmax and the bucketing of the
    token's k pairs): E up to the 256 limit, k = E, k = 1, a hidden size needing
    two passes of the row loads (4096). With k <= 4 the down projection and the
    combine run as one launch (k_mx_down1), here also after the general router and
    bucketing (E = 300), without biases, and at the 92-block K limit (I = 2944)."""
    layer = syn.make_layer(E, H, I, K, seed=E * 3 + K, with_bias=bias)
    x = syn.make_x(1, H, seed=E + H)
    _check_layer(oracle, layer, x, f"batch-1 route E={E} H={H} I={I} K={K}")


def test_layer_batch1_route_ties_and_nan(oracle):
    """Batch-1 route with three equal leading logits (ties go to the lower index)
    and with a NaN activation (every logit NaN: NaN ranks lowest, so the first k
    experts by index, as the oracle selects)."""
    E, H, I, K = 16, 128, 64, 4
    layer = syn.make_layer(E, H, I, K, seed=21)
    rw = layer.router_w.copy()
    rw[[9, 2, 5]] = rw[2]
    rb = syn.bf16_to_f32(layer.router_b).copy()
    rb[[2, 5, 9]] = 20.0
    layer.router_w, layer.router_b = rw, syn.bf16_from_f32(rb)
    x = syn.make_x(1, H, seed=21)
    got, gidx, _, _ = _run_layer(layer, x)
    assert gidx[0, :3].tolist() == [2, 5, 9]
    _check_layer(oracle, layer, x, "batch-1 ties")
    xn = x.copy()
    xn[0, 7] = 0x7FC0
    _, nidx, nw, _ = _run_layer(layer, xn)
    r = oracle.moe_layer(layer, xn)
    assert np.array_equal(nidx, r["idx"]) and nidx[0].tolist() == [0, 1, 2, 3]
    assert np.array_equal(np.isnan(nw), np.isnan(r["wts"]))


@pytest.mark.parametrize("E,H,I,K,B", [(32, 2880, 2880, 4, 64), (32, 2880, 256, 4, 128), (64, 256, 128, 8, 64),
                                       (8, 96, 64, 2, 2), (16, 128, 96, 1, 37), (64, 64, 64, 4, 17)])
def test_layer_decode_route_small(oracle, E, H, I, K, B):
    """Decode batches with E <= 64 and B * E <= 4096 route in two launches: the logits
    over many waves, then one workgroup selects every token's top k (ranks among its
    token's logits), takes the softmax and buckets the pairs. The layer's indices and
    weights equal the general router's (physllm_moe_route_topk) bit for bit, with tied
    router rows and a token whose logits are all NaN, and the output matches the oracle
    on the other tokens. (B = 2 with B * k <= 16 takes the batch-1 launches instead, whose
    selection runs inside the gate_up launch: the same indices and weights.)"""
    layer = syn.make_layer(E, H, I, K, seed=E + 7 * B)
    rw = layer.router_w.copy()
    rw[[3, 5]] = rw[1]  # three experts with equal logits for every token
    layer.router_w = rw
    x = syn.make_x(B, H, seed=B + H)
    x[1, 5] = 0x7FC0  # token 1: every logit NaN
    got, gidx, gw, _ = _run_layer(layer, x)
    idx = torch.empty((B, K), dtype=torch.int32, device="cuda")
    wt = torch.empty((B, K), dtype=torch.float32, device="cuda")
    ops.route_topk(dev(x), dev(layer.router_w), dev(layer.router_b), idx, wt, K, stream())
    torch.cuda.synchronize()
    assert np.array_equal(gidx, host(idx))
    assert np.array_equal(gw.view(np.uint32), host(wt).view(np.uint32))
    assert gidx[1].tolist() == list(range(K))
    rows = [r for r in range(B) if r != 1]
    _check_layer(oracle, layer, x, f"decode route E={E} H={H} I={I} K={K} B={B}", rows=rows)


def _run_stages(dl, xd, B):
    """The layer through the per-stage entry points (route, gate_up, down, combine)."""
    L, s = capi.lib(), stream()
    ws = torch.empty(dl.workspace_bytes(B), dtype=torch.uint8, device="cuda")
    n = ws.numel()
    cfg, w = ctypes.byref(dl.cfg), ctypes.byref(dl.weights)
    K = dl.cfg.top_k
    idx = torch.empty((B, K), dtype=torch.int32, device="cuda")
    wts = torch.empty((B, K), dtype=torch.float32, device="cuda")
    out = torch.empty((B, dl.cfg.hidden), dtype=torch.int16, device="cuda")
    assert L.physllm_moe_stage_route(cfg, w, xd.data_ptr(), B, idx.data_ptr(), wts.data_ptr(), ws.data_ptr(), n, s) == 0
    assert L.physllm_moe_stage_gate_up(cfg, w, xd.data_ptr(), B, ws.data_ptr(), n, s) == 0
    assert L.physllm_moe_stage_down(cfg, w, B, ws.data_ptr(), n, s) == 0
    assert L.physllm_moe_stage_combine(cfg, B, out.data_ptr(), wts.data_ptr(), ws.data_ptr(), n, s) == 0
    torch.cuda.synchronize()
    return host(out, np.uint16), host(idx), host(wts)


@pytest.mark.parametrize("E,H,I,K,bias", [(32, 2880, 2880, 4, True), (32, 2880, 2880, 4, False),
                                          (8, 2048, 512, 4, True), (128, 2944, 2944, 3, True),
                                          (16, 2560, 1280, 4, True)])
def test_layer_batch1_three_launches_equal_stages(oracle, E, H, I, K, bias):
    """Batch 1 runs as three launches: the router logits (one workgroup per expert),
    selection + gate_up, then down + combine. Its output, indices and weights equal the
    per-stage entry points' (one-launch route, gate_up GEMV, down GEMV, combine) bit for
    bit, on shapes where the stage path's down projection is not split over K (at least
    512 16-row tiles), repeated calls give the same bits, and the output matches the
    oracle."""
    layer = syn.make_layer(E, H, I, K, seed=E * 5 + H, with_bias=bias)
    x = syn.make_x(1, H, seed=H + I)
    got, gidx, gw, dl = _run_layer(layer, x)
    sout, sidx, sw = _run_stages(dl, dev(x), 1)
    assert np.array_equal(gidx, sidx) and np.array_equal(gw.view(np.uint32), sw.view(np.uint32))
    assert np.array_equal(got, sout), "three-launch batch-1 layer differs from the per-stage path"
    for _ in range(3):
        again, _, _ = ops.moe_layer_forward(dl, dev(x), return_routing=True)
        assert np.array_equal(host(again, np.uint16), got)
    _check_layer(oracle, layer, x, f"batch-1 three launches E={E} H={H} I={I} K={K}")


@pytest.mark.parametrize("B", [1, 2])
def test_stage_batch1_launches_equal_layer(B):
    """physllm_moe_stage_batch1 runs the batch-1 layer's launches one at a time: 0
    (logits), 1 (selection + gate_up), 2 (down + combine) in order give the layer
    call's output bit for bit, and launch 1 repeated on the same workspace state gives
    the same bits again (what the bench relies on when it times it alone). A batch the
    batch-1 launches do not serve is EINVAL, and so is a launch number past 2."""
    layer = syn.make_layer(32, 2880, 2880, 4, seed=77 + B)
    x = syn.make_x(B, 2880, seed=78 + B)
    got, _, _, dl = _run_layer(layer, x)
    L, s = capi.lib(), stream()
    xd = dev(x)
    ws = torch.empty(dl.workspace_bytes(B), dtype=torch.uint8, device="cuda")
    out = torch.empty((B, 2880), dtype=torch.int16, device="cuda")
    cfg, w = ctypes.byref(dl.cfg), ctypes.byref(dl.weights)
    for launch in (0, 1, 1, 2):
        assert L.physllm_moe_stage_batch1(cfg, w, xd.data_ptr(), B, launch, out.data_ptr(), ws.data_ptr(),
                                          ws.numel(), s) == 0, capi.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(host(out, np.uint16), got), "batch-1 stage launches differ from the layer call"
    assert L.physllm_moe_stage_batch1(cfg, w, xd.data_ptr(), B, 3, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                      s) == capi.PHYSLLM_MOE_EINVAL
    x5 = dev(syn.make_x(5, 2880, seed=79))
    ws5 = torch.empty(dl.workspace_bytes(5), dtype=torch.uint8, device="cuda")
    out5 = torch.empty((5, 2880), dtype=torch.int16, device="cuda")
    assert L.physllm_moe_stage_batch1(cfg, w, x5.data_ptr(), 5, 0, out5.data_ptr(), ws5.data_ptr(), ws5.numel(),
                                      s) == capi.PHYSLLM_MOE_EINVAL


@pytest.mark.parametrize("E,H,K,B", [(128, 256, 4, 100), (128, 2880, 4, 256), (300, 96, 8, 40), (96, 224, 2, 100),
                                     (64, 256, 4, 100), (32, 2880, 4, 64), (40, 96, 1, 17), (8, 128, 8, 127),
                                     (100, 96, 4, 300), (128, 3072, 8, 130), (65, 64, 2, 129)])
def test_layer_two_launch_router(oracle, E, H, K, B):
    """Mid-size batches (B * E >= 8192 outside the two-pass range) route in two
    launches (logits of 8 tokens x 16 experts per workgroup, then one selection
    workgroup per token); the smaller ones here take k_router. Indices bit-exact and
    weights as the oracle's, with ties to the lower index, a NaN token, more than 256
    experts (arg-max rounds), k = 1 and k = E. Batches of 128 or more with 64 < E <= 128
    take the tiled two-pass router (bounds per 16 x 16 tile, then one 4-wave selection
    workgroup per token; the NaN token makes every expert a candidate, spread over its
    four waves), including expert counts that are not multiples of 16."""
    layer = syn.make_layer(E, H, 64, K, seed=E + B)
    tie = [2, 5, 9] if E > 9 else [1, 3, 5]
    rw = layer.router_w.copy()
    rw[tie] = rw[tie[0]]
    rb = syn.bf16_to_f32(layer.router_b).copy()
    rb[tie] = 20.0
    layer.router_w, layer.router_b = rw, syn.bf16_from_f32(rb)
    x = syn.make_x(B, H, seed=B)
    x[3, 7] = 0x7FC0
    got, gidx, gw, _ = _run_layer(layer, x)
    eidx, ew = oracle.router(x, layer.router_w, layer.router_b, K)
    assert np.array_equal(gidx, eidx)
    fin = ~np.isnan(ew)
    assert np.array_equal(np.isnan(gw), ~fin)
    assert np.allclose(gw[fin], ew[fin], rtol=1e-6, atol=1e-7)
    assert gidx[0, :min(3, K)].tolist() == tie[:min(3, K)]


def test_layer_without_biases(oracle):
    layer = syn.make_layer(8, 128, 64, 2, seed=4, with_bias=False)
    x = syn.make_x(9, 128, seed=4)
    _check_layer(oracle, layer, x, "no biases")


def test_layer_all_tokens_one_expert(oracle):
    """Every token picks expert 5 first (huge router bias): a 40-token bucket plus
    experts with no tokens at all."""
    layer = syn.make_layer(8, 128, 64, 2, seed=8)
    rb = syn.bf16_to_f32(layer.router_b).copy()
    rb[5] = 50.0
    layer.router_b = syn.bf16_from_f32(rb)
    x = syn.make_x(40, 128, seed=8)
    got, gidx, _, _ = _run_layer(layer, x)
    assert np.all(gidx[:, 0] == 5)
    _check_layer(oracle, layer, x, "all tokens -> expert 5")


@pytest.mark.parametrize("B", [2, 4])
def test_layer_nan_activation_propagates(oracle, B):
    """A NaN activation makes its token's logits and output NaN, as in the oracle; the
    other tokens are unaffected (B = 2: the batch-1 launches, B = 4: the per-stage path)."""
    layer = syn.make_layer(4, 64, 64, 2, seed=12)
    x = syn.make_x(B, 64, seed=12)
    x[1, 7] = 0x7FC0
    got, gidx, _, _ = _run_layer(layer, x)
    r = oracle.moe_layer(layer, x)
    assert np.array_equal(gidx, r["idx"])
    gf, ef = refmath.bf16_bits_to_f64(got), refmath.bf16_bits_to_f64(r["out"])
    assert np.array_equal(np.isnan(gf), np.isnan(ef))
    ok = ~np.isnan(ef)
    assert refmath.rel_l2(gf[ok], ef[ok]) < LAYER_TOL


def _random_shapes(seed, n):
    """Seeded layer shapes over every kernel path: E in 1..300, H and I any multiple of
    32 up to 4096, k up to 8, decode and prefill batches, with and without biases."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        E = int(rng.choice([1, 2, 3, 5, 8, 16, 32, 33, 64, 128, 300]))
        H = int(rng.integers(1, 129)) * 32
        I = int(rng.integers(1, 129)) * 32
        K = int(rng.integers(1, min(E, 8) + 1))
        B = int(rng.choice([1, 2, 3, 5, 8, 17, 33, 64, 100, 257, 700]))
        while B * K * H * I > 3e9 and B > 1:
            B //= 2
        out.append((E, H, I, K, B, bool(rng.integers(0, 2)), 1000 + i))
    return out


@pytest.mark.parametrize("E,H,I,K,B,bias,seed", _random_shapes(1, 40))
def test_layer_random_shapes(oracle, E, H, I, K, B, bias, seed):
    """Forty seeded shapes against the oracle (indices bit-exact, output within the layer
    tolerance). Shapes like these found a last 64-row group whose idle waves skipped
    their share of the activation staging."""
    layer = syn.make_layer(E, H, I, K, seed=seed, with_bias=bias)
    x = syn.make_x(B, H, seed=seed + 1000)
    _check_layer(oracle, layer, x, f"random E={E} H={H} I={I} K={K} B={B} bias={bias}")


def test_layer_deterministic(oracle):
    layer = syn.make_layer(32, 2880, 2880, 4, seed=21)
    x = syn.make_x(16, 2880, seed=21)
    dl = ops.DeviceMoELayer.from_host(layer)
    xd = dev(x)
    a = ops.moe_layer_forward(dl, xd)
    b = ops.moe_layer_forward(dl, xd)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("cfg", [0, 2, 4])
def test_layer_benchmark_configs(oracle, cfg):
    say(f"layer config {cfg}: {syn.CONFIGS[cfg]['workload']}")
    layer, x = syn.make_config(cfg)
    _check_layer(oracle, layer, x, f"config {cfg}")


@pytest.fixture(scope="module")
def config3():
    return syn.make_config(3)


def test_layer_prefill_config3(oracle, config3):
    """4096-token prefill: indices, routing weights and all 4096 output rows against the
    oracle (every expert's partial last token tile and every tile range of the persistent
    GEMM schedule included)."""
    say("layer config 3 (prefill 4096), full oracle check")
    layer, x = config3
    _check_layer(oracle, layer, x, "config 3")


@pytest.mark.parametrize("limit", [1024, 1000])
def test_layer_chunked_equals_unchunked_config3(config3, limit):
    """A batch above the chunk limit runs as consecutive whole-layer chunks over one
    workspace. Routing is per token and each output element's sums have a fixed order, so
    when every chunk takes the grouped GEMM (>= 64 routed pairs per touched expert: 1024
    gives 4 chunks of 1024 tokens, 1000 gives 5 of 820 and 819) the outputs, indices and
    weights are bit-identical to the single call's; so is the block (norm + layer +
    residual add per chunk)."""
    say(f"config 3 chunked at {limit} tokens")
    layer, x = config3
    dl = ops.DeviceMoELayer.from_host(layer)
    dc = dl.with_chunk_limit(limit)
    assert dc.workspace_bytes(x.shape[0]) < dl.workspace_bytes(x.shape[0])
    xd = dev(x)
    ref = ops.moe_layer_forward(dl, xd, return_routing=True)
    got = ops.moe_layer_forward(dc, xd, return_routing=True)
    torch.cuda.synchronize()
    for a, b in zip(ref, got):
        assert torch.equal(a, b)
    nw = dev(syn.bf16_from_f32(np.random.default_rng(5).uniform(0.5, 1.5, layer.hidden).astype(np.float32)))
    rb = ops.moe_block_forward(dl, xd, nw, 1e-5, return_routing=True)
    gb = ops.moe_block_forward(dc, xd, nw, 1e-5, return_routing=True)
    torch.cuda.synchronize()
    for a, b in zip(rb, gb):
        assert torch.equal(a, b)


def test_layer_chunked_decode_against_oracle(oracle):
    """Decode chunks (64 tokens at a limit of 24: chunks of 22, 21, 21) may take other
    GEMV forms and K splits than the single call, so they are held to the oracle: identical
    indices and rel L2 < 1e-2."""
    layer, x = syn.make_config(2)
    dc = ops.DeviceMoELayer.from_host(layer, max_chunk_tokens=24)
    out, idx, w = ops.moe_layer_forward(dc, dev(x), return_routing=True)
    torch.cuda.synchronize()
    r = oracle.moe_layer(layer, x)
    assert np.array_equal(host(idx), r["idx"])
    assert np.allclose(host(w), r["wts"], rtol=1e-6, atol=1e-7)
    err = refmath.rel_l2(refmath.bf16_bits_to_f64(host(out, np.uint16)), refmath.bf16_bits_to_f64(r["out"]))
    say(f"config 2 in chunks of <= 24: rel L2 = {err:.3e}")
    assert err < LAYER_TOL


@pytest.mark.parametrize("E,H,I,K,B,bias", [(32, 2880, 2880, 4, 3, True), (32, 2880, 2880, 4, 4, False),
                                            (128, 2944, 2944, 4, 4, True), (8, 2048, 512, 2, 5, True),
                                            (16, 2560, 1280, 1, 16, True), (32, 2880, 2880, 4, 5, False),
                                            (32, 2880, 2880, 4, 6, True), (128, 2944, 2944, 4, 6, True),
                                            (64, 2048, 2048, 1, 24, True)])
def test_layer_small_batch_fused_down_equals_stages(oracle, E, H, I, K, B, bias):
    """Decode batches of at most 24 routed pairs run the down projection and the combine
    as one launch (k_mx_downs). Where the per-stage down projection does not split K (at
    least 512 16-row tiles), the layer's output equals the per-stage entry points' bit for
    bit; everywhere it matches the oracle, and repeated calls give the same bits. The
    block (norm + layer + residual add in the same launch) is checked against the oracle
    block as well."""
    layer = syn.make_layer(E, H, I, K, seed=E * 7 + B, with_bias=bias)
    x = syn.make_x(B, H, seed=H + B)
    got, gidx, gw, dl = _run_layer(layer, x)
    sout, sidx, sw = _run_stages(dl, dev(x), B)
    assert np.array_equal(gidx, sidx) and np.array_equal(gw.view(np.uint32), sw.view(np.uint32))
    tiles = min(B * K, E) * (H // 16)
    if tiles >= 512:
        assert np.array_equal(got, sout), "fused down + combine differs from the per-stage path"
    for _ in range(2):
        again, _, _ = ops.moe_layer_forward(dl, dev(x), return_routing=True)
        torch.cuda.synchronize()
        assert np.array_equal(host(again, np.uint16), got)
    _check_layer(oracle, layer, x, f"fused small-batch down E={E} H={H} I={I} K={K} B={B}")


@pytest.mark.parametrize("B", [64, 1024])
def test_layer_x_not_16_byte_aligned(oracle, B):
    """x two bytes past a 16-byte boundary. The kernels that copy activation rows
    straight into LDS in 16-byte units (the decode streaming GEMV at B = 64, the
    LDS-staged grouped GEMM at 1024 tokens) and the router forms that load x 16 bytes at
    a time are not taken; the fallbacks give the oracle's indices and rel L2 < 1e-2."""
    layer = syn.make_layer(32, 2880, 2880, 4, seed=91)
    x = syn.make_x(B, 2880, seed=92)
    buf = torch.empty(B * 2880 + 8, dtype=torch.int16, device="cuda")
    xv = buf[1:1 + B * 2880].view(B, 2880)
    xv.copy_(dev(x))
    assert xv.data_ptr() % 16 == 2
    dl = ops.DeviceMoELayer.from_host(layer)
    out, idx, w = ops.moe_layer_forward(dl, xv, return_routing=True)
    torch.cuda.synchronize()
    r = oracle.moe_layer(layer, x)
    assert np.array_equal(host(idx), r["idx"])
    err = refmath.rel_l2(refmath.bf16_bits_to_f64(host(out, np.uint16)), refmath.bf16_bits_to_f64(r["out"]))
    say(f"x at 16-byte offset 2, B={B}: rel L2 = {err:.3e}")
    assert err < LAYER_TOL


def test_layer_automatic_chunk_limit_near_2gib(oracle):
    """H = 32, I = 32768, k = E = 32: h [b * k, I] bf16 takes 2 MiB per token, so the
    automatic chunk limit is 1023 tokens, whose h range (2,145,386,496 bytes) lies just
    under the 2^31 - 2^20 bytes a 32-bit buffer range may reach; the loads meant to read
    zeros at offset 2^31 must still land past it. 3069 tokens run as 3 automatic chunks
    of 1023, bit-identical to 6 chunks under max_chunk_tokens = 512 (every chunk takes
    the grouped GEMM), with rows of every chunk against the oracle."""
    H, I, E, K = 32, 32768, 32, 32
    layer = syn.make_layer(E, H, I, K, seed=93)
    B = 3 * 1023
    x = syn.make_x(B, H, seed=94)
    dl = ops.DeviceMoELayer.from_host(layer)
    dc = dl.with_chunk_limit(512)
    xd = dev(x)
    got = ops.moe_layer_forward(dl, xd, return_routing=True)
    ref = ops.moe_layer_forward(dc, xd, return_routing=True)
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.equal(a, b), "automatic chunks differ from 512-token chunks"
    rows = [0, 1022, 1023, 2046, 2047, B - 1]
    r = oracle.moe_layer(layer, x[rows])
    assert np.array_equal(host(got[1])[rows], r["idx"])
    err = refmath.rel_l2(refmath.bf16_bits_to_f64(host(got[0], np.uint16)[rows]),
                         refmath.bf16_bits_to_f64(r["out"]))
    say(f"automatic chunk limit (3 x 1023 tokens, h just under 2^31 bytes): rel L2 = {err:.3e}")
    assert err < LAYER_TOL


# ---- legacy single-token launchers ------------------------------------------------

@pytest.mark.parametrize("H,I", [(2880, 2880), (100, 36)])
def test_legacy_expert_forward_and_combine(oracle, H, I):
    rng = np.random.default_rng(H + I)
    bits = lambda shape, s: syn.bf16_from_f32(rng.standard_normal(shape, dtype=np.float32) * np.float32(s))
    x, wg, wu, wd = bits((H,), 1.0), bits((I, H), 0.02), bits((I, H), 0.02), bits((H, I), 0.02)
    dv = ops.GpuDevice()
    inter = torch.empty(I, dtype=torch.int16, device="cuda")
    out = torch.empty(H, dtype=torch.int16, device="cuda")
    ops.moe_expert_forward_gpu(dv, dev(x), dev(wg), dev(wu), dev(wd), inter, out, H, I)
    e_inter = oracle.legacy_expert_silu(x, wg, wu)
    g_inter = host(inter, np.uint16)
    assert refmath.rel_l2(refmath.bf16_bits_to_f64(g_inter), refmath.bf16_bits_to_f64(e_inter)) < 1e-2
    e_out = oracle.legacy_expert_down(g_inter, wd)
    assert refmath.rel_l2(refmath.bf16_bits_to_f64(host(out, np.uint16)), refmath.bf16_bits_to_f64(e_out)) < 1e-2
    K = 4
    ys = bits((K, H), 1.0)
    wk = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    comb = torch.empty(H, dtype=torch.int16, device="cuda")
    ops.moe_combine_gpu(dv, dev(ys), dev(wk), comb, K)
    assert np.array_equal(host(comb, np.uint16), oracle.legacy_combine(ys, wk))


def test_legacy_dequant_wrapper(oracle):
    packed, scales, numel = syn.make_dequant_input((4, 64, 96), seed=5)
    dv = ops.GpuDevice()
    out = torch.empty(numel, dtype=torch.int16, device="cuda")
    ops.mxfp4_dequant_gpu(dv, dev(packed), dev(scales), out, 32)
    assert np.array_equal(host(out, np.uint16), oracle.mxfp4_dequant(packed, scales, numel))


def test_error_reporting_on_device_path():
    cfg = capi.MoEConfig(2880, 2880, 32, 4, 1.702, 7.0)
    layer = syn.make_layer(32, 2880, 2880, 4, seed=1)
    dl = ops.DeviceMoELayer.from_host(layer)
    x = dev(syn.make_x(2, 2880, seed=1))
    out = torch.empty((2, 2880), dtype=torch.int16, device="cuda")
    small = torch.empty(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(capi.BackendError) as ei:
        dl.forward(x, out, small)
    assert ei.value.code == capi.PHYSLLM_MOE_EWORKSPACE
    n = capi.lib().physllm_moe_workspace_bytes(ctypes.byref(cfg), 2)
    ws = torch.empty(n, dtype=torch.uint8, device="cuda")
    dl.forward(x, out, ws)
    torch.cuda.synchronize()
