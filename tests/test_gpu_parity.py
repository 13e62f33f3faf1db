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
                                        (256, 4, 128, False), (3000, 1, 3, True)])
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


@pytest.mark.parametrize("E,H,I,K,B", [(8, 256, 128, 3, 20), (16, 512, 1024, 4, 40), (3, 96, 160, 1, 37),
                                       (8, 256, 4096, 2, 1), (8, 128, 3200, 2, 3)])
def test_layer_odd_shapes(oracle, E, H, I, K, B):
    """Includes down projections whose reduction (I = 4096, 3200) is split over
    several K ranges at small batch: 128 and 100 scale blocks per row."""
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


@pytest.mark.parametrize("E,H,K,B", [(128, 256, 4, 100), (128, 2880, 4, 256), (300, 96, 8, 40), (96, 224, 2, 100),
                                     (64, 256, 4, 100), (32, 2880, 4, 64), (40, 96, 1, 17), (8, 128, 8, 127),
                                     (100, 96, 4, 300), (128, 3072, 8, 130), (65, 64, 2, 129)])
def test_layer_two_launch_router(oracle, E, H, K, B):
    """Mid-size batches (B * E >= 8192 outside the two-pass range) route in two
    launches (logits of 8 tokens x 16 experts per workgroup, then one selection
    workgroup per token); the smaller ones here take k_router. Indices bit-exact and
    weights as the oracle's, with ties to the lower index, a NaN token, more than 256
    experts (arg-max rounds), k = 1 and k = E. Batches of 128 or more with 64 < E <= 128
    take the tiled two-pass router (bounds per 16 x 16 tile, then one selection wave
    per token), including expert counts that are not multiples of 16."""
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


def test_layer_nan_activation_propagates(oracle):
    layer = syn.make_layer(4, 64, 64, 2, seed=12)
    x = syn.make_x(4, 64, seed=12)
    x[1, 7] = 0x7FC0
    got, gidx, _, _ = _run_layer(layer, x)
    r = oracle.moe_layer(layer, x)
    assert np.array_equal(gidx, r["idx"])
    gf, ef = refmath.bf16_bits_to_f64(got), refmath.bf16_bits_to_f64(r["out"])
    assert np.array_equal(np.isnan(gf), np.isnan(ef))
    ok = ~np.isnan(ef)
    assert refmath.rel_l2(gf[ok], ef[ok]) < LAYER_TOL


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


def test_layer_prefill_config3(oracle):
    """4096-token prefill: indices for every token against the oracle router; layer
    outputs for a seeded sample of 96 tokens (each output row depends only on its
    own token, so the sample is checked exactly as the full run would be)."""
    say("layer config 3 (prefill 4096)")
    layer, x = syn.make_config(3)
    got, gidx, gw, _ = _run_layer(layer, x)
    eidx, ew = oracle.router(x, layer.router_w, layer.router_b, layer.top_k)
    assert np.array_equal(gidx, eidx)
    assert np.allclose(gw, ew, rtol=1e-6, atol=1e-7)
    rows = np.sort(np.random.default_rng(3).choice(x.shape[0], 96, replace=False))
    r = oracle.moe_layer(layer, x[rows])
    err = refmath.rel_l2(refmath.bf16_bits_to_f64(got[rows]), refmath.bf16_bits_to_f64(r["out"]))
    say(f"config 3 sample rel L2 = {err:.3e}")
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
