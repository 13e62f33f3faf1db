// GPU test of the C++ host layer (physllm_amd/host) against the CPU oracle.
// Exercises the ops.rs-style wrappers (router, expert forward, combine, dequant,
// rms_norm, residual add), the whole-layer MoELayer::forward_moe_layer, the block
// MoELayer::forward_moe_block, and BackendError on bad input.
// Prints one line per check and exits nonzero on the first failure.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../oracle/moe_oracle.h"
#include "../../physllm_amd/host/moe_engine.hpp"

using namespace rocm_backend;

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {  // splitmix64
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double uniform() { return (next_u64() >> 11) * (1.0 / 9007199254740992.0); }
static float normal(float sigma) {
    const double u1 = uniform() + 1e-300, u2 = uniform();
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2)) * sigma;
}
static std::vector<bf16> bf16_vec(size_t n, float sigma) {
    std::vector<bf16> v(n);
    for (auto& x : v) x = or_f32_to_bf16(normal(sigma));
    return v;
}
static std::vector<uint8_t> byte_vec(size_t n) {
    std::vector<uint8_t> v(n);
    for (auto& x : v) x = (uint8_t)next_u64();
    return v;
}
static std::vector<uint8_t> scale_vec(size_t n) {
    std::vector<uint8_t> v(n);
    for (auto& x : v) x = (uint8_t)(119 + next_u64() % 5);
    return v;
}
static double rel_l2(const std::vector<bf16>& a, const std::vector<bf16>& b) {
    double num = 0, den = 0;
    for (size_t i = 0; i < a.size(); ++i) {
        const double x = or_bf16_to_f32(a[i]), y = or_bf16_to_f32(b[i]);
        num += (x - y) * (x - y);
        den += y * y;
    }
    return std::sqrt(num / (den > 0 ? den : 1));
}

static int failures = 0;
static void check(bool ok, const char* name, double v = 0) {
    std::printf("%s %s %.3e\n", ok ? "PASS" : "FAIL", name, v);
    std::fflush(stdout);
    if (!ok) ++failures;
}

int main() {
    GpuDevice dev = GpuDevice::open_best();

    // ---- whole layer through MoELayer::forward_moe_layer ----
    {
        const int E = 8, H = 256, I = 128, K = 2, B = 7;
        auto rw = bf16_vec((size_t)E * H, 0.02f), rb = bf16_vec(E, 0.02f);
        auto gub = byte_vec((size_t)E * 2 * I * H / 2), gus = scale_vec((size_t)E * 2 * I * H / 32);
        auto gbias = bf16_vec((size_t)E * 2 * I, 0.02f);
        auto db = byte_vec((size_t)E * H * I / 2), ds = scale_vec((size_t)E * H * I / 32);
        auto dbias = bf16_vec((size_t)E * H, 0.02f);
        auto x = bf16_vec((size_t)B * H, 1.0f);

        llm_core::MoELayerWeightsMXFP4 w;
        w.router_weight = DeviceTensor<bf16>::from_slice(rw, {(size_t)E, (size_t)H});
        w.router_bias = DeviceTensor<bf16>::from_slice(rb, {(size_t)E});
        w.gate_up_blocks = DeviceTensor<uint8_t>::from_slice(gub, {(size_t)E, 2 * (size_t)I, (size_t)H / 2});
        w.gate_up_scales = DeviceTensor<uint8_t>::from_slice(gus, {(size_t)E, 2 * (size_t)I, (size_t)H / 32});
        w.gate_up_bias = DeviceTensor<bf16>::from_slice(gbias, {(size_t)E, 2 * (size_t)I});
        w.down_blocks = DeviceTensor<uint8_t>::from_slice(db, {(size_t)E, (size_t)H, (size_t)I / 2});
        w.down_scales = DeviceTensor<uint8_t>::from_slice(ds, {(size_t)E, (size_t)H, (size_t)I / 32});
        w.down_bias = DeviceTensor<bf16>::from_slice(dbias, {(size_t)E, (size_t)H});
        llm_core::MoELayer layer({H, I, E, K}, std::move(w));
        auto xd = DeviceTensor<bf16>::from_slice(x, {(size_t)B, (size_t)H});
        auto out = DeviceTensor<bf16>::alloc({(size_t)B, (size_t)H});
        auto idx = DeviceTensor<int32_t>::alloc({(size_t)B, (size_t)K});
        auto wts = DeviceTensor<float>::alloc({(size_t)B, (size_t)K});
        layer.forward_moe_layer(dev, xd, out, &idx, &wts);

        or_moe_cfg oc{H, I, E, K, 1.702f, 7.0f};
        or_moe_weights ow{rw.data(), rb.data(), gub.data(), gus.data(), gbias.data(), db.data(), ds.data(), dbias.data()};
        std::vector<bf16> eout((size_t)B * H);
        std::vector<int32_t> eidx((size_t)B * K);
        std::vector<float> ew((size_t)B * K);
        or_moe_layer(&oc, &ow, x.data(), B, eout.data(), eidx.data(), ew.data(), nullptr, nullptr, 4);
        check(idx.copy_to_host() == eidx, "layer top-k indices bit-exact");
        const double err = rel_l2(out.copy_to_host(), eout);
        check(err < 1e-2, "layer output rel L2 < 1e-2", err);

        // ---- the block: rms_norm -> layer -> residual add, in place (moe.rs:238-313) ----
        auto nw = bf16_vec(H, 0.5f);
        auto nwd = DeviceTensor<bf16>::from_slice(nw, {(size_t)H});
        auto resid = DeviceTensor<bf16>::from_slice(x, {(size_t)B, (size_t)H});
        layer.forward_moe_block(dev, resid, nwd, 1e-5f, &idx, &wts);
        std::vector<bf16> bout((size_t)B * H);
        or_moe_block(&oc, &ow, x.data(), nw.data(), 1e-5f, B, bout.data(), eidx.data(), ew.data(), 4);
        check(idx.copy_to_host() == eidx, "block top-k indices bit-exact");
        const double berr = rel_l2(resid.copy_to_host(), bout);
        check(berr < 1e-2, "block output rel L2 < 1e-2", berr);
        // the same through the separate wrappers (ops.rs:366-384, :421-435)
        auto hn = DeviceTensor<bf16>::alloc({(size_t)B, (size_t)H});
        rms_norm_gpu(dev, xd, nwd, hn, 1e-5f);
        std::vector<bf16> ehn((size_t)B * H);
        or_rms_norm(x.data(), nw.data(), ehn.data(), B, H, 1e-5f);
        check(hn.copy_to_host() == ehn, "rms_norm_gpu bit-exact");
        layer.forward_moe_layer(dev, hn, out);
        residual_add_gpu(dev, out, xd);
        check(out.copy_to_host() == resid.copy_to_host(), "block == rms_norm_gpu + layer + residual_add_gpu");
    }

    // ---- legacy wrappers (ops.rs:597-696) ----
    {
        const int B = 3, H = 192, E = 16, K = 4, I = 96;
        auto h = bf16_vec((size_t)B * H, 1.0f), rw = bf16_vec((size_t)E * H, 0.02f);
        auto hd = DeviceTensor<bf16>::from_slice(h, {(size_t)B, (size_t)H});
        auto rwd = DeviceTensor<bf16>::from_slice(rw, {(size_t)E, (size_t)H});
        auto idx = DeviceTensor<int32_t>::alloc({(size_t)B, (size_t)K});
        auto wts = DeviceTensor<float>::alloc({(size_t)B, (size_t)K});
        moe_router_gpu(dev, hd, rwd, idx, wts, E, K);
        std::vector<int32_t> eidx((size_t)B * K);
        std::vector<float> ew((size_t)B * K);
        or_router(h.data(), rw.data(), nullptr, B, H, E, K, eidx.data(), ew.data(), nullptr, 1);
        check(idx.copy_to_host() == eidx, "moe_router_gpu indices bit-exact");
        auto gw = wts.copy_to_host();
        double werr = 0;
        for (size_t i = 0; i < gw.size(); ++i) werr = std::fmax(werr, std::fabs(gw[i] - ew[i]));
        check(werr < 1e-6, "moe_router_gpu weights", werr);

        auto x = bf16_vec(H, 1.0f), wg = bf16_vec((size_t)I * H, 0.05f), wu = bf16_vec((size_t)I * H, 0.05f),
             wd = bf16_vec((size_t)H * I, 0.05f);
        auto xd1 = DeviceTensor<bf16>::from_slice(x, {1, (size_t)H});
        auto wgd = DeviceTensor<bf16>::from_slice(wg, {(size_t)I, (size_t)H});
        auto wud = DeviceTensor<bf16>::from_slice(wu, {(size_t)I, (size_t)H});
        auto wdd = DeviceTensor<bf16>::from_slice(wd, {(size_t)H, (size_t)I});
        auto inter = DeviceTensor<bf16>::alloc({1, (size_t)I});
        auto y = DeviceTensor<bf16>::alloc({1, (size_t)H});
        moe_expert_forward_gpu(dev, xd1, wgd, wud, wdd, inter, y, H, I);
        std::vector<bf16> einter(I), ey(H);
        or_legacy_expert_silu(x.data(), wg.data(), wu.data(), einter.data(), H, I);
        auto ginter = inter.copy_to_host();
        check(rel_l2(ginter, einter) < 1e-2, "moe_expert_forward_gpu intermediate", rel_l2(ginter, einter));
        or_legacy_expert_down(ginter.data(), wd.data(), ey.data(), H, I);
        check(rel_l2(y.copy_to_host(), ey) < 1e-2, "moe_expert_forward_gpu output", rel_l2(y.copy_to_host(), ey));

        auto ys = bf16_vec((size_t)K * H, 1.0f);
        std::vector<float> wk = {0.4f, 0.3f, 0.2f, 0.1f};
        auto ysd = DeviceTensor<bf16>::from_slice(ys, {(size_t)K, (size_t)H});
        auto wkd = DeviceTensor<float>::from_slice(wk, {(size_t)K});
        auto comb = DeviceTensor<bf16>::alloc({(size_t)H});
        moe_combine_gpu(dev, ysd, wkd, comb, K);
        std::vector<bf16> ecomb(H);
        or_legacy_combine(ys.data(), wk.data(), ecomb.data(), H, K);
        check(comb.copy_to_host() == ecomb, "moe_combine_gpu bit-exact");

        const size_t numel = 4096;
        auto pk = byte_vec(numel / 2), sc = byte_vec(numel / 32);
        auto pkd = DeviceTensor<uint8_t>::from_slice(pk, {numel / 2});
        auto scd = DeviceTensor<uint8_t>::from_slice(sc, {numel / 32});
        auto dq = DeviceTensor<bf16>::alloc({numel});
        mxfp4_dequant_gpu(dev, pkd, scd, dq, 32);
        std::vector<bf16> edq(numel);
        or_mxfp4_dequant(pk.data(), sc.data(), edq.data(), (int64_t)numel, 32, 1);
        check(dq.copy_to_host() == edq, "mxfp4_dequant_gpu bit-exact");

        bool threw = false;
        try {
            moe_router_gpu(dev, hd, rwd, idx, wts, E, 40);  // top_k > num_experts
        } catch (const BackendError& e) {
            threw = e.code == PHYSLLM_MOE_EINVAL;
        }
        check(threw, "BackendError on top_k > num_experts");
    }
    std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
