// C++ host layer over libphysllm_moe's C ABI, mirroring PhysLLM's Rust crate
// crates/rocm-backend: GpuDevice (src/device.rs:24-133), DeviceTensor<T>
// (src/tensor.rs:21-146), BackendError (src/lib.rs:35-47), the MoE operator
// wrappers (src/ops.rs:597-696) and the RMSNorm / residual-add wrappers around the
// MoE layer (src/ops.rs:366-384, :421-435) with the same names, size derivation and error
// behaviour: each wrapper launches on the device's stream, then synchronises and
// throws BackendError if the launch or the stream reported an error.
//
// 16-bit tensors hold bf16 bit patterns (the Rust side carries them in
// DeviceTensor<f16> storage); E8M0 scales are DeviceTensor<uint8_t>.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <numeric>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/physllm_moe.h"

namespace rocm_backend {

using bf16 = uint16_t;

struct BackendError : std::runtime_error {
    int code;
    BackendError(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw BackendError((int)e, std::string(what) + ": " + hipGetErrorString(e));
}

// Legacy launchers return void: their argument errors arrive through the
// library's thread-local last-error channel.
inline void moe_check(const char* what) {
    const int c = physllm_moe_last_error();
    if (c != PHYSLLM_MOE_OK) throw BackendError(c, std::string(what) + ": " + physllm_moe_last_error_message());
}

// One HIP device and its stream (device.rs:24-27, open_device at :42-113).
class GpuDevice {
  public:
    static GpuDevice open_device(int idx) {
        hip_check(hipSetDevice(idx), "hipSetDevice");
        hipStream_t s = nullptr;
        hip_check(hipStreamCreate(&s), "hipStreamCreate");
        return GpuDevice(idx, s);
    }
    static GpuDevice open_best() { return open_device(0); }
    GpuDevice(GpuDevice&& o) noexcept : idx_(o.idx_), stream_(std::exchange(o.stream_, nullptr)) {}
    GpuDevice(const GpuDevice&) = delete;
    GpuDevice& operator=(const GpuDevice&) = delete;
    ~GpuDevice() {
        if (stream_) (void)hipStreamDestroy(stream_);
    }
    // device.rs:116-127
    void synchronise() const { hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }
    // device.rs:130-132
    hipStream_t raw_stream() const { return stream_; }
    int device_id() const { return idx_; }

  private:
    GpuDevice(int idx, hipStream_t s) : idx_(idx), stream_(s) {}
    int idx_;
    hipStream_t stream_;
};

// A typed device buffer with a shape (tensor.rs:21-146): hipMalloc on alloc,
// hipFree on destruction, blocking host copies.
template <class T>
class DeviceTensor {
  public:
    static DeviceTensor alloc(std::vector<size_t> shape) {
        DeviceTensor t;
        t.shape_ = std::move(shape);
        t.numel_ = std::accumulate(t.shape_.begin(), t.shape_.end(), (size_t)1, std::multiplies<size_t>());
        if (t.numel_) hip_check(hipMalloc((void**)&t.ptr_, t.numel_ * sizeof(T)), "hipMalloc");
        return t;
    }
    static DeviceTensor from_slice(const std::vector<T>& data, std::vector<size_t> shape) {
        DeviceTensor t = alloc(std::move(shape));
        t.copy_from_host(data);
        return t;
    }
    // numel elements straight from host memory (e.g. a file mapping), no staging copy.
    static DeviceTensor from_host(const T* data, std::vector<size_t> shape) {
        DeviceTensor t = alloc(std::move(shape));
        if (t.numel_) hip_check(hipMemcpy(t.ptr_, data, t.numel_ * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
        return t;
    }
    DeviceTensor() = default;
    DeviceTensor(DeviceTensor&& o) noexcept
        : ptr_(std::exchange(o.ptr_, nullptr)), shape_(std::move(o.shape_)), numel_(std::exchange(o.numel_, 0)) {}
    DeviceTensor& operator=(DeviceTensor&& o) noexcept {
        if (this != &o) {
            release();
            ptr_ = std::exchange(o.ptr_, nullptr);
            shape_ = std::move(o.shape_);
            numel_ = std::exchange(o.numel_, 0);
        }
        return *this;
    }
    DeviceTensor(const DeviceTensor&) = delete;
    DeviceTensor& operator=(const DeviceTensor&) = delete;
    ~DeviceTensor() { release(); }

    void copy_from_host(const std::vector<T>& data) {
        if (data.size() != numel_) throw BackendError(PHYSLLM_MOE_EINVAL, "host slice length != tensor numel");
        if (numel_) hip_check(hipMemcpy(ptr_, data.data(), numel_ * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    std::vector<T> copy_to_host() const {
        std::vector<T> out(numel_);
        if (numel_) hip_check(hipMemcpy(out.data(), ptr_, numel_ * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
        return out;
    }
    const std::vector<size_t>& shape() const { return shape_; }
    size_t numel() const { return numel_; }
    size_t rows() const { return shape_.size() >= 2 ? shape_[shape_.size() - 2] : 1; }
    size_t cols() const { return shape_.empty() ? 0 : shape_.back(); }
    T* raw_ptr() const { return ptr_; }

  private:
    void release() {
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = nullptr;
    }
    T* ptr_ = nullptr;
    std::vector<size_t> shape_;
    size_t numel_ = 0;
};

// ---- ops.rs:366-384, :421-435 (the steps either side of the MoE layer) ---------

// ops.rs:366-384: batch = input.rows(), hidden = input.cols().
inline void rms_norm_gpu(const GpuDevice& dev, const DeviceTensor<bf16>& input, const DeviceTensor<bf16>& weight,
                         DeviceTensor<bf16>& output, float eps) {
    launch_rms_norm(input.raw_ptr(), weight.raw_ptr(), output.raw_ptr(), (int)input.rows(), (int)input.cols(), eps,
                    dev.raw_stream());
    moe_check("launch_rms_norm");
    dev.synchronise();
}

// ops.rs:421-435: output += residual over output.numel() elements.
inline void residual_add_gpu(const GpuDevice& dev, DeviceTensor<bf16>& output, const DeviceTensor<bf16>& residual) {
    launch_residual_add(output.raw_ptr(), residual.raw_ptr(), (int)output.numel(), dev.raw_stream());
    moe_check("launch_residual_add");
    dev.synchronise();
}

// ---- ops.rs:597-696 -----------------------------------------------------------

// ops.rs:597-618: batch = hidden.rows(), hidden_dim = hidden.cols().
inline void moe_router_gpu(const GpuDevice& dev, const DeviceTensor<bf16>& hidden,
                           const DeviceTensor<bf16>& router_weight, DeviceTensor<int32_t>& expert_indices,
                           DeviceTensor<float>& expert_weights, size_t num_experts, size_t top_k) {
    launch_moe_router(hidden.raw_ptr(), router_weight.raw_ptr(), expert_indices.raw_ptr(), expert_weights.raw_ptr(),
                      (int)hidden.rows(), (int)hidden.cols(), (int)num_experts, (int)top_k, dev.raw_stream());
    moe_check("launch_moe_router");
    dev.synchronise();
}

// ops.rs:621-652: SiLU(gate) * up -> intermediate, then the down projection.
inline void moe_expert_forward_gpu(const GpuDevice& dev, const DeviceTensor<bf16>& input,
                                   const DeviceTensor<bf16>& w_gate, const DeviceTensor<bf16>& w_up,
                                   const DeviceTensor<bf16>& w_down, DeviceTensor<bf16>& intermediate,
                                   DeviceTensor<bf16>& output, size_t hidden_dim, size_t intermediate_dim) {
    launch_moe_expert_silu(input.raw_ptr(), w_gate.raw_ptr(), w_up.raw_ptr(), intermediate.raw_ptr(), (int)hidden_dim,
                           (int)intermediate_dim, dev.raw_stream());
    moe_check("launch_moe_expert_silu");
    launch_moe_expert_down(intermediate.raw_ptr(), w_down.raw_ptr(), output.raw_ptr(), (int)hidden_dim,
                           (int)intermediate_dim, dev.raw_stream());
    moe_check("launch_moe_expert_down");
    dev.synchronise();
}

// ops.rs:655-674: hidden_dim = output.numel().
inline void moe_combine_gpu(const GpuDevice& dev, const DeviceTensor<bf16>& expert_outputs,
                            const DeviceTensor<float>& expert_weights, DeviceTensor<bf16>& output, size_t top_k) {
    launch_moe_combine(expert_outputs.raw_ptr(), expert_weights.raw_ptr(), output.raw_ptr(), (int)output.numel(),
                       (int)top_k, dev.raw_stream());
    moe_check("launch_moe_combine");
    dev.synchronise();
}

// ops.rs:677-696: numel = output.numel(); scales are E8M0 bytes, output bf16.
inline void mxfp4_dequant_gpu(const GpuDevice& dev, const DeviceTensor<uint8_t>& packed,
                              const DeviceTensor<uint8_t>& scales, DeviceTensor<bf16>& output, size_t block_size) {
    launch_mxfp4_dequant(packed.raw_ptr(), scales.raw_ptr(), output.raw_ptr(), (int)output.numel(), (int)block_size,
                         dev.raw_stream());
    moe_check("launch_mxfp4_dequant");
    dev.synchronise();
}

}  // namespace rocm_backend
