// Host-side device plumbing shared by the finetune_ops drop-in adapters
// (memory_efficient_attention_hip.cpp, lora_linear_hip.cpp, lm_loss_hip.cpp):
// error checks that throw std::runtime_error with the operator's name, one
// process-wide HIP stream at default priority, an owning device buffer, and
// copies between the reference's host tensors and device memory.
#ifndef MFT_DROPIN_DEVICE_H
#define MFT_DROPIN_DEVICE_H

#include <cstdint>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "mft/attention.h"
#include "ops.h"

namespace ops {
namespace dropin {

inline void hip_check(const char* who, hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string(who) + ": " + what + ": " + hipGetErrorString(e));
}

inline void mft_check(const char* who, mft_status st) {
    if (st != MFT_OK) throw std::runtime_error(std::string(who) + ": " + mft_last_error());
}

// The stream every adapter enqueues on, created on first use.  One stream
// keeps the work of different operators in call order.
inline hipStream_t stream() {
    static std::once_flag once;
    static hipStream_t s = nullptr;
    std::call_once(once, [] { hip_check("drop-in", hipStreamCreate(&s), "hipStreamCreate"); });
    return s;
}

// Device memory owned by one adapter object (freed with it).
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
        if (bytes) hip_check("drop-in", hipMalloc(&ptr_, bytes), "hipMalloc");
    }
    ~DeviceBuffer() {
        if (ptr_) (void)hipFree(ptr_);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    void* get() const { return ptr_; }
    float* f() const { return static_cast<float*>(ptr_); }
    size_t bytes() const { return bytes_; }

private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
};
using Buf = std::unique_ptr<DeviceBuffer>;

// n bytes of host memory into a new device buffer (ordered on stream(); the
// source must stay alive until the stream reaches the copy).
inline Buf upload_bytes(const void* src, size_t n) {
    auto buf = std::make_unique<DeviceBuffer>(n);
    if (n) hip_check("drop-in", hipMemcpyAsync(buf->get(), src, n, hipMemcpyHostToDevice, stream()), "copy to device");
    return buf;
}

// A floating-point host tensor as fp32 values on the device; fp16 and bf16
// storage is widened exactly (the reference's read_tensor_float and
// tensor_row_value do the same).
inline Buf upload_f32(const TensorPtr& t, const char* who) {
    const int64_t n = t->numel();
    if (t->dtype() == kFloat32) return upload_bytes(t->data<float>(), static_cast<size_t>(n) * 4);
    if (t->dtype() != kBFloat16 && t->dtype() != kFloat16)
        throw std::runtime_error(std::string(who) + ": expected floating-point tensor storage, got " +
                                 DTypeUtils::to_string(t->dtype()));
    std::vector<float> v(static_cast<size_t>(n));
    const uint16_t* bits = t->data<uint16_t>();
    for (int64_t i = 0; i < n; ++i)
        v[static_cast<size_t>(i)] =
            t->dtype() == kBFloat16 ? bf16_bits_to_float32(bits[i]) : fp16_bits_to_float32(bits[i]);
    auto buf = upload_bytes(v.data(), v.size() * 4);
    hip_check(who, hipStreamSynchronize(stream()), "synchronize");  // v is a local
    return buf;
}

// fp32 device values into a new host tensor of `shape` (ordered on stream();
// synchronize before reading it).
inline TensorPtr download_f32(const DeviceBuffer& src, const std::vector<int64_t>& shape) {
    auto out = zeros(shape, kFloat32, kCPU);
    hip_check("drop-in",
              hipMemcpyAsync(out->data<float>(), src.get(), static_cast<size_t>(out->numel()) * 4,
                             hipMemcpyDeviceToHost, stream()),
              "copy to host");
    return out;
}

}  // namespace dropin
}  // namespace ops

#endif  // MFT_DROPIN_DEVICE_H
