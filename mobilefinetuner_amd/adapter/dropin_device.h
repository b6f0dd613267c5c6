// Host-side device plumbing shared by the finetune_ops drop-in adapters
// (memory_efficient_attention_hip.cpp, lora_linear_hip.cpp, lm_loss_hip.cpp):
// error checks that throw std::runtime_error with the operator's name, one
// process-wide HIP stream at default priority, a caching device allocator
// behind an owning device buffer, and copies between the reference's host
// tensors and device memory.
#ifndef MFT_DROPIN_DEVICE_H
#define MFT_DROPIN_DEVICE_H

#include <cstdint>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
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

// Caching device allocator of the adapters.  A request is rounded up to a
// size class; a released block goes onto its class's free list and the next
// request of that class takes it, so a training loop's per-step buffers
// (saved operands, gradients, workspaces) stop costing a hipMalloc/hipFree
// pair per buffer per call.  Blocks are reused without waiting: every
// adapter enqueues all of its device work on the one stream(), so work that
// touches a reused block is ordered after the stream's earlier uses of it.
// Cached blocks are returned to the device only when a hipMalloc fails (after
// draining the stream) and are otherwise held until the process ends.
class DevicePool {
public:
    static DevicePool& instance() {
        static DevicePool* pool = new DevicePool();  // never destroyed: HIP may be torn down first
        return *pool;
    }

    // Bytes of the class a request of `bytes` is served from: multiples of
    // 4 KiB up to 1 MiB, then quarter steps between powers of two (at most
    // 25% rounding).
    static size_t size_class(size_t bytes) {
        if (bytes <= (size_t(1) << 20)) return (bytes + 4095) & ~size_t(4095);
        size_t p = size_t(1) << 20;
        while (p * 2 < bytes) p *= 2;
        const size_t step = p / 4;
        return (bytes + step - 1) / step * step;
    }

    void* get(size_t bytes) {
        const size_t cls = size_class(bytes);
        std::lock_guard<std::mutex> lock(mu_);
        auto& fl = free_[cls];
        void* p = nullptr;
        if (!fl.empty()) {
            p = fl.back();
            fl.pop_back();
            cached_ -= cls;
        } else {
            hipError_t e = hipMalloc(&p, cls);
            if (e == hipErrorOutOfMemory && cached_) {
                (void)hipGetLastError();
                release_cached_locked();
                e = hipMalloc(&p, cls);
            }
            hip_check("drop-in", e, "hipMalloc");
            ++mallocs_;
        }
        live_ += cls;
        return p;
    }

    void put(void* p, size_t bytes) {
        const size_t cls = size_class(bytes);
        std::lock_guard<std::mutex> lock(mu_);
        free_[cls].push_back(p);
        live_ -= cls;
        cached_ += cls;
    }

    size_t live_bytes() {
        std::lock_guard<std::mutex> lock(mu_);
        return live_;
    }
    size_t cached_bytes() {
        std::lock_guard<std::mutex> lock(mu_);
        return cached_;
    }
    size_t device_mallocs() {
        std::lock_guard<std::mutex> lock(mu_);
        return mallocs_;
    }

private:
    void release_cached_locked();
    std::mutex mu_;
    std::unordered_map<size_t, std::vector<void*>> free_;
    size_t live_ = 0, cached_ = 0, mallocs_ = 0;
};

// Device memory owned by one adapter object (back to the pool with it).
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
        if (bytes) ptr_ = DevicePool::instance().get(bytes);
    }
    ~DeviceBuffer() {
        if (ptr_) DevicePool::instance().put(ptr_, bytes_);
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

inline void DevicePool::release_cached_locked() {
    (void)hipStreamSynchronize(stream());  // the stream may still read freed blocks
    for (auto& kv : free_) {
        for (void* p : kv.second) (void)hipFree(p);
        kv.second.clear();
    }
    cached_ = 0;
}

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
