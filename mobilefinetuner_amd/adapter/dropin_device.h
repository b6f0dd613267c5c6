// Host-side device plumbing shared by the finetune_ops drop-in adapters
// (memory_efficient_attention_hip.cpp, lora_linear_hip.cpp, lm_loss_hip.cpp):
// error checks that throw std::runtime_error with the operator's name, one
// process-wide HIP stream at default priority, a caching device allocator
// behind an owning device buffer, and copies between the reference's host
// tensors and device memory.
#ifndef MFT_DROPIN_DEVICE_H
#define MFT_DROPIN_DEVICE_H

#include <algorithm>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
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

// Host memcpy split over a few persistent threads and the caller.  One
// thread moves roughly 10-20 GB/s between pinned and pageable memory, well
// under the DMA engines' rate over PCIe.
class CopyPool {
public:
    static CopyPool& instance() {
        static CopyPool* p = new CopyPool();  // never destroyed; its threads idle on a condition variable
        return *p;
    }

    void copy(void* dst, const void* src, size_t n) {
        const size_t parts = std::min<size_t>(kWorkers + 1, std::max<size_t>(1, n / kMinPart));
        if (parts <= 1) {
            std::memcpy(dst, src, n);
            return;
        }
        std::lock_guard<std::mutex> call(call_mu_);  // one job at a time
        const size_t per = ((n + parts - 1) / parts + 63) & ~size_t(63);
        {
            std::lock_guard<std::mutex> lk(mu_);
            dst_ = static_cast<char*>(dst);
            src_ = static_cast<const char*>(src);
            n_ = n;
            per_ = per;
            parts_ = parts;
            pending_ = parts - 1;
            ++gen_;
        }
        work_cv_.notify_all();
        part(parts - 1, static_cast<char*>(dst), static_cast<const char*>(src), n, per);
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return pending_ == 0; });
    }

private:
    static constexpr size_t kWorkers = 4;
    static constexpr size_t kMinPart = size_t(512) << 10;

    static void part(size_t i, char* dst, const char* src, size_t n, size_t per) {
        const size_t off = i * per;
        if (off < n) std::memcpy(dst + off, src + off, std::min(per, n - off));
    }

    CopyPool() {
        for (size_t w = 0; w < kWorkers; ++w) std::thread([this, w] { worker(w); }).detach();
    }

    // Worker w copies part w of every job with more than w + 1 parts (the
    // caller copies the last part).  A job is posted only after the previous
    // one finished, so a worker cannot miss a job it takes part in.
    void worker(size_t w) {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            work_cv_.wait(lk, [&] { return gen_ != seen; });
            seen = gen_;
            if (w + 1 >= parts_) continue;
            char* d = dst_;
            const char* s = src_;
            const size_t n = n_, per = per_;
            lk.unlock();
            part(w, d, s, n, per);
            lk.lock();
            if (--pending_ == 0) done_cv_.notify_one();
        }
    }

    std::mutex call_mu_, mu_;
    std::condition_variable work_cv_, done_cv_;
    char* dst_ = nullptr;
    const char* src_ = nullptr;
    size_t n_ = 0, per_ = 0, parts_ = 0, pending_ = 0;
    uint64_t gen_ = 0;
};

// Copies between the reference's pageable host tensors and device memory,
// staged through kBufs pinned host buffers (hipHostMalloc) chunk by chunk:
// the host copy of one chunk (CopyPool) runs while the DMAs of the others are
// in flight.  A call takes several tensors as one pipeline, so the pipeline
// fills once per call, not once per tensor.  Host tensors are never
// registered (page-locked in place).
struct Segment {
    void* dst;
    const void* src;
    size_t n;
};

class Stager {
public:
    static Stager& instance() {
        static Stager* s = new Stager();  // never destroyed: HIP may be torn down first
        return *s;
    }

    // host -> device; returns once the host bytes are copied out (the sources
    // may be freed), the DMAs ordered on stream().
    void upload(const std::vector<Segment>& segs) {
        std::lock_guard<std::mutex> lock(mu_);
        for (const Segment& g : segs)
            for (size_t off = 0; off < g.n; off += kChunk) {
                const int i = take();
                const size_t len = std::min(kChunk, g.n - off);
                CopyPool::instance().copy(buf_[i], static_cast<const char*>(g.src) + off, len);
                hip_check("drop-in", hipMemcpyAsync(static_cast<char*>(g.dst) + off, buf_[i], len,
                                                    hipMemcpyHostToDevice, stream()),
                          "copy to device");
                hip_check("drop-in", hipEventRecord(ev_[i], stream()), "staging");
            }
    }

    // device -> host, after the work already on stream(); returns when the
    // host holds the data.
    void download(const std::vector<Segment>& segs) {
        std::lock_guard<std::mutex> lock(mu_);
        try {
            for (const Segment& g : segs)
                for (size_t off = 0; off < g.n; off += kChunk) {
                    const int i = take();
                    const size_t len = std::min(kChunk, g.n - off);
                    hip_check("drop-in", hipMemcpyAsync(buf_[i], static_cast<const char*>(g.src) + off, len,
                                                        hipMemcpyDeviceToHost, stream()),
                              "copy to host");
                    hip_check("drop-in", hipEventRecord(ev_[i], stream()), "staging");
                    out_[i] = {static_cast<char*>(g.dst) + off, len};
                }
            for (int k = 0; k < kBufs; ++k) take();  // drain the rest in order
        } catch (...) {
            // The destinations belong to the failed call: never copy into them later.
            for (Pending& p : out_) p = {};
            throw;
        }
    }

private:
    static constexpr size_t kChunk = size_t(4) << 20;
    static constexpr int kBufs = 3;

    // The next buffer in rotation, once free: its last DMA has completed and,
    // for a download, its chunk has been copied out to the host.
    int take() {
        const int i = next_;
        next_ = (next_ + 1) % kBufs;
        if (busy_[i]) hip_check("drop-in", hipEventSynchronize(ev_[i]), "staging");
        if (out_[i].dst) CopyPool::instance().copy(out_[i].dst, buf_[i], out_[i].n);
        out_[i] = {};
        busy_[i] = true;
        return i;
    }

    Stager() {
        for (int i = 0; i < kBufs; ++i) {
            hip_check("drop-in", hipHostMalloc(&buf_[i], kChunk, hipHostMallocDefault), "hipHostMalloc");
            hip_check("drop-in", hipEventCreateWithFlags(&ev_[i], hipEventDisableTiming), "hipEventCreate");
        }
    }
    struct Pending {
        char* dst = nullptr;
        size_t n = 0;
    };
    std::mutex mu_;
    void* buf_[kBufs] = {};
    hipEvent_t ev_[kBufs] = {};
    bool busy_[kBufs] = {};
    Pending out_[kBufs];
    int next_ = 0;
};

// n bytes of host memory into a new device buffer (staged; the source may
// be freed on return).
inline Buf upload_bytes(const void* src, size_t n) {
    auto buf = std::make_unique<DeviceBuffer>(n);
    if (n) Stager::instance().upload({{buf->get(), src, n}});
    return buf;
}

// A floating-point host tensor as fp32 values on the device; fp16 and bf16
// storage is widened exactly (the reference's read_tensor_float and
// tensor_row_value do the same): bf16 on the device (mft_convert), fp16 on
// the host.
inline Buf upload_f32(const TensorPtr& t, const char* who) {
    const int64_t n = t->numel();
    if (t->dtype() == kFloat32) return upload_bytes(t->data<float>(), static_cast<size_t>(n) * 4);
    if (t->dtype() == kBFloat16) {
        auto bits = upload_bytes(t->data<uint16_t>(), static_cast<size_t>(n) * 2);
        auto buf = std::make_unique<DeviceBuffer>(static_cast<size_t>(n) * 4);
        mft_check(who, mft_convert(bits->get(), MFT_BF16, buf->get(), MFT_F32, n, stream()));
        return buf;  // bits goes back to the pool; later users of it are ordered after the convert
    }
    if (t->dtype() != kFloat16)
        throw std::runtime_error(std::string(who) + ": expected floating-point tensor storage, got " +
                                 DTypeUtils::to_string(t->dtype()));
    std::vector<float> v(static_cast<size_t>(n));
    const uint16_t* bits = t->data<uint16_t>();
    for (int64_t i = 0; i < n; ++i) v[static_cast<size_t>(i)] = fp16_bits_to_float32(bits[i]);
    return upload_bytes(v.data(), v.size() * 4);  // staged: v may go on return
}

// Pinned host memory for the adapters' result tensors, so results go from
// the device into them by DMA alone: a result tensor wraps a pinned block
// (the reference's wrapping constructor, core/tensor.h:99-111, which never
// frees the memory), and the block returns to the pool once the tensor is
// gone (checked on the next request).  The reference's tensors never share
// memory between objects (reshape and view copy, core/tensor.cpp:266-292;
// copies allocate their own), so a block is free exactly when its tensor has
// been destroyed.  At most kCap bytes are held; past that, results take the
// reference's own allocation and a staged copy.
class PinnedPool {
public:
    static PinnedPool& instance() {
        static PinnedPool* p = new PinnedPool();  // never destroyed: HIP may be torn down first
        return *p;
    }

    // A new fp32 host tensor of `shape` on a pinned block (contents not
    // initialised), or nullptr when the pool is full.
    TensorPtr tensor(const std::vector<int64_t>& shape) {
        int64_t n = 1;
        for (int64_t x : shape) n *= x;
        if (n <= 0) return nullptr;
        const size_t cls = DevicePool::size_class(static_cast<size_t>(n) * 4);
        std::lock_guard<std::mutex> lock(mu_);
        reclaim_locked();
        void* p = nullptr;
        auto& fl = free_[cls];
        if (!fl.empty()) {
            p = fl.back();
            fl.pop_back();
        } else {
            if (held_ + cls > kCap) return nullptr;
            if (hipHostMalloc(&p, cls, hipHostMallocDefault) != hipSuccess) {
                (void)hipGetLastError();
                return nullptr;
            }
            held_ += cls;
        }
        TensorPtr t;
        try {
            t = std::make_shared<Tensor>(shape, p, kFloat32, kCPU, true);
        } catch (...) {
            free_[cls].push_back(p);
            throw;
        }
        live_.push_back({t, p, cls});
        return t;
    }

    size_t held_bytes() {
        std::lock_guard<std::mutex> lock(mu_);
        return held_;
    }

private:
    static constexpr size_t kCap = size_t(1) << 30;
    struct Lease {
        std::weak_ptr<Tensor> owner;
        void* block;
        size_t cls;
    };
    void reclaim_locked() {
        size_t k = 0;
        for (Lease& l : live_) {
            if (l.owner.expired()) free_[l.cls].push_back(l.block);
            else live_[k++] = std::move(l);
        }
        live_.resize(k);
    }
    std::mutex mu_;
    std::vector<Lease> live_;
    std::unordered_map<size_t, std::vector<void*>> free_;
    size_t held_ = 0;
};

// fp32 device values into new host tensors of the given shapes, after the
// work already on stream(); the tensors are ready on return.  Each goes by
// DMA into a pinned result tensor (PinnedPool), else into a tensor of the
// reference's allocation through the staged pipeline.
struct F32Out {
    const DeviceBuffer* src;
    const std::vector<int64_t>* shape;
};
inline std::vector<TensorPtr> download_f32_all(const std::vector<F32Out>& items) {
    std::vector<TensorPtr> out;
    std::vector<Segment> segs;
    bool direct = false;
    for (const F32Out& it : items) {
        TensorPtr t = PinnedPool::instance().tensor(*it.shape);
        const bool pinned = t != nullptr;
        if (!pinned) t = zeros(*it.shape, kFloat32, kCPU);
        const size_t n = static_cast<size_t>(t->numel()) * 4;
        if (pinned) {
            hip_check("drop-in", hipMemcpyAsync(t->data<float>(), it.src->get(), n, hipMemcpyDeviceToHost, stream()),
                      "copy to host");
            direct = true;
        } else {
            segs.push_back({t->data<float>(), it.src->get(), n});
        }
        out.push_back(std::move(t));
    }
    if (!segs.empty()) Stager::instance().download(segs);
    if (direct) hip_check("drop-in", hipStreamSynchronize(stream()), "synchronize");
    return out;
}

inline TensorPtr download_f32(const DeviceBuffer& src, const std::vector<int64_t>& shape) {
    return download_f32_all({{&src, &shape}})[0];
}

}  // namespace dropin
}  // namespace ops

#endif  // MFT_DROPIN_DEVICE_H
