// Language-model cross-entropy kernels (C ABI in include/mft/lm_loss.h).
//
// Rows are the B*S positions; position (b, s) is scored against
// labels[b, s + 1] (core/lm_loss.cpp:28-47, 292-296), not at s = S - 1 nor
// when that label is ignore_index.  The dense path runs each pass over whole
// rows of V logits; the streaming path runs the same passes over one chunk
// of vocabulary columns at a time (the GEMM output), merging the row
// statistics across chunks.
//
//   ce_row_stats  one workgroup per row: the chunk's online (max, sum of
//                 exp(z - max)) merged into the row's running pair, and the
//                 target logit when the label falls in the chunk
//   ce_finalize   lse = max + log(sum) and nll = lse - z[label] per row, as
//                 core/lm_loss.cpp:305-312 (double logsumexp)
//   ce_reduce     scored-row count and the sum of nll in row order (double);
//                 MEAN divides by the count (NaN if zero), as :345-352
//   ce_grad       (exp(z - lse) - onehot(label)) * coeff, coeff = grad_loss *
//                 (1 / count for MEAN), as LMCrossEntropyBackward
//                 (:85-158): zero rows for unscored positions.
#include <hip/hip_runtime.h>

#include <cmath>

#include "attn_common.h"
#include "lm_loss_kernels.h"

namespace mft {
namespace {

constexpr int kCeThreads = 256;

__device__ __forceinline__ bool scored(const CeArgs& a, int64_t n, int* label) {
    const int64_t s = n % a.S;
    if (s + 1 >= a.S) return false;
    const int y = a.labels[n + 1];
    *label = y;
    return y != a.ignore;
}

template <typename T> __device__ __forceinline__ float to_f(T x) { return (float)x; }

// Block-wide (max, sum) merge of per-thread online pairs.
__device__ __forceinline__ void merge_pair(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;
    s = s * __expf(m - mn) + s2 * __expf(m2 - mn);
    m = mn;
}

// VEC consecutive elements of a row as floats (VEC * sizeof(T) <= 16 bytes).
template <typename T, int VEC> struct RowVec {
    typedef T raw __attribute__((ext_vector_type(VEC)));
    __device__ static void load(const T* p, float* x) {
        const raw r = *reinterpret_cast<const raw*>(p);
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[e] = (float)r[e];
    }
};
template <typename T> struct RowVec<T, 1> {
    __device__ static void load(const T* p, float* x) { x[0] = (float)*p; }
};

// Online (max, sum) update with VEC new values: one rescale per vector.
template <int VEC>
__device__ __forceinline__ void online_add(float& m, float& s, const float* x) {
    float vm = x[0];
#pragma unroll
    for (int e = 1; e < VEC; ++e) vm = fmaxf(vm, x[e]);
    if (vm == -INFINITY) return;  // exp(-inf) adds nothing
    if (vm > m) {
        s *= __expf(m - vm);
        m = vm;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += __expf(x[e] - m);
}

template <typename T, int VEC>
__global__ __launch_bounds__(kCeThreads) void ce_row_stats(CeArgs a, const T* z, int64_t ld, int64_t ncols,
                                                           int64_t v0, int first) {
    __shared__ float sm[kCeThreads / 64], ss[kCeThreads / 64];
    const int64_t n = blockIdx.x;
    int y = 0;
    if (!scored(a, n, &y) || y < 0 || y >= a.V) return;
    const T* row = z + n * ld;
    float m = -INFINITY, s = 0.f;
    const int64_t nvec = ncols / VEC;
    for (int64_t j = threadIdx.x; j < nvec; j += kCeThreads) {
        float x[VEC];
        RowVec<T, VEC>::load(row + j * VEC, x);
        online_add<VEC>(m, s, x);
    }
    for (int64_t v = nvec * VEC + threadIdx.x; v < ncols; v += kCeThreads) {
        float x[1] = {(float)row[v]};
        online_add<1>(m, s, x);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) merge_pair(m, s, __shfl_xor(m, o, 64), __shfl_xor(s, o, 64));
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sm[w] = m;
        ss[w] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float bm = sm[0], bs = ss[0];
        for (int k = 1; k < kCeThreads / 64; ++k) merge_pair(bm, bs, sm[k], ss[k]);
        // merge into the row's running pair (sum kept in double)
        if (first || a.run_m[n] == -INFINITY) {
            a.run_m[n] = bm;
            a.run_s[n] = (double)bs;
        } else if (bm != -INFINITY) {
            const float om = a.run_m[n];
            const float mn = fmaxf(om, bm);
            a.run_s[n] = a.run_s[n] * exp((double)om - (double)mn) + (double)bs * exp((double)bm - (double)mn);
            a.run_m[n] = mn;
        }
        if (y >= v0 && y < v0 + ncols) a.tgt[n] = to_f(row[y - v0]);
    }
}

__global__ __launch_bounds__(kCeThreads) void ce_finalize(CeArgs a) {
    const int64_t n = (int64_t)blockIdx.x * kCeThreads + threadIdx.x;
    if (n >= a.N) return;
    int y = 0;
    double nll = 0.0;
    float lse = 0.f;
    if (scored(a, n, &y)) {
        if (y < 0 || y >= a.V) {
            if (a.status) *a.status = 1;  // the reference throws "label out of range"
            nll = NAN;
        } else {
            const double l = (double)a.run_m[n] + log(a.run_s[n]);
            nll = l - (double)a.tgt[n];
            lse = (float)l;
        }
    }
    a.nll[n] = nll;
    if (a.lse) a.lse[n] = lse;
    if (a.reduction == CE_NONE && a.loss) a.loss[n] = (float)nll;
}

// One workgroup: count of scored rows (and, with nll, the loss) in row order.
__global__ __launch_bounds__(kCeThreads) void ce_reduce(CeArgs a, int write_loss) {
    __shared__ double ps[kCeThreads];
    __shared__ long long pc[kCeThreads];
    // each thread a contiguous block of rows, so the order of the sum is the row order
    const int64_t per = (a.N + kCeThreads - 1) / kCeThreads;
    const int64_t r0 = threadIdx.x * per, r1 = min(a.N, r0 + per);
    double sum = 0.0;
    long long cnt = 0;
    for (int64_t n = r0; n < r1; ++n) {
        int y = 0;
        if (scored(a, n, &y)) {
            ++cnt;
            if (write_loss) sum += a.nll[n];
        }
    }
    ps[threadIdx.x] = sum;
    pc[threadIdx.x] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        long long c = 0;
        for (int k = 0; k < kCeThreads; ++k) {
            t += ps[k];
            c += pc[k];
        }
        *a.count = c;
        if (write_loss && a.reduction != CE_NONE && a.loss) {
            if (a.reduction == CE_SUM)
                a.loss[0] = (float)t;
            else
                a.loss[0] = c > 0 ? (float)(t / (double)c) : NAN;
        }
    }
}

template <typename OutT, int VEC> struct OutVec {
    typedef OutT raw __attribute__((ext_vector_type(VEC)));
    __device__ static void store(OutT* p, const float* x) {
        raw r;
#pragma unroll
        for (int e = 0; e < VEC; ++e) r[e] = (OutT)x[e];
        *reinterpret_cast<raw*>(p) = r;
    }
};
template <typename OutT> struct OutVec<OutT, 1> {
    __device__ static void store(OutT* p, const float* x) { *p = (OutT)x[0]; }
};

template <typename T, typename OutT, int VEC>
__global__ __launch_bounds__(kCeThreads) void ce_grad(CeArgs a, const T* z, int64_t ld, int64_t ncols, int64_t v0,
                                                      OutT* g, int64_t ldg) {
    const int64_t n = blockIdx.x;
    OutT* grow = g + n * ldg;
    int y = 0;
    const bool on = scored(a, n, &y) && y >= 0 && y < a.V;
    float coeff = 0.f;
    if (on) {
        const float outer = a.grad_loss ? (a.reduction == CE_NONE ? a.grad_loss[n] : a.grad_loss[0]) : 1.f;
        const long long c = *a.count;
        const float base = a.reduction == CE_MEAN ? (c > 0 ? 1.0f / (float)c : 0.f) : 1.f;
        coeff = outer * base;
    }
    const int64_t nvec = ncols / VEC;
    if (!on || coeff == 0.f) {
        float zero[VEC] = {};
        for (int64_t j = threadIdx.x; j < nvec; j += kCeThreads) OutVec<OutT, VEC>::store(grow + j * VEC, zero);
        for (int64_t v = nvec * VEC + threadIdx.x; v < ncols; v += kCeThreads) grow[v] = (OutT)0.f;
        return;
    }
    const float l = a.lse_in[n];
    const T* row = z + n * ld;
    for (int64_t j = threadIdx.x; j < nvec; j += kCeThreads) {
        float x[VEC];
        RowVec<T, VEC>::load(row + j * VEC, x);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            float p = __expf(x[e] - l);
            if (v0 + j * VEC + e == y) p -= 1.0f;
            x[e] = p * coeff;
        }
        OutVec<OutT, VEC>::store(grow + j * VEC, x);
    }
    for (int64_t v = nvec * VEC + threadIdx.x; v < ncols; v += kCeThreads) {
        float p = __expf(to_f(row[v]) - l);
        if (v0 + v == y) p -= 1.0f;
        grow[v] = (OutT)(p * coeff);
    }
}

// Vector width (elements) for rows of type T at row stride ld: 16 bytes when
// the base and every row start are 16-byte aligned, else one element.
template <typename T> int vec_for(const void* base, int64_t ld) {
    const int w = 16 / (int)sizeof(T);
    return ((reinterpret_cast<uintptr_t>(base) & 15u) == 0 && ld % w == 0) ? w : 1;
}

}  // namespace

hipError_t launch_ce_stats(const CeArgs& a, const void* z, bool z_bf16, int64_t ld, int64_t ncols, int64_t v0,
                           bool first, hipStream_t st) {
    const dim3 grid((unsigned)a.N), blk(kCeThreads);
    if (z_bf16) {
        if (vec_for<bf16>(z, ld) == 8)
            hipLaunchKernelGGL((ce_row_stats<bf16, 8>), grid, blk, 0, st, a, (const bf16*)z, ld, ncols, v0, (int)first);
        else
            hipLaunchKernelGGL((ce_row_stats<bf16, 1>), grid, blk, 0, st, a, (const bf16*)z, ld, ncols, v0, (int)first);
    } else {
        if (vec_for<float>(z, ld) == 4)
            hipLaunchKernelGGL((ce_row_stats<float, 4>), grid, blk, 0, st, a, (const float*)z, ld, ncols, v0,
                               (int)first);
        else
            hipLaunchKernelGGL((ce_row_stats<float, 1>), grid, blk, 0, st, a, (const float*)z, ld, ncols, v0,
                               (int)first);
    }
    return hipGetLastError();
}

hipError_t launch_ce_finalize(const CeArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(ce_finalize, dim3((unsigned)((a.N + kCeThreads - 1) / kCeThreads)), dim3(kCeThreads), 0, st,
                       a);
    hipLaunchKernelGGL(ce_reduce, dim3(1), dim3(kCeThreads), 0, st, a, 1);
    return hipGetLastError();
}

hipError_t launch_ce_count(const CeArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(ce_reduce, dim3(1), dim3(kCeThreads), 0, st, a, 0);
    return hipGetLastError();
}

hipError_t launch_ce_grad(const CeArgs& a, const void* z, bool z_bf16, int64_t ld, int64_t ncols, int64_t v0, void* g,
                          bool g_bf16, int64_t ldg, hipStream_t st) {
    const dim3 grid((unsigned)a.N), blk(kCeThreads);
    // 4 elements per lane when input and output rows allow it (fp32 16 B, bf16 8 B)
    const bool v4 = (reinterpret_cast<uintptr_t>(z) % (4 * (z_bf16 ? 2 : 4))) == 0 && ld % 4 == 0 &&
                    (reinterpret_cast<uintptr_t>(g) % (4 * (g_bf16 ? 2 : 4))) == 0 && ldg % 4 == 0;
    if (z_bf16 && !g_bf16) {
        if (v4)
            hipLaunchKernelGGL((ce_grad<bf16, float, 4>), grid, blk, 0, st, a, (const bf16*)z, ld, ncols, v0,
                               (float*)g, ldg);
        else
            hipLaunchKernelGGL((ce_grad<bf16, float, 1>), grid, blk, 0, st, a, (const bf16*)z, ld, ncols, v0,
                               (float*)g, ldg);
    } else if (!z_bf16 && !g_bf16) {
        if (v4)
            hipLaunchKernelGGL((ce_grad<float, float, 4>), grid, blk, 0, st, a, (const float*)z, ld, ncols, v0,
                               (float*)g, ldg);
        else
            hipLaunchKernelGGL((ce_grad<float, float, 1>), grid, blk, 0, st, a, (const float*)z, ld, ncols, v0,
                               (float*)g, ldg);
    } else if (!z_bf16 && g_bf16) {
        if (v4)
            hipLaunchKernelGGL((ce_grad<float, bf16, 4>), grid, blk, 0, st, a, (const float*)z, ld, ncols, v0,
                               (bf16*)g, ldg);
        else
            hipLaunchKernelGGL((ce_grad<float, bf16, 1>), grid, blk, 0, st, a, (const float*)z, ld, ncols, v0,
                               (bf16*)g, ldg);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mft
