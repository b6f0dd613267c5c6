// rocBLAS plumbing shared by the C ABI files that run library GEMMs
// (lm_loss_capi.cpp, lora_capi.cpp).
#pragma once

#include <rocblas/rocblas.h>

#include <cstddef>
#include <cstdint>
#include <mutex>

#include "mft/attention.h"

namespace mft {
namespace blas {

// Lock held around every use of a handle: one rocBLAS handle per device,
// created on first use and owned by rocBLAS until the process ends.
std::unique_lock<std::mutex> lock();

// Handle of the current device, bound to `stream` and to `workspace`
// (workspace_bytes of device memory from the caller); call under lock().
mft_status bind(const char* who, hipStream_t stream, void* workspace, size_t workspace_bytes, rocblas_handle* h);

// Row-major C[M, N] = alpha * op(A) . op(B) + beta * C, fp32 output and
// compute.  op(A) is [M, K] (A stored [M, K] with leading dimension lda, or
// [K, M] when ta); op(B) is [K, N] likewise.  A and B share one element type:
// fp32, or bf16 when bf16 is set.
mft_status gemm_rm(const char* who, rocblas_handle h, int64_t M, int64_t N, int64_t K, float alpha, const void* A,
                   int64_t lda, bool ta, const void* B, int64_t ldb, bool tb, float beta, float* C, int64_t ldc,
                   bool bf16);

}  // namespace blas
}  // namespace mft
