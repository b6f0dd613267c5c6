#include "blas_util.h"

#include <string>

#include "capi_util.h"

namespace mft {
namespace blas {

namespace {
std::mutex g_mu;
rocblas_handle g_handle[64] = {};
}  // namespace

std::unique_lock<std::mutex> lock() { return std::unique_lock<std::mutex>(g_mu); }

mft_status bind(const char* who, hipStream_t stream, void* workspace, size_t workspace_bytes, rocblas_handle* h) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return capi::fail(MFT_ERR_HIP, std::string(who) + ": no current HIP device");
    if (!g_handle[dev] && rocblas_create_handle(&g_handle[dev]) != rocblas_status_success)
        return capi::fail(MFT_ERR_HIP, std::string(who) + ": rocblas_create_handle failed");
    if (rocblas_set_stream(g_handle[dev], stream) != rocblas_status_success ||
        rocblas_set_workspace(g_handle[dev], workspace, workspace_bytes) != rocblas_status_success)
        return capi::fail(MFT_ERR_HIP, std::string(who) + ": rocblas_set_stream / set_workspace failed");
    *h = g_handle[dev];
    return MFT_OK;
}

// rocBLAS is column-major: a row-major [R, C] matrix is its column-major
// [C, R] transpose, so C^T = op(B)^T op(A)^T is the call.
mft_status gemm_rm(const char* who, rocblas_handle h, int64_t M, int64_t N, int64_t K, float alpha, const void* A,
                   int64_t lda, bool ta, const void* B, int64_t ldb, bool tb, float beta, float* C, int64_t ldc,
                   bool bf16) {
    if (M == 0 || N == 0) return MFT_OK;
    const rocblas_datatype ab = bf16 ? rocblas_datatype_bf16_r : rocblas_datatype_f32_r;
    const rocblas_status st = rocblas_gemm_ex(
        h, tb ? rocblas_operation_transpose : rocblas_operation_none,
        ta ? rocblas_operation_transpose : rocblas_operation_none, (rocblas_int)N, (rocblas_int)M, (rocblas_int)K,
        &alpha, B, ab, (rocblas_int)ldb, A, ab, (rocblas_int)lda, &beta, C, rocblas_datatype_f32_r, (rocblas_int)ldc,
        C, rocblas_datatype_f32_r, (rocblas_int)ldc, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success)
        return capi::fail(MFT_ERR_HIP, std::string(who) + ": rocblas_gemm_ex failed: " + rocblas_status_to_string(st));
    return MFT_OK;
}

}  // namespace blas
}  // namespace mft
