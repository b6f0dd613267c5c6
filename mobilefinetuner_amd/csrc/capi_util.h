// Shared helpers of the C ABI entry points (defined in attn_capi.cpp).
#pragma once

#include <string>

#include "attn_kernels.h"
#include "mft/attention.h"

namespace mft {
namespace capi {

// Records the thread-local message returned by mft_last_error() and returns st.
mft_status fail(mft_status st, const std::string& msg);

// Validates and resolves one operand layout (all-zero strides = contiguous
// [B, H, S, D]); dense_out tells whether the result is the contiguous layout.
// Rules: positive strides that are multiples of 16 bytes, a sequence stride of
// at least D, and one (batch, head) block under 2^31 elements.
mft_status resolve_layout(const mft_strides& st, int64_t H, int64_t S, int64_t D, int64_t esz, const char* who,
                          const char* name, Strides* out, bool* dense_out);

bool aligned16(const void* p);

mft_status hip_status(hipError_t e, const char* what);

}  // namespace capi
}  // namespace mft
