// Host-visible launchers of the attention kernels (implemented in
// attn_fwd.hip, attn_bwd.hip, repeat_kv.hip; called by attn_capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mft {

struct AttnShape {
    int64_t B, Hq, Hkv, S, D;
    float scale;   // resolved (> 0)
    bool causal;
    bool bf16;     // element type of q, k, v, o, dO
};

// Tile geometry of one kernel variant, exposed so that the C ABI can size
// workspaces and tests can reason about grids.
int fwd_rows_per_block(const AttnShape& s);
int dkdv_keys_per_block(const AttnShape& s);
// Number of head groups the dK/dV pass is split into (1 = no partials).
int dkdv_splits(const AttnShape& s);
// bf16 with D % 8 == 0 and 32 < D <= 256 takes the direct-to-LDS kernels.
bool bwd_fast_path(const AttnShape& s);

hipError_t launch_attn_fwd(const AttnShape& s, const void* q, const void* k, const void* v,
                           void* o, float* lse, hipStream_t st);

// Backward stages (bit mask): DELTA writes delta; MAIN runs the dK/dV and dQ
// work (writing dK/dV partials when dkdv_splits(s) > 1); REDUCE sums them.
enum { BWD_STAGE_DELTA = 1, BWD_STAGE_MAIN = 2, BWD_STAGE_REDUCE = 4, BWD_STAGE_ALL = 7 };

// delta: [B, Hq, S] fp32 scratch.  part: 2 * splits * B*Hkv*S*D fp32 scratch
// (only used when dkdv_splits(s) > 1).
hipError_t launch_attn_bwd(const AttnShape& s, const void* q, const void* k, const void* v,
                           const void* o, const void* dO, const float* lse, float* dq,
                           float* dk, float* dv, float* delta, float* part, int stages,
                           hipStream_t st);

hipError_t launch_repeat_kv_fwd(const void* kv, void* out, int64_t B, int64_t Hkv, int64_t S,
                                int64_t D, int64_t r, int esize, hipStream_t st);
hipError_t launch_repeat_kv_bwd(const float* g, float* dkv, int64_t B, int64_t Hkv, int64_t S,
                                int64_t D, int64_t r, hipStream_t st);

}  // namespace mft
