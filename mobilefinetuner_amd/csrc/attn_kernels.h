// Host-visible launchers of the attention kernels (implemented in
// attn_fwd.hip, attn_bwd.hip, repeat_kv.hip; called by attn_capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_geometry.h"

namespace mft {

// Element strides of a [B, H, S, D] operand's batch, head and sequence
// dimensions; the head dim is contiguous.  Element (b, h, s, d) lives at
// b * b_ + h * h_ + s * s_ + d.  Offsets inside one (b, h) block fit in 32
// bits (checked by the C ABI), so the row stride is an int.
struct Strides {
    int64_t b, h;
    int s;
    __host__ __device__ int64_t at(int64_t bi, int64_t hi) const { return bi * b + hi * h; }
};

// An additive mask operand (mask mode; see mft_mask in include/mft/attention.h):
// element (b, h, i, j) - batch, query head, query row, key - at
// p[b*sb + h*sh + i*si + j*sj], fp32; p null = none.  Zero strides broadcast.
struct MaskView {
    const float* p;
    int64_t sb, sh, si, sj;
    __host__ __device__ float at(int64_t b, int64_t h, int64_t i, int64_t j) const {
        return p[b * sb + h * sh + i * si + j * sj];
    }
};

// The score of (query row i, key j) of batch b, query head h in mask mode,
// with the reference's float operations in their order: dot * scale, replaced
// by -1e10 above the diagonal when causal (the no-grad operator,
// core/memory_efficient_attention.cpp:160-172), then + mask0 and + mask1 (the
// composite's mul then add, :29-38; the model graphs' base then padding mask,
// graph/gemma_model.cpp:494-499).  No fused multiply-add: the reference rounds
// each step.
__device__ __forceinline__ float mask_score(float dot, float scale, int causal, const MaskView& m0,
                                            const MaskView& m1, int b, int h, int i, int j) {
    float x = (causal && j > i) ? -1e10f : __fmul_rn(dot, scale);
    if (m0.p) x = __fadd_rn(x, m0.at(b, h, i, j));
    if (m1.p) x = __fadd_rn(x, m1.at(b, h, i, j));
    return x;
}

struct AttnShape {
    int64_t B, Hq, Hkv, S, D;
    float scale;   // resolved (> 0)
    bool causal;
    bool bf16;     // element type of q, k, v, o, dO
    int window;              // causal sliding window (keys), 0 = none; normalised: 0 < window < S
    const int32_t* kv_len;   // device [B] valid keys per batch (right padding), or null
    // Resolved layouts (contiguous [B, H, S, D] unless the caller gave strides).
    Strides q, k, v, o, dO, dq, dk, dv;
    bool contiguous;  // every operand contiguous [B, H, S, D]
    // Mask mode (mft_mask): additive masks, general kernels only, every key
    // visited (causal = the -1e10 replacement above the diagonal); lse holds
    // two floats per row (the row max of the scores, ln of the sum).
    MaskView m0, m1;
    bool masked;
};

// Tile geometry of one kernel variant, exposed so that the C ABI can size
// workspaces and tests can reason about grids.
int fwd_rows_per_block(const AttnShape& s);
int dkdv_keys_per_block(const AttnShape& s);
// Number of head groups the dK/dV pass is split into (1 = no partials).
int dkdv_splits(const AttnShape& s);
// The direct-to-LDS kernels with work units: bf16 with D % 8 == 0,
// 32 < D <= 256 and one K/V sequence stride, and fp32 with D % 4 == 0,
// 32 < D <= 256 (f32::fast_path).
bool bwd_fast_path(const AttnShape& s);

// Work decomposition of the bf16 fast backward.  Per (batch, kv head) the
// dK/dV iterations (128-key tile, query head, 32-row query block) and per
// (batch, query head) the dQ iterations (128-row query tile, 64-key tile) are
// cut into units of about equal cost (UnitSplit, attn_geometry.h), about one
// unit per CU in total, so the causal triangle no longer sets the critical
// path.  A tile touched by several units gets fp32 partials (at most
// kv_parts_max / q_parts_max slots) that REDUCE sums in slot order.
// The most partial slots one split tile may have: REDUCE and the forward
// combine keep a tile's slot list (and the combine its per-slot weights) in
// LDS arrays of this length.  The planners size units so that no tile goes
// past it; the C ABI rejects a shape whose plan would (MFT_ERR_UNSUPPORTED).
constexpr int kSplitMaxSlots = 64;
// Rows of a split tile that one workgroup of the merge kernels (REDUCE and
// the forward combine) takes: 16 KiB of fp32 row data per slot, so 16 rows
// at a padded head dim of 256, 32 at 128 and 64 below.  Each of its 256
// threads then sums four 16-byte chunks of the rows, and narrow heads do not
// pay one workgroup's fixed cost per 4 KiB.
__host__ __device__ inline int merge_rows(int64_t D) { return D > 128 ? 16 : D > 64 ? 32 : 64; }

// Compute units of the current device (cached; 256 when the query fails).
int device_cus();

struct BwdPlan {
    bool fast;        // the work-unit kernels (bwd_fast_path)
    UnitSplit kv, q;  // units per (batch, kv head) and per (batch, query head)
    int kv_parts_max, q_parts_max;
};

// Costs of the unit splits (UnitSplit): an iteration's and a tile's extra
// (its rows loaded, its outputs or partial stored, the pipeline restarted),
// from per-unit cycle counts of the D = 256 kernels.  Backward iterations
// are priced against each other: a dK/dV one (32 rows x 128 keys, four
// products) 2, a dQ one (128 rows x 64 keys, three products) 3, in tenths
// for bf16 (20 and 30).  At D = 256 in bf16 a dK/dV iteration is priced 22:
// the dK/dV units then end with the dQ units (a sweep of 18-26 against 30
// measured C5 and C4 1.1% and 2.8% faster at 22, C3 at D = 64 best at
// 20-21).  fp32 keeps 2 and 3 (the planner's search steps are relative to
// the costs' scale, and the fp32 plans measured best at that scale).  The
// tile costs were measured at D = 256 only; narrower heads split by
// iteration count (tile cost 0), which measured faster there than the
// D = 256 costs.
constexpr int kFwdIterCost = 1;
inline int kv_iter_cost(int64_t D, bool bf16) { return bf16 ? (D >= 256 ? 22 : 20) : 2; }
inline int q_iter_cost(bool bf16) { return bf16 ? 30 : 3; }
inline int fwd_tile_cost(int64_t D) { return D >= 256 ? 2 : 0; }
inline int kv_tile_cost(int64_t D) { return D >= 256 ? 110 : 0; }
inline int q_tile_cost(int64_t D) { return D >= 256 ? 130 : 0; }
// fp32 iterations take about 16 times as long as bf16 ones (the fp32 MFMA
// rate), so a tile's fixed costs are left out for fp32.
inline int fwd_tile_cost(const AttnShape& s) { return s.bf16 ? fwd_tile_cost(s.D) : 0; }
inline int kv_iter_cost(const AttnShape& s) { return kv_iter_cost(s.D, s.bf16); }
inline int q_iter_cost(const AttnShape& s) { return q_iter_cost(s.bf16); }
inline int kv_tile_cost(const AttnShape& s) { return s.bf16 ? kv_tile_cost(s.D) : 0; }
inline int q_tile_cost(const AttnShape& s) { return s.bf16 ? q_tile_cost(s.D) : 0; }
// The fewest iterations the planners give a unit: backward units 4, forward
// units 2.  A forward unit's fixed costs (its Q rows, a partial tile) are
// smaller; at C4 (B 4, Hq 4, S 1024, D 256) 2 gives 16 units per (batch,
// head) instead of 11 and a 1.5 us shorter forward, and no other config
// moved (1, 2 and 4 measured for each role on C1-C5).
constexpr int kMinUnitIters = 4, kMinFwdUnitIters = 2;
// The plan of one backward call, computed once per call and passed to the
// workspace layout and the launches.
BwdPlan plan_bwd_fast(const AttnShape& s);

// Backward workspace layout in bytes: [delta or row-stat blocks][dK/dV
// partials][dQ partials][masked-row terms (key padding only)]; each region
// 256-byte aligned.
struct BwdLayout {
    size_t stats, kv_part, q_part, masked, total;
};
BwdLayout bwd_layout(const AttnShape& s, const BwdPlan& p);


// Workgroups of the bf16 fast kernels that one CU holds at once, which the
// planners size their launches for.  Registers decide it (LDS allows more):
// the forward needs at most 256 per lane up to D = 128 and the backward up
// to D = 64, so two workgroups - two waves per SIMD - share a CU there; the
// wider kernels keep one wave per SIMD.
inline int fwd_wgs_per_cu(int64_t D) { return D <= 128 ? 2 : 1; }
inline int bwd_wgs_per_cu(int64_t D) { return D <= 64 ? 2 : 1; }

// fp32 fast path (attn_f32_fast.h): fp32 operands with D % 4 == 0 and
// 32 < D <= 256 run the same work units, each unit as kF32Halves workgroups
// (one per 64-row or 64-key half of its 128-row tiles).  Registers decide
// how many share a CU as for bf16 (the forward fits 256 per lane up to
// D = 128, the backward up to D = 64; LDS, 128 KiB at D = 256, allows as many).
namespace f32 {
bool fast_path(const AttnShape& s);
}
constexpr int kF32Halves = 2;
// Units a launch of the fast forward / backward holds at once (one round).
inline int64_t fwd_unit_slots(const AttnShape& s) {
    return (int64_t)device_cus() * fwd_wgs_per_cu(s.D) / (s.bf16 ? 1 : kF32Halves);
}
inline int64_t bwd_unit_slots(const AttnShape& s) {
    return (int64_t)device_cus() * bwd_wgs_per_cu(s.D) / (s.bf16 ? 1 : kF32Halves);
}

// Balanced forward (bf16 fast path): per (batch, head) the iterations
// (128-row query tile, 64-key tile) are cut into units of about equal cost
// (UnitSplit, attn_geometry.h); a query tile split across units leaves fp32
// partials in the units' slots (split_slot).
struct FwdPlan {
    bool balanced;  // the shape has a balanced launch (it takes a workspace)
    UnitSplit us;
    bool any_split;
    int parts_max;  // most slots of one query tile
};
// Computed once per call and passed to the workspace size and the launch.
FwdPlan plan_fwd_split(const AttnShape& s);
// Forward workspace bytes (0 where the forward takes no workspace).  With a
// workspace of this size the forward uses the balanced launch; without one
// (NULL) it runs one workgroup per query tile.
size_t fwd_workspace_bytes(const AttnShape& s, const FwdPlan& p);

hipError_t launch_attn_fwd(const AttnShape& s, const FwdPlan& p, const void* q, const void* k, const void* v,
                           void* o, float* lse, void* workspace, hipStream_t st);

// Backward stages (bit mask, values of MFT_BWD_*): DELTA writes the per-row
// terms; DKDV and DQ compute the gradients (writing fp32 partials for split
// tiles); REDUCE sums the partials (and, with key padding, writes the
// gradient terms of rows that see no key).
enum {
    BWD_STAGE_DELTA = 1,
    BWD_STAGE_DKDV = 2,
    BWD_STAGE_REDUCE = 4,
    BWD_STAGE_DQ = 8,
    BWD_STAGE_MAIN = 10,
    BWD_STAGE_ALL = 15
};

// workspace: bwd_layout(s, p).total bytes.
hipError_t launch_attn_bwd(const AttnShape& s, const BwdPlan& p, const void* q, const void* k, const void* v,
                           const void* o, const void* dO, const float* lse, float* dq,
                           float* dk, float* dv, void* workspace, int stages, hipStream_t st);

// Rows that see no key (key padding; attn_masked_rows.hip): the forward
// writes their O after the main pass, the backward their dQ and dK/dV terms
// after REDUCE.  No-ops without key lengths.
size_t masked_rows_workspace_bytes(const AttnShape& s);
hipError_t launch_fwd_masked_rows(const AttnShape& s, const void* v, void* o, hipStream_t st);
hipError_t launch_bwd_masked_rows(const AttnShape& s, const void* q, const void* k, const void* v, const void* o,
                                  const void* dO, float* dq, float* dk, float* dv, void* scratch, hipStream_t st);

hipError_t launch_repeat_kv_fwd(const void* kv, void* out, int64_t B, int64_t Hkv, int64_t S,
                                int64_t D, int64_t r, int esize, hipStream_t st);
hipError_t launch_repeat_kv_bwd(const float* g, float* dkv, int64_t B, int64_t Hkv, int64_t S,
                                int64_t D, int64_t r, hipStream_t st);

}  // namespace mft
