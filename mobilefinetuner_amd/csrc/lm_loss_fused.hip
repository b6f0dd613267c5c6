// Streaming LM cross-entropy with the logits GEMM fused into its consumers
// (bf16 hidden and weight, H a multiple of 64).  Forward: the row statistics
// in the GEMM's epilogue, so the [N, V] logits of
// ops::streaming_lm_cross_entropy (core/lm_loss.cpp:384-481) are never
// written, not even a vocabulary chunk at a time.  Backward
// (SelectedTokenLMCrossEntropyBackward, :165-266): the same kernel recomputes
// a vocabulary chunk's logits and writes G = (exp(z - lse) - onehot) * coeff
// in bf16 for the chunk's dh and dW GEMMs (grad_tile).  The LoRA layer's
// forward (nn/lora_linear.cpp:336-444) runs the same GEMM with W in the
// vocabulary's place and x in the positions', its rank-r update and bias in
// the epilogue (lora_tile).
//
// A workgroup (8 waves) owns 256 positions and a range of 256-row vocabulary
// tiles.  Per tile it computes Z^T = W_tile . hidden_tile^T on
// v_mfma_f32_32x32x16_bf16 (fp32 accumulation over the full H), with both
// operands streamed HBM -> LDS by direct loads into double buffers of
// [256 rows x 64 k] (row reads only: both operands are row-major with k
// contiguous).  Wave (wv, wn) holds vocabulary rows 128 wv .. + 127 of the
// tile for positions 64 wn .. + 63; a lane holds 16 vocabulary rows of one
// position per MFMA tile, so the tile's (max, sum of exp) per position is
// lane-local plus one swap with the other half-wave.  Each lane keeps the
// running (max, sum) of its two positions across the range's tiles and picks
// out its position's target logit when the label falls in its rows.  The
// range's pair per (position, vocabulary half) goes to the workspace;
// ce_fused_merge folds the pairs of every range, in range order and in
// double, into the running (max, sum) that ce_finalize turns into the LSE,
// the NLL and the loss, as for the chunked path.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>

#include "attn_common.h"
#include "attn_geometry.h"
#include "attn_kernels.h"
#include "lm_loss_kernels.h"

namespace mft {
namespace {

constexpr int kCfRows = 256;  // vocabulary rows and positions per workgroup tile
constexpr int kCfThreads = 512;

// A zero accumulator the compiler cannot see as a constant: a builtin MFMA
// chain that starts from a literal zero may get result registers that
// overlap its operands (see mfma_v_first).
__device__ __forceinline__ f32x16 zero_acc() {
    f32x16 z = zero16();
    asm volatile("" : "+v"(z));
    return z;
}

constexpr int kCfBK = 64;                       // k per pipeline stage
constexpr int kCfTile = kCfRows * kCfBK;        // elements of one [256 x 64] tile (32 KiB)
typedef TileDma<kCfBK, kCfRows, kCfThreads, SWZ_ROW> CfDma;

// Workgroup -> (vocabulary range, position block).  After xcd_block each
// XCD runs a contiguous run of logical indices; with xbr > 0 a run of
// xbr * xbp indices is an xbr x xbp rectangle of ranges x position blocks, so
// an XCD's workgroups, which move through their ranges at about the same
// pace, read each weight slice xbp times and each hidden slice xbr times
// through one L2 (per stage the XCD misses on xbr + xbp slices, not 2 xbr xbp).
__device__ __forceinline__ void cf_place(const CeFusedArgs& a, int blk, int* range, int* pb) {
    if (a.xbr > 0) {
        const int per = a.xbr * a.xbp, x = blk / per, in = blk % per, xr = a.ranges / a.xbr;
        *range = (x % xr) * a.xbr + in / a.xbp;
        *pb = (x / xr) * a.xbp + in % a.xbp;
    } else {
        *range = blk / a.nb_pos;
        *pb = blk % a.nb_pos;
    }
}

// The backward's epilogue of one tile: g = (exp(z - lse) - [v == label]) *
// coeff for the wave's 128 vocabulary rows (chunk-relative, from vw) and the
// lane's two positions, stored in bf16 to G[pos, v] (row stride ldg, a
// multiple of 8 elements).  Registers 4q .. 4q + 3 of an MFMA tile hold the
// four consecutive rows 8q + 4hh ..; one v_permlane32_swap per register pair
// gives the half-wave hh = 0 rows 16j .. 16j + 7 and hh = 1 rows 16j + 8 ..
// 16j + 15 (q = 2j, 2j + 1), so each lane stores 16 bytes and a position's 32
// bytes are contiguous.  The accumulators are cleared for the next tile.
template <bool FAST>
__device__ __forceinline__ void grad_tile(const CeFusedArgs& a, f32x16 (&acc)[4][2], int64_t vw, const int64_t* pos,
                                          const int* y, const float* lse2, const float* coeff, int hh) {
    // Row bound as an offset from this half-wave's first stored row
    // (vw + 8 hh), so that each group's row is a compile-time value.
    const int lim = (int)min<int64_t>(a.V - vw, 128) - 8 * hh;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const bool live = FAST || pos[nt] < a.N;
        bf16* grow = a.g + (live ? pos[nt] : 0) * a.ldg + vw + 8 * hh;
        const int64_t yr = (int64_t)y[nt] - vw - 4 * hh;
        const int yl = yr >= 0 && yr < 128 ? (int)yr : -1;  // label row less 4 hh, or none
        const float c = coeff[nt], ml = -lse2[nt];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            uint32_t pk[4][2];  // [q][pair]: bf16 pairs of rows 8q + 4hh + 0..3
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r0 = 32 * mt + 8 * q;  // row of register 4q, less 4 hh
                bf16x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = fast_exp2(fmaf(acc[mt][nt][4 * q + e], kLog2e, ml));
                    if (yl == r0 + e) x -= 1.0f;
                    o[e] = (bf16)(c != 0.f ? x * c : 0.f);
                }
                const uint2 u = __builtin_bit_cast(uint2, o);
                pk[q][0] = u.x;
                pk[q][1] = u.y;
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint4 o8;
                const auto s0 = __builtin_amdgcn_permlane32_swap(pk[2 * j][0], pk[2 * j + 1][0], false, false);
                const auto s1 = __builtin_amdgcn_permlane32_swap(pk[2 * j][1], pk[2 * j + 1][1], false, false);
                o8.x = s0[0];
                o8.y = s1[0];
                o8.z = s0[1];
                o8.w = s1[1];
                if (!live) continue;
                const int r0 = 32 * mt + 16 * j;  // first stored row, less 8 hh
                if (FAST || r0 + 8 <= lim) {
                    *reinterpret_cast<uint4*>(grow + r0) = o8;
                } else {
                    const bf16x8 v8 = __builtin_bit_cast(bf16x8, o8);
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        if (r0 + e < lim) grow[r0 + e] = v8[e];
                }
            }
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[mt][nt] = zero_acc();
    }
}

enum { kCeFwd = 0, kCeGrad = 1, kLoraFwd = 2 };

// The LoRA forward's epilogue of one tile: the rank-r update accumulated
// onto the GEMM's tile by v_mfma_f32_32x32x2_f32 (fp32 operands: lane (n, hh)
// gives B(row 32 mt + n, k) * scale and u(position 32 nt + n, k) for k = 2 kk
// + hh; the 32 x 32 output layout is the bf16 product's), then the bias, and
// y stored 16 bytes per register group (four consecutive output columns of
// one position).  Rows past out and positions past N are neither read nor
// stored.  The accumulators are cleared for the next tile.
template <bool FAST>
__device__ __forceinline__ void lora_tile(const CeFusedArgs& a, f32x16 (&acc)[4][2], int64_t vw, const int64_t* pos,
                                          int hh, int n) {
    const int ksteps = (a.rank + 1) / 2;
    for (int kk = 0; kk < ksteps; ++kk) {
        const int k = 2 * kk + hh;
        float ub[2], bb[4];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
            ub[nt] = (k < a.rank && (FAST || pos[nt] < a.N)) ? a.u[pos[nt] * a.ldu + k] : 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int64_t row = vw + 32 * mt + n;
            bb[mt] = (k < a.rank && (FAST || row < a.V)) ? a.lb[row * a.lb_so + k * a.lb_sk] * a.scale : 0.f;
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mfma_f32(bb[mt], ub[nt], acc[mt][nt]);
    }
    const int lim = (int)min<int64_t>(a.V - vw, 128) - 4 * hh;  // rows left, less this half-wave's offset
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const bool live = FAST || pos[nt] < a.N;
        float* yrow = a.y + (live ? pos[nt] : 0) * a.ldy + vw + 4 * hh;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r0 = 32 * mt + 8 * q;  // row of register 4q, less 4 hh
                f32x4 o{acc[mt][nt][4 * q], acc[mt][nt][4 * q + 1], acc[mt][nt][4 * q + 2], acc[mt][nt][4 * q + 3]};
                if (!live) continue;
                if (FAST || r0 + 4 <= lim) {
                    if (a.bias) o += *reinterpret_cast<const f32x4*>(a.bias + vw + 4 * hh + r0);
                    *reinterpret_cast<f32x4*>(yrow + r0) = o;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (r0 + e < lim) yrow[r0 + e] = o[e] + (a.bias ? a.bias[vw + 4 * hh + r0 + e] : 0.f);
                }
            }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) acc[mt][nt] = zero_acc();
    }
}

// MODE kCeFwd: the forward (row statistics and target logits).  kCeGrad: the
// backward's logits recompute for one vocabulary chunk, writing G =
// (exp(z - lse) - onehot(label)) * coeff in bf16 (ce_grad's arithmetic).
// kLoraFwd: the LoRA layer's forward, y = x W^T + scale u B^T + bias
// (lora_tile), W in the vocabulary's place and x in the positions'.
template <bool FAST, int MODE>
__global__ __launch_bounds__(kCfThreads) void ce_fused_kernel(CeFusedArgs a) {
    constexpr bool GRAD = MODE == kCeGrad, LORA = MODE == kLoraFwd;
    // [W tile 0][W tile 1][hidden tile 0][hidden tile 1]
    __shared__ __attribute__((aligned(1024))) bf16 smem[4 * kCfTile];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int wv = w & 1, wn = w >> 1;
    int range, pb;
    cf_place(a, xcd_block((int)blockIdx.x, (int)gridDim.x), &range, &pb);
    const int64_t p0 = (int64_t)pb * kCfRows;
    const int t0 = range * a.tiles_per_range, t1 = min(t0 + a.tiles_per_range, a.ntiles_v);
    const int KS = a.H / kCfBK;
    const int total = (t1 - t0) * KS;  // pipeline stages of this workgroup (>= 1: ranges are never empty)

    // This lane's two positions and their target labels (INT_MIN: none).
    // GRAD: labels relative to the chunk, the LSE times log2(e), and the
    // coefficient (0 for a position that scores nothing or whose label is
    // out of range, as ce_grad).
    int64_t pos[2];
    int y[2];
    float lse2[2] = {0.f, 0.f}, coeff[2] = {0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        pos[nt] = p0 + 64 * wn + 32 * nt + n;
        y[nt] = INT_MIN;
        if (!LORA && pos[nt] < a.N && (pos[nt] % a.S) + 1 < a.S) {
            const int lab = a.labels[pos[nt] + 1];
            if constexpr (GRAD) {
                if (lab != a.ignore && lab >= 0 && lab < a.vall) {
                    const long long cnt = *a.count;
                    const float outer = a.grad_loss ? a.grad_loss[0] : 1.f;
                    coeff[nt] = outer * (a.reduction == CE_MEAN ? (cnt > 0 ? 1.0f / (float)cnt : 0.f) : 1.f);
                    y[nt] = (int)(lab - a.v0);
                    lse2[nt] = a.lse_in[pos[nt]] * kLog2e;
                }
            } else {
                if (lab != a.ignore) y[nt] = lab;
            }
        }
    }

    CfDma dw, dh;
    dw.init(lane, wave_id(), a.H);
    dh.init(lane, wave_id(), a.H);
    const uint32_t sbase = lds_addr(smem);
    // The issue cursor: tile and k offset of the next stage to load.
    int it = t0, ik = 0;
    auto issue_next = [&](int buf) {
        const bf16* W = static_cast<const bf16*>(a.weight) + ik;
        const bf16* Hd = static_cast<const bf16*>(a.hidden) + ik;
#pragma unroll
        for (int j = 0; j < CfDma::PER; ++j) {
            issue_tile_j<FAST, kCfBK, kCfRows, kCfThreads, SWZ_ROW>(dw, W, it * kCfRows, (int)a.V, kCfBK, a.H,
                                                                     smem + buf * kCfTile,
                                                                     sbase + 2u * (uint32_t)(buf * kCfTile), j);
            issue_tile_j<FAST, kCfBK, kCfRows, kCfThreads, SWZ_ROW>(dh, Hd, (int)p0, (int)a.N, kCfBK, a.H,
                                                                     smem + (2 + buf) * kCfTile,
                                                                     sbase + 2u * (uint32_t)((2 + buf) * kCfTile), j);
        }
        ik += kCfBK;
        if (ik == a.H) {
            ik = 0;
            ++it;
        }
    };

    // Per-lane LDS byte offsets of k-step c's chunk 2c + hh (= 2c ^ hh ^
    // swz_row(n)) in buffer 0: A = vocabulary row 128 wv + n of the W tile,
    // B = position 64 wn + n of the hidden tile.  swz_row depends on row bits
    // 1..3 only, so the MFMA tiles' 32-row bases leave it unchanged and go
    // into the instructions' immediate offsets.
    constexpr uint32_t kRow = kCfBK * 2, kMt = 32 * kRow, kTileB = kCfTile * 2;
    uint32_t ro_a[4], ro_b[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t y16 = 16u * (uint32_t)((2 * c + hh) ^ swz_row<kCfBK / 8>(n));
        ro_a[c] = (uint32_t)(128 * wv + n) * kRow + y16;
        ro_b[c] = 2 * kTileB + (uint32_t)(64 * wn + n) * kRow + y16;
    }
    const char* lds = reinterpret_cast<const char*>(smem);

    f32x16 acc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = zero_acc();
    float m_run[2] = {-INFINITY, -INFINITY}, s_run[2] = {0.f, 0.f};

    issue_next(0);
    int ct = t0, ck = 0;  // tile and k offset of the stage being multiplied
    for (int g = 0; g < total; ++g) {
        // Stage g has landed in every wave's share; every wave is done with
        // the buffer stage g + 1 streams into (stage g - 1's).
        wait_vmcnt<0>();
        lds_barrier();
        if (g + 1 < total) issue_next((g + 1) & 1);
        // Four k-steps, each six operand reads and eight MFMAs; the reads of
        // step c + 1 are issued before the MFMAs of step c (pinned below), so
        // two steps' operands are live at most.
        const uint32_t boff = (uint32_t)(g & 1) * kTileB;
        struct Ops {
            bf16x8 a[4], b[2];
        };
        auto read = [&](int c) {
            Ops o;
            const char* pa = lds + (ro_a[c] + boff);
            const char* pb = lds + (ro_b[c] + boff);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) o.a[mt] = *reinterpret_cast<const bf16x8*>(pa + mt * kMt);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) o.b[nt] = *reinterpret_cast<const bf16x8*>(pb + nt * kMt);
            return o;
        };
        Ops cur = read(0);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            Ops nxt;
            if (c + 1 < 4) nxt = read(c + 1);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mfma_bf16(cur.a[mt], cur.b[nt], acc[mt][nt]);
            if (c + 1 < 4) cur = nxt;
        }
        pin_read_ahead<4, 1, 6, 8>();
        ck += kCfBK;
        if (ck != a.H) continue;
        ck = 0;
        const int64_t vw = (int64_t)ct * kCfRows + 128 * wv;  // this wave's first vocabulary row
        ++ct;
        if constexpr (GRAD) {
            grad_tile<FAST>(a, acc, vw, pos, y, lse2, coeff, hh);
            continue;
        }
        if constexpr (LORA) {
            lora_tile<FAST>(a, acc, vw, pos, hh, n);
            continue;
        }

        // The tile's logits are complete: fold them into the running pairs.
        const bool partial_v = vw + 128 > a.V;
        // rows of the wave's 128 at or past V, as a bound on the row within
        // the wave less this half-wave's offset (row_of_reg(r, hh) - 4 hh is
        // a compile-time value)
        const int lim = (int)min<int64_t>(a.V - vw, 128) - 4 * hh;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            if (partial_v) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (32 * mt + row_of_reg(r, 0) >= lim) acc[mt][nt][r] = -INFINITY;
            }
            float mx = -INFINITY;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[mt][nt][r]);
            mx = half_max(mx);
            // the target logit, when this lane holds it
            const int64_t rel = (int64_t)y[nt] - vw;
            if (rel >= 0 && rel < 128) {
                const int mt_t = (int)rel >> 5, rho = (int)rel & 31;
                if (((rho >> 2) & 1) == hh) {
                    const int r_t = 4 * (rho >> 3) + (rho & 3);
                    float z = 0.f;
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                        for (int r = 0; r < 16; ++r) z = (mt == mt_t && r == r_t) ? acc[mt][nt][r] : z;
                    a.tgt[pos[nt]] = z;
                }
            }
            // exp in place (the accumulators are cleared next), then summed
            const float m_new = fmaxf(m_run[nt], mx);
            if (m_new != -INFINITY) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int r = 0; r < 16; ++r)  // exp(z - m) as exp2(z log2 e - m log2 e), one fma
                        acc[mt][nt][r] = fast_exp2(fmaf(acc[mt][nt][r], kLog2e, -m_new * kLog2e));
                float s = m_run[nt] == -INFINITY ? 0.f : s_run[nt] * __expf(m_run[nt] - m_new);
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) s += acc[mt][nt][r];
                s_run[nt] = s;
                m_run[nt] = m_new;
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) acc[mt][nt] = zero_acc();
        }
    }
    wait_vmcnt<0>();
    if constexpr (GRAD || LORA) return;
    // The two half-waves hold the same max and halves of the sum.
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float s = half_sum(s_run[nt]);
        if (hh == 0 && pos[nt] < a.N)
            a.part[pos[nt] * a.nparts + 2 * range + wv] = make_float2(m_run[nt], s);
    }
}

// run_m[n], run_s[n] = the (max, sum) pairs of position n folded in part
// order, the sum in double.
__global__ __launch_bounds__(256) void ce_fused_merge(CeFusedArgs a, float* run_m, double* run_s) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= a.N) return;
    const float2* p = a.part + n * a.nparts;
    float m = -INFINITY;
    for (int i = 0; i < a.nparts; ++i) m = fmaxf(m, p[i].x);
    double s = 0.0;
    if (m != -INFINITY)
        for (int i = 0; i < a.nparts; ++i)
            if (p[i].x != -INFINITY) s += (double)p[i].y * exp((double)p[i].x - (double)m);
    run_m[n] = m;
    run_s[n] = s;
}

}  // namespace

bool ce_fused_supported(int64_t H, bool bf16) { return bf16 && H >= 64 && H % 64 == 0; }

CeFusedArgs ce_fused_plan(int64_t N, int64_t V, int64_t H) {
    CeFusedArgs f{};
    f.N = N;
    f.V = V;
    f.H = (int)H;
    f.nb_pos = (int)((N + kCfRows - 1) / kCfRows);
    f.ntiles_v = (int)((V + kCfRows - 1) / kCfRows);
    // About one workgroup per CU: vocabulary ranges x position blocks.
    int ranges = (int)std::max<int64_t>(1, (device_cus() + f.nb_pos - 1) / f.nb_pos);
    ranges = std::min({ranges, f.ntiles_v, kCeFusedMaxRanges});
    f.tiles_per_range = (f.ntiles_v + ranges - 1) / ranges;
    f.ranges = (f.ntiles_v + f.tiles_per_range - 1) / f.tiles_per_range;  // none empty
    f.nparts = 2 * f.ranges;
    // The XCD rectangle: each XCD's run (grid / 8 workgroups) split as xbr
    // ranges x xbp position blocks, xbr + xbp smallest; on a tie fewer
    // ranges (weight slices, which come from HBM; the hidden rows are small
    // enough to stay in the last-level cache).  None fits: xbr = 0, range-major.
    f.xbr = f.xbp = 0;
    const int grid = f.ranges * f.nb_pos;
    if (grid % kXcds == 0) {
        const int run = grid / kXcds;
        for (int br = 1; br <= std::min(run, f.ranges); ++br) {
            const int bp = run / br;
            if (run % br || f.ranges % br || f.nb_pos % bp) continue;
            if (f.xbr == 0 || br + bp < f.xbr + f.xbp) {
                f.xbr = br;
                f.xbp = bp;
            }
        }
    }
    return f;
}

hipError_t launch_ce_fused_fwd(const CeArgs& a, const CeFusedArgs& plan, const void* hidden, const void* weight,
                               float2* part, hipStream_t st) {
    CeFusedArgs f = plan;
    f.hidden = hidden;
    f.weight = weight;
    f.labels = a.labels;
    f.tgt = a.tgt;
    f.part = part;
    f.S = a.S;
    f.ignore = a.ignore;
    const dim3 grid((unsigned)(f.nb_pos * f.ranges));
    const bool fast = f.N % kCfRows == 0 && f.V % kCfRows == 0;
    if (fast)
        hipLaunchKernelGGL((ce_fused_kernel<true, kCeFwd>), grid, dim3(kCfThreads), 0, st, f);
    else
        hipLaunchKernelGGL((ce_fused_kernel<false, kCeFwd>), grid, dim3(kCfThreads), 0, st, f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(ce_fused_merge, dim3((unsigned)((f.N + 255) / 256)), dim3(256), 0, st, f, a.run_m, a.run_s);
    return hipGetLastError();
}

hipError_t launch_ce_fused_grad(const CeArgs& a, const CeFusedArgs& plan, const void* hidden, const void* weight_chunk,
                                int64_t v0, void* g, int64_t ldg, hipStream_t st) {
    CeFusedArgs f = plan;
    f.hidden = hidden;
    f.weight = weight_chunk;
    f.labels = a.labels;
    f.S = a.S;
    f.ignore = a.ignore;
    f.g = static_cast<bf16*>(g);
    f.ldg = ldg;
    f.v0 = v0;
    f.vall = a.V;
    f.lse_in = a.lse_in;
    f.count = a.count;
    f.grad_loss = a.grad_loss;
    f.reduction = a.reduction;
    const dim3 grid((unsigned)(f.nb_pos * f.ranges));
    if (f.N % kCfRows == 0 && f.V % kCfRows == 0)
        hipLaunchKernelGGL((ce_fused_kernel<true, kCeGrad>), grid, dim3(kCfThreads), 0, st, f);
    else
        hipLaunchKernelGGL((ce_fused_kernel<false, kCeGrad>), grid, dim3(kCfThreads), 0, st, f);
    return hipGetLastError();
}

hipError_t launch_lora_fused_fwd(const CeFusedArgs& f, hipStream_t st) {
    const dim3 grid((unsigned)(f.nb_pos * f.ranges));
    if (f.N % kCfRows == 0 && f.V % kCfRows == 0)
        hipLaunchKernelGGL((ce_fused_kernel<true, kLoraFwd>), grid, dim3(kCfThreads), 0, st, f);
    else
        hipLaunchKernelGGL((ce_fused_kernel<false, kLoraFwd>), grid, dim3(kCfThreads), 0, st, f);
    return hipGetLastError();
}

}  // namespace mft
