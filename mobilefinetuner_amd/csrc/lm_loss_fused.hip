// Streaming LM cross-entropy forward with the logits GEMM and the row
// statistics fused (bf16 hidden and weight, H a multiple of 64): the [N, V]
// logits of ops::streaming_lm_cross_entropy (core/lm_loss.cpp:384-481) are
// never written, not even a vocabulary chunk at a time.
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
constexpr int kCfBK = 64;     // k per pipeline stage
constexpr int kCfThreads = 512;
constexpr int kCfTileElems = kCfRows * kCfBK;  // one [256 x 64] bf16 tile (32 KiB)
typedef TileDma<kCfBK, kCfRows, kCfThreads, SWZ_ROW> CfDma;

// A zero accumulator the compiler cannot see as a constant: a builtin MFMA
// chain that starts from a literal zero may get result registers that
// overlap its operands (see mfma_v_first).
__device__ __forceinline__ f32x16 zero_acc() {
    f32x16 z = zero16();
    asm volatile("" : "+v"(z));
    return z;
}

// Byte offset of row r's 16-byte chunk c in a swizzled [256 x 64] tile.
__device__ __forceinline__ uint32_t cf_off(int r, int c) {
    return (uint32_t)r * (kCfBK * 2) + 16u * (uint32_t)(c ^ swz_row<kCfBK / 8>(r));
}

template <bool FAST>
__global__ __launch_bounds__(kCfThreads) void ce_fused_fwd(CeFusedArgs a) {
    // [W tile 0][W tile 1][hidden tile 0][hidden tile 1]
    __shared__ __attribute__((aligned(1024))) bf16 smem[4 * kCfTileElems];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, hh = lane >> 5;
    const int wv = w & 1, wn = w >> 1;
    const int blk = xcd_block((int)blockIdx.x, (int)gridDim.x);
    const int range = blk / a.nb_pos, pb = blk % a.nb_pos;
    const int64_t p0 = (int64_t)pb * kCfRows;
    const int t0 = range * a.tiles_per_range, t1 = min(t0 + a.tiles_per_range, a.ntiles_v);
    const int KS = a.H / kCfBK;
    const int total = (t1 - t0) * KS;  // pipeline stages of this workgroup (>= 1: ranges are never empty)

    // This lane's two positions and their target labels (INT_MIN: none).
    int64_t pos[2];
    int y[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        pos[nt] = p0 + 64 * wn + 32 * nt + n;
        y[nt] = INT_MIN;
        if (pos[nt] < a.N && (pos[nt] % a.S) + 1 < a.S) {
            const int lab = a.labels[pos[nt] + 1];
            if (lab != a.ignore) y[nt] = lab;
        }
    }

    CfDma dw, dh;
    dw.init(lane, wave_id(), a.H);
    dh.init(lane, wave_id(), a.H);
    const uint32_t sbase = lds_addr(smem);
    auto issue = [&](int g) {
        const int t = t0 + g / KS, k0 = (g % KS) * kCfBK, b = g & 1;
        const bf16* W = static_cast<const bf16*>(a.weight) + k0;
        const bf16* Hd = static_cast<const bf16*>(a.hidden) + k0;
#pragma unroll
        for (int j = 0; j < CfDma::PER; ++j) {
            issue_tile_j<FAST, kCfBK, kCfRows, kCfThreads, SWZ_ROW>(dw, W, t * kCfRows, (int)a.V, kCfBK, a.H,
                                                                     smem + b * kCfTileElems,
                                                                     sbase + 2u * (uint32_t)(b * kCfTileElems), j);
            issue_tile_j<FAST, kCfBK, kCfRows, kCfThreads, SWZ_ROW>(
                dh, Hd, (int)p0, (int)a.N, kCfBK, a.H, smem + (2 + b) * kCfTileElems,
                sbase + 2u * (uint32_t)((2 + b) * kCfTileElems), j);
        }
    };

    // Per-lane LDS read offsets (bytes, within a tile) of k-step c's chunk
    // 2c + hh: A = vocabulary rows 128 wv + 32 mt + n, B = positions
    // 64 wn + 32 nt + n.  swz_row depends on the row's bits 1..3 only, so
    // the rows' 32-row bases leave it unchanged.
    uint32_t ro[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) ro[c] = cf_off(n, 2 * c + hh);
    const uint32_t a_base = (uint32_t)(128 * wv) * (kCfBK * 2), b_base = (uint32_t)(64 * wn) * (kCfBK * 2);
    constexpr uint32_t kMt = 32u * (kCfBK * 2);  // bytes of 32 tile rows

    f32x16 acc[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = zero_acc();
    float m_run[2] = {-INFINITY, -INFINITY}, s_run[2] = {0.f, 0.f};

    issue(0);
    for (int g = 0; g < total; ++g) {
        const int b = g & 1;
        // Stage g has landed in every wave's share; every wave is done with
        // the buffers stage g + 1 streams into.
        wait_vmcnt<0>();
        lds_barrier();
        if (g + 1 < total) issue(g + 1);
        const char* At = reinterpret_cast<const char*>(smem + b * kCfTileElems) + a_base;
        const char* Bt = reinterpret_cast<const char*>(smem + (2 + b) * kCfTileElems) + b_base;
        // Four k-steps, each six operand reads and eight MFMAs; the reads of
        // step c + 1 are issued before the MFMAs of step c (pinned below), so
        // two steps' operands are live at most.
        struct Ops {
            bf16x8 a[4], b[2];
        };
        auto read = [&](int c) {
            Ops o;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) o.a[mt] = *reinterpret_cast<const bf16x8*>(At + mt * kMt + ro[c]);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) o.b[nt] = *reinterpret_cast<const bf16x8*>(Bt + nt * kMt + ro[c]);
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
        if (g % KS != KS - 1) continue;

        // The tile's logits are complete: fold them into the running pairs.
        const int64_t vw = (int64_t)(t0 + g / KS) * kCfRows + 128 * wv;  // this wave's first vocabulary row
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
            mx = fmaxf(mx, other_half(mx));
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
                    for (int r = 0; r < 16; ++r) acc[mt][nt][r] = __expf(acc[mt][nt][r] - m_new);
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
    // The two half-waves hold the same max and halves of the sum.
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float s = s_run[nt] + other_half(s_run[nt]);
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

bool ce_fused_supported(int64_t H, bool bf16) { return bf16 && H >= kCfBK && H % kCfBK == 0; }

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
    if (f.N % kCfRows == 0 && f.V % kCfRows == 0)
        hipLaunchKernelGGL(ce_fused_fwd<true>, grid, dim3(kCfThreads), 0, st, f);
    else
        hipLaunchKernelGGL(ce_fused_fwd<false>, grid, dim3(kCfThreads), 0, st, f);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(ce_fused_merge, dim3((unsigned)((f.N + 255) / 256)), dim3(256), 0, st, f, a.run_m, a.run_s);
    return hipGetLastError();
}

}  // namespace mft
