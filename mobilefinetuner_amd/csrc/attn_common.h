// Shared device definitions for the gfx950 attention kernels.
//
// MFMA shapes used (CDNA4, 64-lane waves):
//   v_mfma_f32_32x32x16_bf16 : A,B = 8 bf16 per lane, C = 16 fp32 per lane
//   v_mfma_f32_32x32x2_f32   : A,B = 1 fp32 per lane,  C = 16 fp32 per lane
// Lane l = 32*hh + n (n = l % 32, hh = l / 32).
//   A operand: lane holds row i = n, reduction slots owned by half hh.
//   B operand: lane holds column n, the same reduction slots (half hh).
//   C (32x32): lane holds column n, rows 8*(r/4) + 4*hh + (r%4), r = 0..15.
// A reduction index only has to be assigned to the same (hh, slot) in A and
// B; the kernels exploit that to feed the C registers of one product
// straight into the B operand of the next (see row_of_reg()).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mft {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef __bf16 bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Online softmax: headroom (log2 units) before the running max is moved.
constexpr float kLazyRescale = 8.0f;

// Element traits: a "vec" is one 16-byte chunk of a row.
template <typename T> struct Elt;
template <> struct Elt<float> {
    static constexpr int VEC = 4;
    typedef f32x4 vec;
};
template <> struct Elt<bf16> {
    static constexpr int VEC = 8;
    typedef bf16x8 vec;
};

// C-register r of a 32x32 accumulator on lane half hh -> row/column index
// (0..31) along the accumulator's M dimension.
__device__ __forceinline__ constexpr int row_of_reg(int r, int hh) {
    return 8 * (r >> 2) + 4 * hh + (r & 3);
}

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// One 16-byte chunk pair of a dot product: bf16 = one 32x32x16 MFMA over the
// 8 values each half holds; fp32 = four 32x32x2 MFMAs, one per value.
__device__ __forceinline__ f32x16 mfma_chunk(bf16x8 a, bf16x8 b, f32x16 c) {
    return mfma_bf16(a, b, c);
}
__device__ __forceinline__ f32x16 mfma_chunk(f32x4 a, f32x4 b, f32x16 c) {
    c = mfma_f32(a[0], b[0], c);
    c = mfma_f32(a[1], b[1], c);
    c = mfma_f32(a[2], b[2], c);
    c = mfma_f32(a[3], b[3], c);
    return c;
}

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

template <typename V> __device__ __forceinline__ V zero_vec() {
    V z;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(V) / sizeof(z[0])); ++i) z[i] = 0;
    return z;
}

// Load the 16-byte chunk starting at column d0 of a row of length D.
// vec_ok: D is a multiple of the chunk width and the row base is 16-byte
// aligned, so a whole in-range chunk can be read as one vector.  Columns
// >= D and rows that do not exist read as zero.
template <typename T>
__device__ __forceinline__ typename Elt<T>::vec load_chunk(const T* __restrict__ row, int d0, int D,
                                                          bool row_ok, bool vec_ok) {
    typedef typename Elt<T>::vec V;
    constexpr int W = Elt<T>::VEC;
    V r = zero_vec<V>();
    if (row_ok && d0 < D) {
        if (vec_ok) {
            r = *reinterpret_cast<const V*>(row + d0);
        } else {
#pragma unroll
            for (int i = 0; i < W; ++i)
                if (d0 + i < D) r[i] = row[d0 + i];
        }
    }
    return r;
}

// Store 4 consecutive values (columns d0..d0+3) of an output row.
template <typename T>
__device__ __forceinline__ void store4(T* __restrict__ row, int d0, int D, float a, float b, float c,
                                       float d, bool vec4_ok) {
    if (d0 >= D) return;
    if (vec4_ok) {
        if constexpr (sizeof(T) == 4) {
            f32x4 v = {a, b, c, d};
            *reinterpret_cast<f32x4*>(row + d0) = v;
        } else {
            bf16x4 v = {(bf16)a, (bf16)b, (bf16)c, (bf16)d};
            *reinterpret_cast<bf16x4*>(row + d0) = v;
        }
    } else {
        const float x[4] = {a, b, c, d};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (d0 + i < D) row[d0 + i] = (T)x[i];
    }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Max and sum of x over the lane pairs (i, i ^ 32) and (i, i ^ 16), the same
// value in both lanes of a pair, in registers: v_permlane32_swap(x, x) gives
// (x of lane i & 31, x of lane (i & 31) + 32) in every lane, and
// v_permlane16_swap(x, x) the same for rows 2k and 2k + 1 of 16 lanes.  Both
// lanes add the two values in one order, which is also the bits of
// x + shfl_xor(x, 32) (addition commutes).  All lanes must be active.
__device__ __forceinline__ float half_max(float x) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float half_sum(float x) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float row16_max(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float row16_sum(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// Keys visible to query row i: [lo(i), hi(i)], the reference's additive masks
// (-1e10 entries, core/ops.cpp:2167-2180 and the Gemma sliding / padding masks
// of graph/gemma_model.cpp:272-320) as ranges:
//   hi(i) = min(causal ? i : S - 1, len - 1)   causal mask, key padding
//   lo(i) = W > 0 ? i - W + 1 : 0              causal sliding window of W keys
// len = valid keys of the batch (S without padding).  Both bounds are
// non-decreasing in i, so a block of rows and a block of keys either
// certainly never meet (!any), certainly always meet (all), or need the
// per-element mask.
struct KeyVis {
    int S, W, len;
    bool causal;
    __device__ __forceinline__ int hi(int i) const { return min(causal ? i : S - 1, len - 1); }
    __device__ __forceinline__ int lo(int i) const { return W > 0 ? i - W + 1 : 0; }
    __device__ __forceinline__ bool visible(int i, int j) const { return j <= hi(i) && j >= lo(i); }
    // Some row of [r0, r1] may see some key of [k0, k1].
    __device__ __forceinline__ bool any(int r0, int r1, int k0, int k1) const { return k0 <= hi(r1) && k1 >= lo(r0); }
    // Every row of [r0, r1] sees every key of [k0, k1].
    __device__ __forceinline__ bool all(int r0, int r1, int k0, int k1) const { return k1 <= hi(r0) && k0 >= lo(r1); }
    // The rows that see key j: [rlo(j), rhi(j)) (none for a padding key).
    __device__ __forceinline__ int rlo(int j) const { return j >= len ? (1 << 30) : (causal ? j : -(1 << 30)); }
    __device__ __forceinline__ int rhi(int j) const { return W > 0 ? j + W : (1 << 30); }
};

// ---------------------------------------------------------------------------
// LDS staging primitives of the bf16 fast path (gfx950).
//
// global_load_lds_dwordx4: every lane fetches 16 bytes from its own global
// address and the wave writes them to LDS at base + 16 * lane (measured on
// gfx950), without passing through VGPRs.  `base` must be wave-uniform.
// The load counts against vmcnt like an ordinary global load.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;

// LDS byte address of a __shared__ pointer (wave-uniform where p is).  A
// generic pointer into LDS carries the LDS offset in its low 32 bits (the
// high half is the shared aperture), so this is a truncation; an address-space
// cast would add a null check.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// global_load_lds_dwordx4: lane l copies 16 bytes from gptr (its own address)
// to LDS byte address M0 + 16 l, without a VGPR round trip.  Issued as inline
// asm so that the compiler does not track it as an LDS write: it would
// otherwise wait for every outstanding direct load (vmcnt(0)) before LDS
// reads it cannot prove disjoint, including reads of the OTHER buffer while
// the next tile streams in.  The kernels order these loads themselves with
// lds_barrier_vm (explicit vmcnt) and workgroup barriers.  Loads complete in
// order, so the compiler's own vmcnt waits stay correct (they only become
// more conservative).  An LDS DMA that reads M0 right after an SALU write of
// M0 needs one wait state (the s_nop), which the compiler's hazard pass
// cannot insert inside an asm block.
__device__ __forceinline__ void load_lds_16(const void* gptr, void* lds_base) {
    const uint32_t m0 = lds_addr(lds_base);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(m0)
                 : "memory", "m0");
}

// The same load with the address split into a wave-uniform 64-bit base (an
// SGPR pair: the instruction's saddr form) and this lane's 32-bit byte offset,
// so that a tile's loads need no per-lane 64-bit address arithmetic.
// lds_addr: the wave-uniform LDS byte address of the 1 KiB destination.
__device__ __forceinline__ void load_lds_16_s(const void* sbase, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
                 "s"(lds_addr)
                 : "memory", "m0");
}


// ---------------------------------------------------------------------------
// v_mfma_f32_32x32x16_bf16 with its accumulator in VGPRs, as inline asm.
//
// The builtin puts every MFMA accumulator of a function in AGPRs or every one
// in VGPRs (the register form is chosen per compile).  The D = 256 kernels
// need both at once: their loop-carried accumulators fill the 256 AGPRs, so
// the per-tile score products (S, dP) run through these VGPR forms.
//
// The hazard recognizer does not look inside inline asm, so these carry the
// wait states the compiler inserts around the builtin on gfx950:
//   - 2 wait states between a VALU write of an operand and the MFMA
//     (s_nop 1 in front of every MFMA);
//   - after the last MFMA of a chain, mfma_v_drain: 16 wait states (the
//     builtin gets 12 for this 8-pass MFMA) before any instruction reads or
//     writes its result registers.  The drain takes the accumulators as
//     operands, so nothing that uses them can be scheduled before it.
// Back-to-back MFMAs accumulating into the same registers need none.  Early
// clobber keeps the result registers apart from the operands.
//
// mfma_v_first also starts every builtin accumulation chain: for the builtin
// with a literal-zero accumulator the compiler (ROCm 7.2) may place the
// result registers over the A/B operands, which gave NaN results on gfx950
// (the scan in tests/test_geometry.py checks the built code for it).
__device__ __forceinline__ void mfma_v_first(f32x16& c, const bf16x8& a, const bf16x8& b) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_v(f32x16& c, const bf16x8& a, const bf16x8& b) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
// The first step of a 16x16x32 accumulator chain (srcC = 0), early-clobber
// like mfma_v_first.
__device__ __forceinline__ void mfma16_first(f32x4& c, const bf16x8& a, const bf16x8& b) {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
}
// A 16x16x32 step whose A operand stays live past the instruction, so that
// its result registers cannot take the A operand's (the compiler would
// otherwise reuse a dead operand's registers for the result).
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    asm volatile("" ::"v"(a));
    return d;
}

__device__ __forceinline__ void mfma_v_drain(f32x16& c0, f32x16& c1) {
    asm volatile("s_nop 7\n\ts_nop 7" : "+v"(c0), "+v"(c1));
}
__device__ __forceinline__ void mfma_v_drain(f32x16& c0) { asm volatile("s_nop 7\n\ts_nop 7" : "+v"(c0)); }

// First chunk of an accumulation chain (accumulator in AGPRs where AGPR,
// else VGPRs), the rest through the builtins: keeps the result registers
// apart from the operands (see mfma_v_first).  The chain must continue with
// at least one builtin MFMA before its result is read.
template <bool AGPR> __device__ __forceinline__ void mfma_chunk_first(f32x16& c, const bf16x8& a, const bf16x8& b) {
    if constexpr (AGPR)
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&a"(c) : "v"(a), "v"(b));
    else
        mfma_v_first(c, a, b);
}
template <bool AGPR> __device__ __forceinline__ void mfma_chunk_first(f32x16& c, const f32x4& a, const f32x4& b) {
    if constexpr (AGPR)
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x2_f32 %0, %1, %2, 0" : "=&a"(c) : "v"(a[0]), "v"(b[0]));
    else
        asm volatile("s_nop 1\n\tv_mfma_f32_32x32x2_f32 %0, %1, %2, 0" : "=&v"(c) : "v"(a[0]), "v"(b[0]));
    c = mfma_f32(a[1], b[1], c);
    c = mfma_f32(a[2], b[2], c);
    c = mfma_f32(a[3], b[3], c);
}

// Wave index in the workgroup as a wave-uniform (scalar) value, for LDS
// addresses of the direct loads.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// A condition that is the same in every lane of the wave, as a scalar: an
// if/else on it is a scalar branch, so a wave that skips a block does not
// step through it with an empty exec mask (and vice versa).
__device__ __forceinline__ bool wave_uniform(bool c) { return __builtin_amdgcn_readfirstlane((int)c) != 0; }

// s_waitcnt vmcnt(n) with the other counters left unconstrained (gfx9
// encoding: vmcnt low bits [3:0], high bits [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barriers for the direct-to-LDS pipelines.  __syncthreads()
// carries a release fence, which makes every wave wait for ALL its
// outstanding loads (vmcnt(0)) - including the prefetch of the next tile -
// before the barrier, serialising the double buffer.  These barriers wait
// only for this wave's LDS operations and, with VM = N, for all but its N
// most recent global loads (loads return in order), then s_barrier.  The
// "memory" clobber keeps the compiler from moving memory operations across.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
template <int VM>
__device__ __forceinline__ void lds_barrier_vm() {
    static_assert(VM >= 0 && VM < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(VM) : "memory");
}

// ds_read_b64_tr_b16 (measured on gfx950): within each aligned group of 16
// lanes, reader lane j supplies an 8-byte row M[j][0..3]; output lane i gets
// { M[i/4][i%4], M[4+i/4][i%4], M[8+i/4][i%4], M[12+i/4][i%4] }.  So if lane j
// reads X[r0 + j/4][c0 + 4*(j%4) .. +3] of a row-major b16 matrix, lane i
// receives X[r0 + 0..3][c0 + i]: four consecutive rows of one column.
__device__ __forceinline__ bf16x4 ds_read_tr4(const bf16* lds_elem_ptr) {
    const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(lds_elem_ptr));
    return __builtin_bit_cast(bf16x4, r);
}

// XOR swizzles of 16-byte chunks inside an unpadded LDS tile row of CPR
// chunks (CPR = row bytes / 16; 8, 16 or 32).  A tile element (r, col) lives
// at r * ROW + ((col / 8) ^ swz(r)) * 8 + col % 8 (bf16 elements).
// LDS has 64 four-byte banks (256 bytes per cycle).
//  swz_row : for row reads, where 16 lanes read one chunk column of 16
//            consecutive rows (ds_read_b128) -> 16 distinct bank groups.
//  swz_tr  : for transposing reads, where a wave reads 8 consecutive rows x
//            64 bytes (ds_read_b64_tr_b16) -> 2 cycles, the minimum.
//  swz_dual: both patterns at their minimum (tiles read both ways).
template <int CPR> __host__ __device__ __forceinline__ constexpr int swz_row(int r) {
    return CPR >= 16 ? (r & 15) : ((r >> 1) & 7);
}
template <int CPR> __host__ __device__ __forceinline__ constexpr int swz_tr(int r) {
    return (CPR >= 16 ? (r & 3) : ((r >> 1) & 1)) << 2;
}
template <int CPR> __host__ __device__ __forceinline__ constexpr int swz_dual(int r) {
    return CPR >= 16 ? (4 * (r & 3) + ((r >> 2) & 3)) : (4 * ((r >> 1) & 1) + ((r >> 2) & 3));
}

//  swz_tr16: for transposing reads where a wave reads 16 consecutive rows x
//            32 bytes (ds_read_b64_tr_b16 in the 16x16x32 MFMA layout): rows
//            r..r+7 land in distinct 32-byte windows (CPR >= 16).
template <int CPR> __host__ __device__ __forceinline__ constexpr int swz_tr16(int r) { return 2 * (r & 7); }

enum { SWZ_ROW = 0, SWZ_TR = 1, SWZ_DUAL = 2, SWZ_TR16 = 3 };

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
enum { SG_MFMA = 0x008, SG_DS_READ = 0x100 };

// Pin the order of an unrolled "operands read PF steps ahead" loop in the
// current scheduling region.  A step reads R LDS operands and issues M
// MFMAs: PF steps of reads, then (M MFMAs, R reads) NI-PF times, then the
// last PF steps of MFMAs.  Without it the machine scheduler moves every read
// next to its MFMA and the LDS latency is exposed once per MFMA.
template <int NI, int PF, int R, int M = 1>
__device__ __forceinline__ void pin_read_ahead() {
    __builtin_amdgcn_sched_group_barrier(SG_DS_READ, PF * R, 0);
#pragma unroll
    for (int i = 0; i < NI - PF; ++i) {
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, M, 0);
        __builtin_amdgcn_sched_group_barrier(SG_DS_READ, R, 0);
    }
    __builtin_amdgcn_sched_group_barrier(SG_MFMA, PF * M, 0);
}

template <int CPR, int SWZ> __host__ __device__ __forceinline__ constexpr int swz(int r) {
    return SWZ == SWZ_ROW ? swz_row<CPR>(r)
           : SWZ == SWZ_TR ? swz_tr<CPR>(r)
           : SWZ == SWZ_TR16 ? swz_tr16<CPR>(r)
                             : swz_dual<CPR>(r);
}

// Element offset of (row r, column col) in a swizzled bf16 tile.
template <int CPR, int SWZ>
__host__ __device__ __forceinline__ constexpr int tile_off(int r, int col) {
    return r * (CPR * 8) + (((col >> 3) ^ swz<CPR, SWZ>(r)) << 3) + (col & 7);
}

// Issue the direct loads of a [ROWS x DP] bf16 tile whose first global row is
// row0 (row stride ld elements, D valid columns) into a swizzled LDS tile.  NT threads share
// the work; every thread issues ROWS*DP/8/NT loads (wave-uniform count).
// Rows >= S read row S-1 and chunks >= D read chunk 0, so every address is
// in bounds; callers mask such rows and never use such columns.
// Load j (0 <= j < ROWS*DP/8/NT) of this thread's share of such a tile, so
// that a tile's loads can be spread between other instructions.
template <int DP, int ROWS, int NT, int SWZ>
__device__ __forceinline__ void issue_tile_part(const bf16* __restrict__ src, int row0, int S, int D, int ld,
                                                bf16* lds_tile, int j) {
    constexpr int CPR = DP / 8;
    constexpr int PER_WAVE = ROWS * CPR / NT;
    static_assert(PER_WAVE * NT == ROWS * CPR, "tile must split evenly over the threads");
    const int lane = threadIdx.x & 63;
    const int w = wave_id();
    const int m = w * PER_WAVE + j;
    const int P = m * 64 + lane;
    const int r = P / CPR, p = P % CPR;
    const int c = p ^ swz<CPR, SWZ>(r);
    const int gr = min(row0 + r, S - 1);
    const int col = 8 * c < D ? 8 * c : 0;
    load_lds_16(src + (int64_t)gr * ld + col, lds_tile + m * 512);
}

// The same loads with loop-invariant per-lane offsets.  Load j of wave w
// (m = w * PER + j, PER loads per thread) covers the R = 64 / CPR tile rows
// R*m .. R*m + R - 1 and fills LDS bytes m * 1024 ..; lane (q = lane / CPR,
// p = lane % CPR) reads row R*m + q, chunk p ^ swz(R*m + q).  The swizzles
// are XOR-linear over disjoint row bits and R*m + q = R*w*PER | R*j | q, so
// that chunk is (p ^ swz(q) ^ swz(R*w*PER)) ^ swz(R*j): a per-lane part and a
// compile-time part.  The lane's byte offset inside the rows of load j is
//   q * ld * 2 + (lx ^ 16 * swz(R*j)),   lx = 16 * (p ^ swz(q) ^ swz(R*w*PER)).
// The rows' base (row0 + R*m) goes into the instruction's scalar address.
// Valid for D == DP (whole rows; no column clamp) and rows < S; callers
// take issue_tile_part for a load that would cross S.
template <int DP, int ROWS, int NT, int SWZ> struct TileDma {
    static constexpr int CPR = DP / 8, R = 64 / CPR, PER = ROWS * CPR / NT;
    static_assert(PER * NT == ROWS * CPR && R * CPR == 64, "tile must split evenly over the threads");
    uint32_t lx, lrow;
    // Row offset (within the tile) of this wave's first load.
    static __host__ __device__ constexpr int row_w(int w) { return R * w * PER; }
    static __host__ __device__ constexpr uint32_t cx(int j) { return 16u * (uint32_t)swz<CPR, SWZ>(R * j); }
    __host__ __device__ void init(int lane, int w, int ld_elems) {
        const int q = lane / CPR, p = lane % CPR;
        lx = 16u * (uint32_t)(p ^ swz<CPR, SWZ>(q) ^ swz<CPR, SWZ>(row_w(w)));
        lrow = (uint32_t)q * (uint32_t)ld_elems * 2u;
    }
    __host__ __device__ uint32_t voff(int j) const { return lrow + (lx ^ cx(j)); }
};

// Load j of this thread's share of a tile (at lds_tile, LDS byte address
// lds_tile_addr).  FAST: the tile uses TileDma, which the launch may choose
// when every tile is whole (D == DP and S a multiple of the tile's rows).
// Otherwise issue_tile_part, which clamps rows and columns per lane.
template <bool FAST, int DP, int ROWS, int NT, int SWZ>
__device__ __forceinline__ void issue_tile_j(const TileDma<DP, ROWS, NT, SWZ>& t, const bf16* __restrict__ src,
                                             int row0, int S, int D, int ld, bf16* lds_tile, uint32_t lds_tile_addr,
                                             int j) {
    typedef TileDma<DP, ROWS, NT, SWZ> TD;
    if constexpr (FAST) {
        const int w = wave_id();
        // wave-uniform: the scalar base of this wave's rows, and M0 (the
        // tile's LDS byte address, passed as an integer)
        const char* base = reinterpret_cast<const char*>(src + (int64_t)(row0 + TD::row_w(w)) * ld) +
                           (int64_t)(TD::R * j) * ld * 2;
        const uint32_t m0 = lds_tile_addr + (uint32_t)(w * TD::PER) * 1024u;
        // M0 is set with s_mov (no SCC write inside the asm statement; the
        // address arithmetic stays with the compiler, which knows SCC).
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(t.voff(j)),
                     "s"(base), "s"(m0 + (uint32_t)(j * 1024))
                     : "memory", "m0");
    } else {
        issue_tile_part<DP, ROWS, NT, SWZ>(src, row0, S, D, ld, lds_tile, j);
    }
}

template <int DP, int ROWS, int NT, int SWZ>
__device__ __forceinline__ void issue_tile(const bf16* __restrict__ src, int row0, int S, int D, int ld,
                                           bf16* lds_tile) {
    constexpr int PER_WAVE = ROWS * (DP / 8) / NT;
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) issue_tile_part<DP, ROWS, NT, SWZ>(src, row0, S, D, ld, lds_tile, j);
}

}  // namespace mft
