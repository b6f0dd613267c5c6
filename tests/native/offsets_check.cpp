// Host check of the fast kernels' precomputed LDS and direct-load offsets: the
// per-lane closed forms of TileDma (attn_common.h), FwdLane (attn_fwd_fast.h),
// W16Lane (attn_fwd_w16.h) and BwdLane (attn_bwd_fast.h)
// against the swizzled tile addressing they replace (tile_off, and the per-lane
// address arithmetic of issue_tile_part), for every lane, wave and load.
#include "attn_fwd_fast.h"
#include "attn_fwd_w16.h"
#include "attn_bwd_fast.h"
#include <cstdio>
using namespace mft;
static int bad = 0;
#define CHECK(c, ...) do { if (!(c)) { if (bad++ < 10) printf(__VA_ARGS__); } } while (0)

template <int DP, int ROWS, int SWZ, int NT = 256> void check_dma(int ld) {
  constexpr int CPR = DP / 8, PER = ROWS * CPR / NT;
  for (int w = 0; w < NT / 64; ++w) for (int lane = 0; lane < 64; ++lane) {
    TileDma<DP, ROWS, NT, SWZ> t; t.init(lane, w, ld);
    for (int j = 0; j < PER; ++j) {
      const int m = w * PER + j, P = m * 64 + lane, r = P / CPR, p = P % CPR, c = p ^ swz<CPR, SWZ>(r);
      const long old_b = ((long)r * ld + 8 * c) * 2;           // bytes from tile row 0
      const long new_b = (long)(TileDma<DP, ROWS, NT, SWZ>::row_w(w) + TileDma<DP, ROWS, NT, SWZ>::R * j) * ld * 2 + t.voff(j);
      CHECK(old_b == new_b, "dma DP%d ROWS%d SWZ%d w%d lane%d j%d: %ld vs %ld\n", DP, ROWS, SWZ, w, lane, j, old_b, new_b);
    }
  }
}
template <int DP> void check_fwd() {
  constexpr int CPR = DP / 8, NC = DP / 16, NDT = DP / 32;
  for (int lane = 0; lane < 64; ++lane) {
    const int n = lane & 31, hh = lane >> 5, i16 = lane & 15, nh = (lane >> 4) & 1;
    fwd::FwdLane<DP> ln; ln.init(lane, 0, DP, DP);
    for (int kk = 0; kk < 2; ++kk) for (int c = 0; c < NC; ++c) {
      const int old_b = 2 * tile_off<CPR, SWZ_ROW>(32 * kk + n, 16 * c + 8 * hh);
      CHECK(old_b == (int)ln.k_off(kk, c), "K DP%d lane%d kk%d c%d: %d vs %d\n", DP, lane, kk, c, old_b, (int)ln.k_off(kk, c));
    }
    for (int ke = 0; ke < 4; ++ke) for (int dt = 0; dt < NDT; ++dt) for (int hi = 0; hi < 2; ++hi) {
      const int r0 = 16 * ke + 4 * hh + (i16 >> 2) + 8 * hi;
      const int col = 32 * dt + 16 * nh + 4 * (i16 & 3);
      const int old_b = 2 * tile_off<CPR, SWZ_TR>(r0, col);
      CHECK(old_b == (int)ln.v_off(ke, dt, hi), "V DP%d lane%d ke%d dt%d hi%d: %d vs %d\n", DP, lane, ke, dt, hi, old_b, (int)ln.v_off(ke, dt, hi));
    }
  }
}
// 16x16x32 layout: K row reads (lane n = l % 16 reads row 16kb + n, k 32j +
// 8g) and transposed V reads (reading lane n reads row 32s2 + 16h + 4g + n/4,
// columns 16dt + 4(n%4) .. +3).
template <int DP> void check_w16() {
  constexpr int CPR = DP / 8, NJ = DP / 32, NDT = DP / 16;
  for (int lane = 0; lane < 64; ++lane) {
    const int n = lane & 15, g = lane >> 4;
    fwd::W16Lane<DP> ln; ln.init(lane, 0, DP, DP);
    for (int kb = 0; kb < 4; ++kb) for (int j = 0; j < NJ; ++j) {
      const int old_b = 2 * tile_off<CPR, SWZ_ROW>(16 * kb + n, 32 * j + 8 * g);
      CHECK(old_b == (int)ln.k_off(kb, j), "w16 K lane%d kb%d j%d: %d vs %d\n", lane, kb, j, old_b, (int)ln.k_off(kb, j));
    }
    for (int dt = 0; dt < NDT; ++dt) for (int s2 = 0; s2 < 2; ++s2) for (int h = 0; h < 2; ++h) {
      const int r = 32 * s2 + 16 * h + 4 * g + (n >> 2), col = 16 * dt + 4 * (n & 3);
      const int old_b = 2 * tile_off<CPR, SWZ_TR16>(r, col);
      CHECK(old_b == (int)ln.v_off(dt, s2, h), "w16 V lane%d dt%d s2%d h%d: %d vs %d\n", lane, dt, s2, h, old_b, (int)ln.v_off(dt, s2, h));
    }
  }
}
// The transposed V reads of one instruction reach 8 distinct 32-byte bank
// windows for rows 4g + n/4 in each half wave (lanes 0-31: rows 0-7, lanes
// 32-63: rows 8-15): two LDS cycles, the minimum for 512 bytes.
template <int DP> void check_w16_banks() {
  constexpr int NDT = DP / 16;
  for (int dt = 0; dt < NDT; ++dt) for (int half = 0; half < 2; ++half) {
    unsigned seen = 0;
    for (int lane = 32 * half; lane < 32 * half + 32; ++lane) {
      fwd::W16Lane<DP> ln; ln.init(lane, 0, DP, DP);
      const int win = (int)((ln.v_off(dt, 0, 0) % 256) / 32);
      seen |= 1u << win;
    }
    CHECK(seen == 0xFFu, "w16 V banks dt%d half%d: windows %x\n", dt, half, seen);
  }
}
template <int DP> void check_bwd() {
  constexpr int CPR = DP / 8, NC = DP / 16, NDT = DP / 32;
  for (int lane = 0; lane < 64; ++lane) {
    const int n = lane & 31, hh = lane >> 5, i16 = lane & 15, nh = (lane >> 4) & 1;
    bwd::BwdLane<DP> ln; ln.init(lane);
    for (int k = 0; k < 4; ++k) for (int c = 0; c < NC; ++c) {
      const int old_b = 2 * tile_off<CPR, SWZ_DUAL>(32 * k + n, 16 * c + 8 * hh);
      CHECK(old_b == (int)ln.row(k, c), "bwd row DP%d lane%d k%d c%d: %d vs %d\n", DP, lane, k, c, old_b, (int)ln.row(k, c));
    }
    for (int k = 0; k < 2; ++k) for (int e = 0; e < 2; ++e) for (int dt = 0; dt < NDT; ++dt) for (int hi = 0; hi < 2; ++hi) {
      const int r0 = 32 * k + 16 * e + 4 * hh + (i16 >> 2) + 8 * hi;
      const int col = 32 * dt + 16 * nh + 4 * (i16 & 3);
      const int old_b = 2 * tile_off<CPR, SWZ_DUAL>(r0, col);
      CHECK(old_b == (int)ln.trn(k, e, dt, hi), "bwd tr DP%d lane%d k%d e%d dt%d hi%d: %d vs %d\n", DP, lane, k, e, dt, hi, old_b, (int)ln.trn(k, e, dt, hi));
    }
  }
}
int main() {
  for (int ld : {64, 128, 256, 1024, 3584}) {
    check_dma<64, 64, SWZ_ROW>(ld); check_dma<64, 64, SWZ_TR>(ld); check_dma<64, 64, SWZ_DUAL>(ld);
    check_dma<128, 64, SWZ_ROW>(ld); check_dma<128, 64, SWZ_TR>(ld); check_dma<128, 64, SWZ_DUAL>(ld);
    check_dma<256, 64, SWZ_ROW>(ld); check_dma<256, 64, SWZ_TR>(ld); check_dma<256, 64, SWZ_DUAL>(ld);
    check_dma<64, 32, SWZ_DUAL>(ld); check_dma<128, 32, SWZ_DUAL>(ld); check_dma<256, 32, SWZ_DUAL>(ld);
    check_dma<64, 128, SWZ_ROW>(ld); check_dma<128, 128, SWZ_ROW>(ld); check_dma<256, 128, SWZ_ROW>(ld);
  }
  for (int ld : {256, 1024, 3584}) {
    check_dma<256, 64, SWZ_ROW, 512>(ld); check_dma<256, 64, SWZ_TR16, 512>(ld);
  }
  check_fwd<64>(); check_fwd<128>(); check_fwd<256>();
  check_w16<256>(); check_w16_banks<256>();
  check_bwd<64>(); check_bwd<128>(); check_bwd<256>();
  printf("%s %d mismatches\n", bad ? "FAIL" : "ok", bad);
  return bad != 0;
}
