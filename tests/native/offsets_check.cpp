// Host check of the fast kernels' precomputed LDS and direct-load offsets: the
// per-lane closed forms of TileDma (attn_common.h), FwdLane (attn_fwd_fast.h) and
// BwdLane (attn_bwd_fast.h)
// against the swizzled tile addressing they replace (tile_off, and the per-lane
// address arithmetic of issue_tile_part), for every lane, wave and load.
#include "attn_fwd_fast.h"
#include "attn_bwd_fast.h"
#include <cstdio>
using namespace mft;
static int bad = 0;
#define CHECK(c, ...) do { if (!(c)) { if (bad++ < 10) printf(__VA_ARGS__); } } while (0)

template <int DP, int ROWS, int SWZ> void check_dma(int ld) {
  constexpr int CPR = DP / 8, NT = 256, PER = ROWS * CPR / NT;
  for (int w = 0; w < 4; ++w) for (int lane = 0; lane < 64; ++lane) {
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
  check_fwd<64>(); check_fwd<128>(); check_fwd<256>();
  check_bwd<64>(); check_bwd<128>(); check_bwd<256>();
  printf("%s %d mismatches\n", bad ? "FAIL" : "ok", bad);
  return bad != 0;
}
