// The launch shape of a q4 launch: the kernel family that runs it, its grid
// and its workgroup size. runner.cpp's launch_qmv applies it; the Python
// package's test helper restates it, and a CPU test checks the two agree.
#pragma once
#include <stdint.h>

#include "lisa_kernels.h"
#include "lisa_model.h"

enum LisaQmvFamily {
  LISA_QMV_FOUR_WAVE = 0,   // lisa_qmv_k{K}_m{M}_{prologue}[_{epilogue}], 256 threads
  LISA_QMV_GATEUP_WIDE = 1, // lisa_qmv_k5120_m{M}_prenorm_gateup_wide
  LISA_QMV_INPROJ_WIDE = 2, // lisa_qmv_k5120_m{M}_prenorm_wide{nw}
  LISA_QMV_X_WIDE = 3,      // lisa_qmv_k5120_m1_x_wide9
};

struct LisaQmvShape {
  int family;
  uint32_t grid, block, nw;  // nw: waves per workgroup
};

// kinds: the epilogue kind of each of the n matrices; tiles: their tiles in
// total (8 rows, or 4 output pairs of a GATEUP matrix).
inline LisaQmvShape lisa_qmv_shape(uint32_t K, int m_rows, uint32_t pro_mode, const uint32_t* kinds, int n,
                                   uint32_t tiles, bool gate_ab, bool am_val) {
  bool all_store = n > 0, store_conv = n > 0;
  for (int e = 0; e < n; ++e) {
    all_store = all_store && kinds[e] == LISA_EPI_STORE;
    store_conv = store_conv && (kinds[e] == LISA_EPI_STORE || kinds[e] == LISA_EPI_CONV);
  }
  const bool k5120 = K == LISA_HIDDEN;
  // the MLP gate/up alone under PRENORM: one 16-wave workgroup per 17 tiles
  // (the 4352 tiles of the model's pair are 256 x 17)
  if (k5120 && n == 1 && kinds[0] == LISA_EPI_GATEUP && pro_mode == LISA_PRO_PRENORM && !gate_ab && !am_val) {
    const uint32_t g = (tiles + LISA_QMV_WIDE_TILES - 1) / LISA_QMV_WIDE_TILES;
    return {LISA_QMV_GATEUP_WIDE, g ? g : 1, LISA_QMV_WIDE_THREADS, LISA_QMV_WIDE_THREADS / 64};
  }
  // the GDN (2048 tiles) and attention (1792) in-projections under PRENORM:
  // one workgroup of nw = tiles / 256 waves per CU, one tile per wave
  const uint32_t nw = tiles / LISA_QMV_WIDE_GROUPS;
  if (k5120 && pro_mode == LISA_PRO_PRENORM && store_conv && !am_val && tiles % LISA_QMV_WIDE_GROUPS == 0 &&
      (nw == 7 || nw == 8))
    return {LISA_QMV_INPROJ_WIDE, LISA_QMV_WIDE_GROUPS, 64 * nw, nw};
  // a one-row plain-x launch of 2049..2304 tiles (a 17408-row projection):
  // one workgroup of nine waves per CU
  const uint32_t xw = LISA_QMV_X_WIDE_WAVES;
  if (k5120 && m_rows == 1 && pro_mode == LISA_PRO_LOADX && all_store && !am_val && !gate_ab &&
      tiles > (xw - 1) * LISA_QMV_WIDE_GROUPS && tiles <= xw * LISA_QMV_WIDE_GROUPS)
    return {LISA_QMV_X_WIDE, (tiles + xw - 1) / xw, 64 * xw, xw};
  // four waves: one tile per wave at K = 5120, else one tile per workgroup
  // with its group iterations split over the waves
  const uint32_t g = k5120 ? (tiles + 3) / 4 : tiles;
  return {LISA_QMV_FOUR_WAVE, g ? g : 1, 256, 4};
}
