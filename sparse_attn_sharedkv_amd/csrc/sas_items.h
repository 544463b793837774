// Per-item geometry shared by the host scheduler and the device kernel.
//
// An "item" is one query row (b, s) of one sequence (the reference's
// (bn2, s1g) work unit with mBaseSize = num_heads, metadata.py:388). Its
// attended list is [window rows ++ compressed positions]:
//   s_global = act_kv - act_q + s                       (golden.py:125)
//   window   = [max(s_global - win_left, 0), s_global + 1) of the raw cache
//                                                       (golden.py:128-131)
//   thr      = floor((s_global + 1) / cmp_ratio)        (golden.py:44, :147)
//   compressed positions: scenario 3 scans min(K, thr) top-k slots
//                         (golden.py:48), scenario 2 takes [0, thr).
// Host and device must agree bit for bit, so both include this header.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sas {

struct ItemGeom {
  int32_t win_lo;  // first raw row of the window
  int32_t n_win;   // window rows
  int32_t thr;     // causal bound on compressed ids (0 when no compressed cache)
  int32_t n_cmp;   // compressed positions scanned
};

__host__ __device__ inline int64_t floor_div_pos(int64_t a, int64_t b) {
  // floor(a / b) for b > 0, including negative a (Python semantics)
  return a >= 0 ? a / b : -((-a + b - 1) / b);
}

__host__ __device__ inline ItemGeom item_geom(int32_t act_q, int32_t act_kv, int32_t s,
                                              int32_t win_left, int32_t scenario,
                                              int32_t cmp_ratio, int32_t topk) {
  ItemGeom g;
  const int64_t sg = (int64_t)act_kv - (int64_t)act_q + (int64_t)s;
  int64_t hi = sg + 1;
  int64_t lo = sg - (int64_t)win_left;
  if (lo < 0) lo = 0;
  if (hi < lo) hi = lo;
  g.win_lo = (int32_t)lo;
  g.n_win = (int32_t)(hi - lo);
  g.thr = 0;
  g.n_cmp = 0;
  if (scenario >= 2 && cmp_ratio > 0) {
    const int64_t thr = floor_div_pos(sg + 1, cmp_ratio);
    int64_t n = thr;
    if (scenario == 3 && (int64_t)topk < n) n = topk;
    if (n < 0) n = 0;
    g.thr = (int32_t)(thr < 0 ? 0 : thr);
    g.n_cmp = (int32_t)n;
  }
  return g;
}

}  // namespace sas
