// Degree-bucketed row schedule shared by the SpMM and GAT kernels.
//
// A schedule is one int32 device buffer built once per CSR (or CSC) on the
// host (cign_row_schedule_build) and uploaded by the caller:
//
//   [0] n_light   [1] n_seg   [2] n_hrow   [3] seg_edges
//   light rows           : n_light ints, rows with degree <= light_max,
//                          sorted by degree (descending)
//   segments             : n_seg x {row, edge_begin, edge_end, hrow}
//   heavy-row table      : n_hrow x {first_seg, n_seg_of_row}
//
// Light rows are processed one per wavefront (4 per 256-thread workgroup).
// Every heavy row (degree > light_max) is cut into segments of at most
// seg_edges edges, one workgroup each; when a row has more than one segment,
// the workgroups publish partial results and the last one to finish merges
// them in segment order (deterministic) and writes the row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cign {

struct Sched {
  const int32_t* light;  // [n_light]
  const int4* seg;       // [n_seg]  {row, beg, end, hrow}
  const int2* hrow;      // [n_hrow] {first_seg, nseg}
  int n_light;
  int n_seg;
  int n_hrow;
};

// Header size (ints) before the light-row list.
constexpr int kSchedHeader = 4;

inline Sched make_sched(const int32_t* dev, int n_light, int n_seg, int n_hrow) {
  Sched s;
  s.light = dev + kSchedHeader;
  // Segment records start on a 16-byte boundary.
  const int seg_off = (kSchedHeader + n_light + 3) & ~3;
  s.seg = reinterpret_cast<const int4*>(dev + seg_off);
  s.hrow = reinterpret_cast<const int2*>(dev + seg_off + 4 * n_seg);
  s.n_light = n_light;
  s.n_seg = n_seg;
  s.n_hrow = n_hrow;
  return s;
}

inline int64_t sched_ints(int n_light, int n_seg, int n_hrow) {
  const int seg_off = (kSchedHeader + n_light + 3) & ~3;
  return static_cast<int64_t>(seg_off) + 4LL * n_seg + 2LL * n_hrow;
}

// Grid size for a schedule: one workgroup per segment plus one per 4 light rows.
__host__ __device__ inline int sched_blocks(const Sched& s) { return s.n_seg + (s.n_light + 3) / 4; }

}  // namespace cign
