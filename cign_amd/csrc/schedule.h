// Degree-bucketed row schedule shared by the SpMM and GAT kernels.
//
// A schedule is one int32 device buffer built once per CSR (or CSC) on the
// host (cign_row_schedule_build) and uploaded by the caller:
//
//   header (12 ints): n_light, n_seg, n_hrow, seg_edges, light_max, 0,
//                     n_gt1, n_gt2, n_gt4, n_gt8, n_gt16, n_gt32
//                     (light rows with degree > 1, 2, 4, 8, 16, 32)
//   light records  : n_light x {row, edge_begin, edge_end, 0}, sorted by
//                    degree (descending), rows with degree <= light_max
//   segments       : n_seg x {row, edge_begin, edge_end, hrow}
//   heavy-row table: n_hrow x {first_seg, n_seg_of_row}
//
// Light rows carry their edge range so a kernel reaches its edges with one
// dependent load instead of two. Kernels process light rows one per wavefront
// or, for rows short enough, one per group of lanes (n_gt* gives the split of
// the degree-sorted list). Every heavy row (degree > light_max) is cut into
// segments of at most seg_edges edges, one workgroup each; when a row has more
// than one segment the workgroups publish partial results and the last one to
// finish merges them in segment order (deterministic) and writes the row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cign {

struct Sched {
  const int4* light;  // [n_light] {row, beg, end, 0}
  const int4* seg;    // [n_seg]   {row, beg, end, hrow}
  const int2* hrow;   // [n_hrow]  {first_seg, nseg}
  int n_light;
  int n_seg;
  int n_hrow;
};

constexpr int kSchedHeader = 12;

// Light rows with degree > 2^k, k = 0..5, are header[6 + k].
inline int sched_count_gt(const int32_t* hdr, int lanes) {
  int k = 0;
  while ((1 << k) < lanes && k < 5) ++k;
  return (1 << k) == lanes ? hdr[6 + k] : hdr[0];
}

inline Sched make_sched(const int32_t* dev, int n_light, int n_seg, int n_hrow) {
  Sched s;
  s.light = reinterpret_cast<const int4*>(dev + kSchedHeader);
  s.seg = reinterpret_cast<const int4*>(dev + kSchedHeader + 4 * n_light);
  s.hrow = reinterpret_cast<const int2*>(dev + kSchedHeader + 4 * n_light + 4 * n_seg);
  s.n_light = n_light;
  s.n_seg = n_seg;
  s.n_hrow = n_hrow;
  return s;
}

inline int64_t sched_ints(int n_light, int n_seg, int n_hrow) {
  return static_cast<int64_t>(kSchedHeader) + 4LL * n_light + 4LL * n_seg + 2LL * n_hrow;
}

// Grid size when every light row gets a wavefront: one workgroup per segment
// plus one per 4 light rows.
__host__ __device__ inline int sched_blocks(const Sched& s) { return s.n_seg + (s.n_light + 3) / 4; }

}  // namespace cign
