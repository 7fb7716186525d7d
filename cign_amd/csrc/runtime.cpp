// Host-side runtime of libcign_amd: error text, version, row schedules and the
// calibration copy used by the traffic measurement. Compiled with hipcc.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <vector>

#include "common.h"
#include "schedule.h"

namespace cign {

static thread_local char g_last_error[1024] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(kHipError, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return kOk;
}

}  // namespace cign

using namespace cign;

extern "C" {

const char* cign_last_error(void) { return g_last_error; }

int cign_version(void) { return 1; }

// Computes the sizes of a row schedule (see schedule.h) from a host copy of
// a CSR row pointer. Pure host code.
int cign_row_schedule_size(const int64_t* rowptr, int32_t n_rows, int32_t light_max, int32_t seg_edges,
                           int32_t* n_light, int32_t* n_seg, int32_t* n_hrow, int64_t* total_ints) {
  if (n_rows < 0 || light_max < 1 || seg_edges < 1 || !rowptr) {
    return set_error(kInvalid, "cign_row_schedule_size: bad arguments");
  }
  if (rowptr[n_rows] > INT32_MAX) return set_error(kInvalid, "cign_row_schedule_size: more than 2^31-1 edges");
  int64_t nl = 0, ns = 0, nh = 0;
  for (int32_t r = 0; r < n_rows; ++r) {
    const int64_t deg = rowptr[r + 1] - rowptr[r];
    if (deg < 0) return set_error(kInvalid, "cign_row_schedule_size: row pointer not monotone at %d", r);
    if (deg <= light_max) {
      ++nl;
    } else {
      ++nh;
      ns += (deg + seg_edges - 1) / seg_edges;
    }
  }
  if (ns > INT32_MAX / 8) return set_error(kInvalid, "cign_row_schedule_size: too many segments");
  *n_light = static_cast<int32_t>(nl);
  *n_seg = static_cast<int32_t>(ns);
  *n_hrow = static_cast<int32_t>(nh);
  *total_ints = sched_ints(static_cast<int>(nl), static_cast<int>(ns), static_cast<int>(nh));
  return kOk;
}

// Fills a host buffer of `total_ints` int32 with the schedule layout of
// schedule.h. Heavy rows are emitted heaviest first so their workgroups start
// early; light rows are sorted by degree, descending, ties by row id.
int cign_row_schedule_build(const int64_t* rowptr, int32_t n_rows, int32_t light_max, int32_t seg_edges,
                            int32_t* out, int64_t total_ints) {
  int32_t nl = 0, ns = 0, nh = 0;
  int64_t tot = 0;
  int rc = cign_row_schedule_size(rowptr, n_rows, light_max, seg_edges, &nl, &ns, &nh, &tot);
  if (rc != kOk) return rc;
  if (tot != total_ints || !out) return set_error(kInvalid, "cign_row_schedule_build: buffer size mismatch");
  std::memset(out, 0, sizeof(int32_t) * static_cast<size_t>(total_ints));
  std::vector<int32_t> rows(static_cast<size_t>(n_rows));
  std::iota(rows.begin(), rows.end(), 0);
  std::stable_sort(rows.begin(), rows.end(), [&](int32_t a, int32_t b) {
    return (rowptr[a + 1] - rowptr[a]) > (rowptr[b + 1] - rowptr[b]);
  });
  int32_t* light = out + kSchedHeader;
  int32_t* seg = light + 4 * static_cast<int64_t>(nl);
  int32_t* hrow = seg + 4 * static_cast<int64_t>(ns);
  int32_t li = 0, si = 0, hi = 0;
  int32_t gt[6] = {0, 0, 0, 0, 0, 0};
  for (int32_t r : rows) {
    const int64_t b = rowptr[r], e = rowptr[r + 1];
    const int64_t deg = e - b;
    if (deg <= light_max) {
      light[4 * li + 0] = r;
      light[4 * li + 1] = static_cast<int32_t>(b);
      light[4 * li + 2] = static_cast<int32_t>(e);
      ++li;
      for (int k = 0; k < 6; ++k) gt[k] += deg > (1 << k);
    } else {
      const int32_t first = si;
      for (int64_t s = b; s < e; s += seg_edges) {
        seg[4 * si + 0] = r;
        seg[4 * si + 1] = static_cast<int32_t>(s);
        seg[4 * si + 2] = static_cast<int32_t>(std::min<int64_t>(s + seg_edges, e));
        seg[4 * si + 3] = hi;
        ++si;
      }
      hrow[2 * hi + 0] = first;
      hrow[2 * hi + 1] = si - first;
      ++hi;
    }
  }
  const int32_t hdr[kSchedHeader] = {nl, ns, nh, seg_edges, light_max, 0, gt[0], gt[1], gt[2], gt[3], gt[4], gt[5]};
  std::memcpy(out, hdr, sizeof(hdr));
  return kOk;
}

}  // extern "C"
