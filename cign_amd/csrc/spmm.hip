// CSR SpMM for the fixed graph operator: y = P x (+ add), and the chained
// three-hop pipeline built on it.
//
// Replaces the cuSPARSE SpMM calls of the reference MultiHopCsrPlan
// (multihop_csr_ext/multihop_csr_pipeline_cuda.cu:264-321) and the
// torch.sparse.mm recurrence of FixedCSRSpMMFunction (model.py:57-106).
//
// Layout: x, add, y are row-major [n_rows, ld] (fp32 or bf16 storage, fp32
// accumulation); P is CSR with int32 row pointer / column index and fp32
// values. One launch handles a column tile [c0, c0 + tile) of width <= 256
// chunks per lane-row; wider matrices are tiled by the host.
//
// Work decomposition (schedule.h): a wavefront owns a light row; the wave's
// lanes are split into G = 64 / L groups of L lanes, each group gathering a
// different neighbour row with 16-byte loads (lane l of a group owns chunks
// l, l + L, ...), so G edges are in flight per step and U steps are unrolled.
// Heavy rows are cut into 256-edge segments, one workgroup each (one 64-edge
// tile per wave); segment results merge through `partial` in segment order.
#include "common.h"
#include "schedule.h"

namespace cign {
namespace {

constexpr int kTile = 64;          // edges staged per wave per tile
constexpr int kSegEdges = kWavesPerBlock * kTile;  // 256 edges per segment

template <typename T, int W, int VPL>
struct SpmmArgs {
  int ld;       // row stride of x / add / y (elements)
  int c0;       // first column of this tile
  int nch;      // chunks (of W elements) in this tile
  int L;        // lanes per group (power of two, L * VPL >= nch)
  int lgL;      // log2(L)
  const int32_t* rowptr;
  const int32_t* col;
  const float* val;
  const T* x;
  const T* add;  // may be null
  T* y;
  float* partial;   // [n_seg, nch * W] scratch for multi-segment rows
  int32_t* counters;  // [n_hrow], zero on entry, left zero on exit
};

// Accumulates sum_e val[e] * x[col[e], chunks] over edges [eb, ee) (at most
// kTile of them) into acc. Lanes of group g handle edges g, g + G, ...
template <typename T, int W, int VPL, int U>
__device__ __forceinline__ void gather_tile(const SpmmArgs<T, W, VPL>& a, int eb, int ee,
                                            float (&acc)[VPL][W]) {
  const int lane = lane_id();
  const int G = kWave >> a.lgL;
  const int g = lane >> a.lgL;
  const int gl = lane & (a.L - 1);
  const int cnt = ee - eb;
  int jj = 0;
  float vv = 0.0f;
  if (lane < cnt) {
    jj = a.col[eb + lane];
    vv = a.val[eb + lane];
  }
  for (int k = 0; k < cnt; k += G * U) {
    float buf[U][VPL][W];
    float wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int src = k + u * G + g;  // < 64 because G * U divides 64
      const int j = shfl(jj, src);
      wv[u] = shfl(vv, src);
      const bool ok = src < cnt;
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        const int c = gl + (v << a.lgL);
        if (ok && c < a.nch) {
          const T* p = a.x + static_cast<int64_t>(j) * a.ld + a.c0 + c * W;
          Chunk<T, W>::load(p, buf[u][v]);
        } else {
#pragma unroll
          for (int w = 0; w < W; ++w) buf[u][v][w] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int v = 0; v < VPL; ++v)
#pragma unroll
        for (int w = 0; w < W; ++w) acc[v][w] = fmaf(wv[u], buf[u][v][w], acc[v][w]);
  }
}

template <typename T, int W, int VPL>
__device__ __forceinline__ void group_reduce(const SpmmArgs<T, W, VPL>& a, float (&acc)[VPL][W]) {
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int w = 0; w < W; ++w) acc[v][w] = sum_across(acc[v][w], a.L);
}

template <typename T, int W, int VPL>
__device__ __forceinline__ void write_row(const SpmmArgs<T, W, VPL>& a, int row, const float (&acc)[VPL][W]) {
  const int lane = lane_id();
  if (lane >= a.L) return;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = lane + (v << a.lgL);
    if (c < a.nch) {
      const int64_t off = static_cast<int64_t>(row) * a.ld + a.c0 + c * W;
      float out[W];
#pragma unroll
      for (int w = 0; w < W; ++w) out[w] = acc[v][w];
      if (a.add) {
        float ad[W];
        Chunk<T, W>::load(a.add + off, ad);
#pragma unroll
        for (int w = 0; w < W; ++w) out[w] += ad[w];
      }
      Chunk<T, W>::store(a.y + off, out);
    }
  }
}

template <typename T, int W, int VPL, int U>
__global__ __launch_bounds__(kBlock) void spmm_kernel(SpmmArgs<T, W, VPL> a, Sched s) {
  const int lane = lane_id();
  const int wave = wave_id();
  const int b = blockIdx.x;
  float acc[VPL][W];
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int w = 0; w < W; ++w) acc[v][w] = 0.0f;

  if (b >= s.n_seg) {
    // Light rows: one per wave.
    const int li = (b - s.n_seg) * kWavesPerBlock + wave;
    if (li >= s.n_light) return;
    const int row = s.light[li];
    const int eb = a.rowptr[row], ee = a.rowptr[row + 1];
    for (int t = eb; t < ee; t += kTile) gather_tile<T, W, VPL, U>(a, t, min(ee, t + kTile), acc);
    group_reduce(a, acc);
    write_row(a, row, acc);
    return;
  }

  // Heavy-row segment: one 64-edge tile per wave, reduced through LDS.
  __shared__ float red[kWavesPerBlock][VPL * W * kWave];
  __shared__ int flag;
  const int4 sg = s.seg[b];
  const int row = sg.x;
  for (int t = sg.y + wave * kTile; t < sg.z; t += kSegEdges)
    gather_tile<T, W, VPL, U>(a, t, min(sg.z, t + kTile), acc);
  group_reduce(a, acc);
  const int width = a.nch * W;  // fp32 columns in this tile
  if (lane < a.L) {
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int c = lane + (v << a.lgL);
      if (c < a.nch)
#pragma unroll
        for (int w = 0; w < W; ++w) red[wave][c * W + w] = acc[v][w];
    }
  }
  __syncthreads();
  const int2 hr = s.hrow[sg.w];
  if (hr.y == 1) {
    // Single segment: combine the four waves and write the row directly.
    for (int c = threadIdx.x; c < width; c += kBlock) {
      float t = red[0][c] + red[1][c] + red[2][c] + red[3][c];
      const int64_t off = static_cast<int64_t>(row) * a.ld + a.c0 + c;
      if (a.add) t += to_f32(a.add[off]);
      a.y[off] = from_f32<T>(t);
    }
    return;
  }
  float* mine = a.partial + static_cast<int64_t>(b) * width;
  for (int c = threadIdx.x; c < width; c += kBlock) mine[c] = red[0][c] + red[1][c] + red[2][c] + red[3][c];
  if (!arrive_last(a.counters + sg.w, hr.y, &flag)) return;
  for (int c = threadIdx.x; c < width; c += kBlock) {
    float t = 0.0f;
    for (int q = 0; q < hr.y; ++q) t += a.partial[static_cast<int64_t>(hr.x + q) * width + c];
    const int64_t off = static_cast<int64_t>(row) * a.ld + a.c0 + c;
    if (a.add) t += to_f32(a.add[off]);
    a.y[off] = from_f32<T>(t);
  }
}

inline int ilog2(int v) {
  int r = 0;
  while ((1 << r) < v) ++r;
  return r;
}

template <typename T, int W, int VPL>
int launch_tile(hipStream_t stream, const Sched& s, int ld, int c0, int nch, const int32_t* rowptr,
                const int32_t* col, const float* val, const T* x, const T* add, T* y, float* partial,
                int32_t* counters) {
  SpmmArgs<T, W, VPL> a;
  a.ld = ld;
  a.c0 = c0;
  a.nch = nch;
  const int lanes_needed = (nch + VPL - 1) / VPL;
  a.lgL = ilog2(lanes_needed < 1 ? 1 : lanes_needed);
  a.L = 1 << a.lgL;
  a.rowptr = rowptr;
  a.col = col;
  a.val = val;
  a.x = x;
  a.add = add;
  a.y = y;
  a.partial = partial;
  a.counters = counters;
  const int blocks = sched_blocks(s);
  if (blocks == 0) return kOk;
  // Unroll U steps so that a 64-edge tile needs as few dependent gather
  // rounds as possible (G * U <= 64) while keeping at most 16 chunks of loads
  // in flight per lane.
  const int G = kWave / a.L;
  const int cap = 16 / VPL;
  const int U = min(cap, kWave / G);
  switch (U) {
    case 16: hipLaunchKernelGGL((spmm_kernel<T, W, VPL, 16>), dim3(blocks), dim3(kBlock), 0, stream, a, s); break;
    case 8: hipLaunchKernelGGL((spmm_kernel<T, W, VPL, 8>), dim3(blocks), dim3(kBlock), 0, stream, a, s); break;
    case 4: hipLaunchKernelGGL((spmm_kernel<T, W, VPL, 4>), dim3(blocks), dim3(kBlock), 0, stream, a, s); break;
    case 2: hipLaunchKernelGGL((spmm_kernel<T, W, VPL, 2>), dim3(blocks), dim3(kBlock), 0, stream, a, s); break;
    default: hipLaunchKernelGGL((spmm_kernel<T, W, VPL, 1>), dim3(blocks), dim3(kBlock), 0, stream, a, s); break;
  }
  return check_launch("cign_spmm");
}

template <typename T, int W>
int launch_all(hipStream_t stream, const Sched& s, int ld, const int32_t* rowptr, const int32_t* col,
               const float* val, const T* x, const T* add, T* y, float* partial, int32_t* counters) {
  const int total_ch = ld / W;
  constexpr int kMaxCh = kWave * 4;  // chunks per tile
  for (int ch0 = 0; ch0 < total_ch; ch0 += kMaxCh) {
    const int nch = min(kMaxCh, total_ch - ch0);
    int rc;
    if (nch <= kWave) {
      rc = launch_tile<T, W, 1>(stream, s, ld, ch0 * W, nch, rowptr, col, val, x, add, y, partial, counters);
    } else if (nch <= 2 * kWave) {
      rc = launch_tile<T, W, 2>(stream, s, ld, ch0 * W, nch, rowptr, col, val, x, add, y, partial, counters);
    } else {
      rc = launch_tile<T, W, 4>(stream, s, ld, ch0 * W, nch, rowptr, col, val, x, add, y, partial, counters);
    }
    if (rc != kOk) return rc;
  }
  return kOk;
}

template <typename T>
int spmm_dispatch(hipStream_t stream, const Sched& s, int d, const int32_t* rowptr, const int32_t* col,
                  const float* val, const void* x, const void* add, void* y, float* partial,
                  int32_t* counters) {
  constexpr int kVec = 16 / sizeof(T);
  const T* xt = static_cast<const T*>(x);
  const T* at = static_cast<const T*>(add);
  T* yt = static_cast<T*>(y);
  const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
                       (add == nullptr || reinterpret_cast<uintptr_t>(add) % 16 == 0);
  if (d % kVec == 0 && aligned) {
    return launch_all<T, kVec>(stream, s, d, rowptr, col, val, xt, at, yt, partial, counters);
  }
  return launch_all<T, 1>(stream, s, d, rowptr, col, val, xt, at, yt, partial, counters);
}

}  // namespace
}  // namespace cign

using namespace cign;

extern "C" {

// Bytes of fp32 scratch `partial` needed by cign_spmm for a schedule with
// n_seg segments and d dense columns.
int64_t cign_spmm_partial_bytes(int32_t n_seg, int32_t d) {
  const int64_t tile = static_cast<int64_t>(d < kWave * 4 * 8 ? d : kWave * 4 * 8);
  return static_cast<int64_t>(n_seg) * tile * 4;
}

// y = P x (+ add). See spmm.hip header for layout. Replaces one cusparseSpMM
// (multihop_csr_ext/multihop_csr_pipeline_cuda.cu:264-285) or one
// torch.sparse.mm (model.py:91,101).
int cign_spmm(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* rowptr,
              const int32_t* col, const float* val, const int32_t* sched, int32_t n_light, int32_t n_seg,
              int32_t n_hrow, const void* x, const void* add, void* y, float* partial, int32_t* counters) {
  if (n_rows < 0 || d <= 0) return set_error(kInvalid, "cign_spmm: bad sizes n_rows=%d d=%d", n_rows, d);
  if (n_light + n_hrow != n_rows) return set_error(kInvalid, "cign_spmm: schedule does not cover %d rows", n_rows);
  if (!rowptr || !col || !val || !sched || !x || !y) return set_error(kInvalid, "cign_spmm: null pointer");
  if (n_seg > 0 && (!partial || !counters)) return set_error(kInvalid, "cign_spmm: heavy rows need partial/counters");
  const Sched s = make_sched(sched, n_light, n_seg, n_hrow);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == kF32) return spmm_dispatch<float>(st, s, d, rowptr, col, val, x, add, y, partial, counters);
  if (dtype == kBF16) return spmm_dispatch<bf16>(st, s, d, rowptr, col, val, x, add, y, partial, counters);
  return set_error(kInvalid, "cign_spmm: unsupported dtype %d", dtype);
}

// Three chained hops without host work: y1 = P x, y2 = P y1, y3 = P y2.
// Replaces MultiHopCsrPlan::forward3 (multihop_csr_pipeline_cuda.cu:287-297).
int cign_spmm_fwd3(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* rowptr,
                   const int32_t* col, const float* val, const int32_t* sched, int32_t n_light, int32_t n_seg,
                   int32_t n_hrow, const void* x, void* y1, void* y2, void* y3, float* partial,
                   int32_t* counters) {
  int rc = cign_spmm(stream, dtype, n_rows, d, rowptr, col, val, sched, n_light, n_seg, n_hrow, x, nullptr, y1,
                     partial, counters);
  if (rc) return rc;
  rc = cign_spmm(stream, dtype, n_rows, d, rowptr, col, val, sched, n_light, n_seg, n_hrow, y1, nullptr, y2,
                 partial, counters);
  if (rc) return rc;
  return cign_spmm(stream, dtype, n_rows, d, rowptr, col, val, sched, n_light, n_seg, n_hrow, y2, nullptr, y3,
                   partial, counters);
}

// Chain-rule backward on P^T with the "+ g_k" adds fused into the SpMM
// epilogue: t2 = g2 + P^T g3, t1 = g1 + P^T t2, gx = P^T t1.
// Replaces MultiHopCsrPlan::backward3 (multihop_csr_pipeline_cuda.cu:299-321).
int cign_spmm_bwd3(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* rowptr,
                   const int32_t* col, const float* val, const int32_t* sched, int32_t n_light, int32_t n_seg,
                   int32_t n_hrow, const void* g1, const void* g2, const void* g3, void* t2, void* t1, void* gx,
                   float* partial, int32_t* counters) {
  int rc = cign_spmm(stream, dtype, n_rows, d, rowptr, col, val, sched, n_light, n_seg, n_hrow, g3, g2, t2,
                     partial, counters);
  if (rc) return rc;
  rc = cign_spmm(stream, dtype, n_rows, d, rowptr, col, val, sched, n_light, n_seg, n_hrow, t2, g1, t1, partial,
                 counters);
  if (rc) return rc;
  return cign_spmm(stream, dtype, n_rows, d, rowptr, col, val, sched, n_light, n_seg, n_hrow, t1, nullptr, gx,
                   partial, counters);
}

}  // extern "C"
