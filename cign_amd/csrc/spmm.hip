// CSR SpMM for the fixed graph operator: y = P x (+ add), and the chained
// three-hop pipeline built on it.
//
// Replaces the cuSPARSE SpMM calls of the reference MultiHopCsrPlan
// (multihop_csr_ext/multihop_csr_pipeline_cuda.cu:264-321) and the
// torch.sparse.mm recurrence of FixedCSRSpMMFunction (model.py:57-106).
//
// Layout: x, add, y are row-major [n_rows, ld] (fp32 or bf16 storage, fp32
// accumulation); P is CSR with int32 row pointer / column index and fp32
// values. One launch handles a column tile of at most 256 16-byte chunks per
// row; wider matrices are tiled by the host.
//
// A row's output is owned by a group of L lanes (L = power of two covering
// the tile's chunks, 16-byte loads, lane l owns chunks l, l + L, ...). Three
// work shapes, from the degree-sorted schedule (schedule.h):
//   tiny rows   (degree <= L):  one row per lane group, G = 64 / L rows per
//                               wavefront; one col/val load, then the row's
//                               gathers in one batch;
//   medium rows (<= 64 edges):  one row per wavefront, its G groups split the
//                               edges, reduced with a butterfly;
//   heavy rows:                 segments (512 edges by the host default), one
//                               workgroup each, in rounds of 64 edges per
//                               wave; multi-segment rows merge through
//                               `partial` in segment order.
// A batch's gathers are unconditional (indices clamped to a valid edge,
// weight zero) so they all issue before the first is consumed; its size is
// the wavefront's largest per-group edge count rounded up to a power of two.
#include <mutex>

#include "common.h"
#include "schedule.h"

namespace cign {
namespace {

// Workgroup shape of the SpMM: kSpmmWaves wavefronts; a heavy-row segment is
// processed in rounds of kSpmmWaves x 64 edges.
#ifndef CIGN_SPMM_WAVES
#define CIGN_SPMM_WAVES 8
#endif
constexpr int kSpmmWaves = CIGN_SPMM_WAVES;
// Chunks in flight per lane (a batch of U edges x VPL chunks), and the
// smallest number of chunks a lane owns per row (more rows per wavefront).
#ifndef CIGN_SPMM_INFLIGHT
#define CIGN_SPMM_INFLIGHT 8
#endif
#ifndef CIGN_SPMM_MIN_VPL
#define CIGN_SPMM_MIN_VPL 1
#endif
constexpr int kSpmmInflight = CIGN_SPMM_INFLIGHT;
constexpr int kSpmmMinVpl = CIGN_SPMM_MIN_VPL;
constexpr int kSpmmBlock = kSpmmWaves * kWave;
constexpr int kTile = 64;
constexpr int kSegEdges = kSpmmWaves * kTile;

template <typename T, int W, int VPL>
struct SpmmArgs {
  int ld;       // row stride of x / add / y (elements)
  int c0;       // first column of this tile
  int nch;      // chunks (of W elements) in this tile
  int L;        // lanes per group (power of two, L * VPL >= nch)
  int lgL;      // log2(L)
  int n_mid;    // light rows processed one per wavefront (the first n_mid)
  int mid_blocks;
  const int32_t* col;
  const float* val;
  const T* x;
  const T* add;  // may be null
  T* y;
  float* partial;     // [n_seg, nch * W] scratch for multi-segment rows
  int32_t* counters;  // [n_hrow], zero on entry, left zero on exit
};

template <typename T, int W, int VPL>
__device__ __forceinline__ void zero(float (&acc)[VPL][W]) {
#pragma unroll
  for (int v = 0; v < VPL; ++v)
#pragma unroll
    for (int w = 0; w < W; ++w) acc[v][w] = 0.0f;
}

// Raw chunks of x[j] owned by lane gl (zero past the tile).
template <typename T, int W, int VPL>
__device__ __forceinline__ void load_row(const SpmmArgs<T, W, VPL>& a, int j, int gl,
                                         typename Chunk<T, W>::Raw (&buf)[VPL]) {
  const T* base = a.x + static_cast<int64_t>(j) * a.ld + a.c0;
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = gl + (v << a.lgL);
    buf[v] = c < a.nch ? Chunk<T, W>::load_raw(base + c * W) : Chunk<T, W>::zero_raw();
  }
}

// Batches of U edge slots of a lane group: slot u = first + (k0 + k) * step,
// valid while u < cnt, whose column index and weight lane (base + u) holds in
// jj / vv. Every gather of a batch is issued before any is consumed; slots
// past the end reload an edge of the group with weight 0.
template <typename T, int W, int VPL>
struct SpmmBatches {
  const SpmmArgs<T, W, VPL>& a;
  int jj;
  float vv;
  int base, first, step, cnt, gl;
  float (&acc)[VPL][W];

  template <int U>
  __device__ __forceinline__ void run(int k0) {
    typename Chunk<T, W>::Raw buf[U][VPL];
    float wv[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const int src = (base + (u < cnt ? u : 0)) & (kWave - 1);
      const float v = shfl(vv, src);
      wv[k] = u < cnt ? v : 0.0f;
      load_row(a, shfl(jj, src), gl, buf[k]);
    }
#pragma unroll
    for (int k = 0; k < U; ++k)
#pragma unroll
      for (int v = 0; v < VPL; ++v) {
        float f[W];
        Chunk<T, W>::unpack(buf[k][v], f);
#pragma unroll
        for (int w = 0; w < W; ++w) acc[v][w] = fmaf(wv[k], f[w], acc[v][w]);
      }
  }
};

// Largest of v over the lane groups of a wavefront (runtime group size L).
__device__ __forceinline__ int wave_max_over_groups(int v, int L) {
  for (int o = L; o < kWave; o <<= 1) v = max(v, shfl_xor_i(v, o));
  return v;
}

// Gathers `need` (wave-uniform) slots per lane group, at most kSpmmInflight
// chunks in flight per lane.
template <typename T, int W, int VPL>
__device__ __forceinline__ void gather(const SpmmArgs<T, W, VPL>& a, int jj, float vv, int base, int first, int step,
                                       int cnt, int need, int gl, float (&acc)[VPL][W]) {
  SpmmBatches<T, W, VPL> sb{a, jj, vv, base, first, step, cnt, gl, acc};
  for_batches<(kSpmmInflight / VPL > 0 ? kSpmmInflight / VPL : 1)>(need, sb);
}

// The add row's chunks of a light row, loaded once the row is known and
// before its gathers (at the write they were one more memory round trip
// after the gathers, on every hop with a fused add). Chunks past the tile
// read the tile's last chunk (never used).
template <typename T, int W, int VPL>
struct AddRow {
  typename Chunk<T, W>::Raw raw[VPL];
  __device__ __forceinline__ void load(const SpmmArgs<T, W, VPL>& a, int row, int gl) {
    if (!a.add) return;  // uniform
    const T* base = a.add + static_cast<int64_t>(row) * a.ld + a.c0;
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
      const int c = min(gl + (v << a.lgL), a.nch - 1);
      raw[v] = Chunk<T, W>::load_raw(base + c * W);
    }
  }
};

template <typename T, int W, int VPL>
__device__ __forceinline__ void write_row(const SpmmArgs<T, W, VPL>& a, int row, int gl, const float (&acc)[VPL][W],
                                          const AddRow<T, W, VPL>& ar) {
#pragma unroll
  for (int v = 0; v < VPL; ++v) {
    const int c = gl + (v << a.lgL);
    if (c < a.nch) {
      const int64_t off = static_cast<int64_t>(row) * a.ld + a.c0 + c * W;
      float out[W];
#pragma unroll
      for (int w = 0; w < W; ++w) out[w] = acc[v][w];
      if (a.add) {
        float ad[W];
        Chunk<T, W>::unpack(ar.raw[v], ad);
#pragma unroll
        for (int w = 0; w < W; ++w) out[w] += ad[w];
      }
      Chunk<T, W>::store(a.y + off, out);
    }
  }
}

template <typename T, int W, int VPL>
__global__ __launch_bounds__(kSpmmBlock) void spmm_kernel(SpmmArgs<T, W, VPL> a, Sched s) {
  const int lane = lane_id();
  const int wave = wave_id();
  const int gl = lane & (a.L - 1);
  const int G = kWave >> a.lgL;
  const int g = lane >> a.lgL;
  int b = blockIdx.x;
  float acc[VPL][W];
  zero<T, W, VPL>(acc);

  if (b >= s.n_seg) {
    b -= s.n_seg;
    if (b < a.mid_blocks) {
      // Medium row (L < degree <= 64): one per wavefront, group g takes edges
      // g, g + G, ...
      const int li = b * kSpmmWaves + wave;
      if (li >= a.n_mid) return;
      const int4 r = s.light[li];
      const int deg = r.z - r.y;
      const bool mine = lane < deg;
      const int jj = mine ? a.col[r.y + lane] : 0;
      const float vv = mine ? a.val[r.y + lane] : 0.0f;
      AddRow<T, W, VPL> ar;
      ar.load(a, r.x, gl);
      gather(a, jj, vv, 0, g, G, deg, (deg + G - 1) / G, gl, acc);
      sum_across_n(acc, a.L);
      if (lane < a.L) write_row(a, r.x, gl, acc, ar);
      return;
    }
    // Tiny rows (degree <= L): one per lane group.
    const int li = a.n_mid + ((b - a.mid_blocks) * kSpmmWaves + wave) * G + g;
    const bool has = li < s.n_light;
    const int4 r = has ? s.light[li] : make_int4(0, 0, 0, 0);
    const int deg = r.z - r.y;
    const bool mine = gl < deg;
    const int jj = mine ? a.col[r.y + gl] : 0;
    const float vv = mine ? a.val[r.y + gl] : 0.0f;
    AddRow<T, W, VPL> ar;
    ar.load(a, r.x, gl);  // (row 0 for a group with no row: read, unused)
    gather(a, jj, vv, g << a.lgL, 0, 1, deg, wave_max_over_groups(deg, a.L), gl, acc);
    if (has) write_row(a, r.x, gl, acc, ar);
    return;
  }

  // Heavy-row segment: wave w takes the segment's edges [64w, 64w + 64) of
  // every 256-edge round, reduced through LDS.
  __shared__ float red[kSpmmWaves][VPL * W * kWave];
  __shared__ int flag;
  const int4 sg = s.seg[b];
  const int row = sg.x;
  // Rounds of 4 x 64 edges when the schedule's segments are longer than 256.
  // The next round's indices and weights are loaded before this round's
  // gathers, so a round waits on one memory latency instead of two.
  int tb = sg.y + wave * kTile;
  int jj = tb + lane < sg.z ? a.col[tb + lane] : 0;
  float vv = tb + lane < sg.z ? a.val[tb + lane] : 0.0f;
  for (; tb < sg.z; tb += kSegEdges) {
    const int cnt = min(kTile, sg.z - tb);
    const int tn = tb + kSegEdges + lane;
    const int jn = tn < sg.z ? a.col[tn] : 0;
    const float vn = tn < sg.z ? a.val[tn] : 0.0f;
    gather(a, jj, vv, 0, g, G, cnt, (cnt + G - 1) / G, gl, acc);
    jj = jn;
    vv = vn;
  }
  sum_across_n(acc, a.L);
  const int width = a.nch * W;
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
    for (int c = threadIdx.x; c < width; c += kSpmmBlock) {
      float t = 0.0f;
#pragma unroll
      for (int v = 0; v < kSpmmWaves; ++v) t += red[v][c];
      const int64_t off = static_cast<int64_t>(row) * a.ld + a.c0 + c;
      if (a.add) t += to_f32(a.add[off]);
      a.y[off] = from_f32<T>(t);
    }
    return;
  }
  float* part = a.partial + static_cast<int64_t>(b) * width;
  for (int c = threadIdx.x; c < width; c += kSpmmBlock) {
    float t = 0.0f;
#pragma unroll
    for (int v = 0; v < kSpmmWaves; ++v) t += red[v][c];
    st_agent(part + c, t);
  }
  if (!arrive_last(a.counters + sg.w, hr.y, &flag)) return;
  for (int c = threadIdx.x; c < width; c += kSpmmBlock) {
    float t = 0.0f;
    for (int q = 0; q < hr.y; ++q) t += ld_agent(a.partial + static_cast<int64_t>(hr.x + q) * width + c);
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

struct SchedInfo {
  const int32_t* hdr;
  int n_light, n_seg, n_hrow;
};

inline SchedInfo read_info(const int32_t* hdr) { return SchedInfo{hdr, hdr[0], hdr[1], hdr[2]}; }

template <typename T, int W, int VPL>
int launch_tile(hipStream_t stream, const Sched& s, const SchedInfo& info, int ld, int c0, int nch,
                const int32_t* col, const float* val, const T* x, const T* add, T* y, float* partial,
                int32_t* counters) {
  SpmmArgs<T, W, VPL> a;
  a.ld = ld;
  a.c0 = c0;
  a.nch = nch;
  const int lanes_needed = (nch + VPL - 1) / VPL;
  a.lgL = ilog2(lanes_needed < 1 ? 1 : lanes_needed);
  a.L = 1 << a.lgL;
  a.col = col;
  a.val = val;
  a.x = x;
  a.add = add;
  a.y = y;
  a.partial = partial;
  a.counters = counters;
  const int G = kWave / a.L;
  // Rows with degree <= L go one per lane group (tiny); the rest of the
  // light list (sorted by degree, descending) one per wavefront.
  const int n_mid = (G > 1 && a.L >= 8) ? sched_count_gt(info.hdr, a.L) : info.n_light;
  a.n_mid = n_mid;
  a.mid_blocks = (n_mid + kSpmmWaves - 1) / kSpmmWaves;
  const int n_tiny = info.n_light - n_mid;
  const int tiny_blocks = (n_tiny + kSpmmWaves * G - 1) / (kSpmmWaves * G);
  const int blocks = s.n_seg + a.mid_blocks + tiny_blocks;
  if (blocks == 0) return kOk;
  hipLaunchKernelGGL((spmm_kernel<T, W, VPL>), dim3(blocks), dim3(kSpmmBlock), 0, stream, a, s);
  return check_launch("cign_spmm");
}

template <typename T, int W>
int launch_all(hipStream_t stream, const Sched& s, const SchedInfo& info, int ld, const int32_t* col,
               const float* val, const T* x, const T* add, T* y, float* partial, int32_t* counters) {
  const int total_ch = ld / W;
  constexpr int kMaxCh = kWave * 4;  // chunks per tile
  for (int ch0 = 0; ch0 < total_ch; ch0 += kMaxCh) {
    const int nch = min(kMaxCh, total_ch - ch0);
    int rc;
    if (nch <= kWave && kSpmmMinVpl <= 1) {
      rc = launch_tile<T, W, 1>(stream, s, info, ld, ch0 * W, nch, col, val, x, add, y, partial, counters);
    } else if (nch <= 2 * kWave && kSpmmMinVpl <= 2) {
      rc = launch_tile<T, W, 2>(stream, s, info, ld, ch0 * W, nch, col, val, x, add, y, partial, counters);
    } else {
      rc = launch_tile<T, W, 4>(stream, s, info, ld, ch0 * W, nch, col, val, x, add, y, partial, counters);
    }
    if (rc != kOk) return rc;
  }
  return kOk;
}

template <typename T>
int spmm_dispatch(hipStream_t stream, const Sched& s, const SchedInfo& info, int d, const int32_t* col,
                  const float* val, const void* x, const void* add, void* y, float* partial, int32_t* counters) {
  constexpr int kVec = 16 / sizeof(T);
  const T* xt = static_cast<const T*>(x);
  const T* at = static_cast<const T*>(add);
  T* yt = static_cast<T*>(y);
  const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
                       (add == nullptr || reinterpret_cast<uintptr_t>(add) % 16 == 0);
  if (d % kVec == 0 && aligned) {
    return launch_all<T, kVec>(stream, s, info, d, col, val, xt, at, yt, partial, counters);
  }
  return launch_all<T, 1>(stream, s, info, d, col, val, xt, at, yt, partial, counters);
}

__global__ __launch_bounds__(kBlock) void zero_i32_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i < n) p[i] = 0;
}

}  // namespace
}  // namespace cign

// Scratch of cign_spmm_fwd3_noalloc: kNoAllocCounterInts int32 merge
// counters, then the segment partial sums of multi-segment rows. Each GPU
// the library runs on holds its own copy until the process ends. In host
// code `scratch` names a host-side stand-in, never the device memory: host
// code uses only the address hipGetSymbolAddress returns for the current
// device (noalloc_scratch below).
constexpr int64_t kNoAllocScratchBytes = 16ll << 20;
constexpr int64_t kNoAllocCounterInts = 1ll << 18;
constexpr int64_t kNoAllocPartialBytes = kNoAllocScratchBytes - kNoAllocCounterInts * 4;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace cign {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, looked up once per device
// and kept for the life of the process: a hipDeviceReset (or unloading the
// library's code object) invalidates it, and the entry point must not be
// called on that device afterwards.
int noalloc_scratch(const char* what, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(kHipError, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(kInvalid, "%s: device ordinal %d out of range", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      return set_error(kHipError, "%s: hipGetSymbolAddress(scratch) on device %d: %s", what, dev,
                       hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return kOk;
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

// y = P x (+ add). Replaces one cusparseSpMM of MultiHopCsrPlan::spmm
// (multihop_csr_ext/multihop_csr_pipeline_cuda.cu:264-285) or one
// torch.sparse.mm (model.py:91,101).
int cign_spmm(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* col, const float* val,
              const int32_t* sched, const int32_t* sched_info, const void* x, const void* add, void* y,
              float* partial, int32_t* counters) {
  if (n_rows < 0 || d <= 0) return set_error(kInvalid, "cign_spmm: bad sizes n_rows=%d d=%d", n_rows, d);
  if (!sched_info) return set_error(kInvalid, "cign_spmm: null schedule header");
  const SchedInfo info = read_info(sched_info);
  if (info.n_light + info.n_hrow != n_rows) return set_error(kInvalid, "cign_spmm: schedule does not cover %d rows", n_rows);
  if (!sched || !x || !y) return set_error(kInvalid, "cign_spmm: null pointer");
  if (info.n_seg > 0 && (!partial || !counters)) return set_error(kInvalid, "cign_spmm: heavy rows need partial/counters");
  const Sched s = make_sched(sched, info.n_light, info.n_seg, info.n_hrow);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == kF32) return spmm_dispatch<float>(st, s, info, d, col, val, x, add, y, partial, counters);
  if (dtype == kBF16) return spmm_dispatch<bf16>(st, s, info, d, col, val, x, add, y, partial, counters);
  return set_error(kInvalid, "cign_spmm: unsupported dtype %d", dtype);
}

// Three chained hops without host work: y1 = P x, y2 = P y1, y3 = P y2.
// Replaces MultiHopCsrPlan::forward3 (multihop_csr_pipeline_cuda.cu:287-297).
int cign_spmm_fwd3(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* col, const float* val,
                   const int32_t* sched, const int32_t* sched_info, const void* x, void* y1, void* y2, void* y3,
                   float* partial, int32_t* counters) {
  int rc = cign_spmm(stream, dtype, n_rows, d, col, val, sched, sched_info, x, nullptr, y1, partial, counters);
  if (rc) return rc;
  rc = cign_spmm(stream, dtype, n_rows, d, col, val, sched, sched_info, y1, nullptr, y2, partial, counters);
  if (rc) return rc;
  return cign_spmm(stream, dtype, n_rows, d, col, val, sched, sched_info, y2, nullptr, y3, partial, counters);
}

// Chain-rule backward on P^T with the "+ g_k" adds fused into the SpMM
// epilogue: t2 = g2 + P^T g3, t1 = g1 + P^T t2, gx = P^T t1.
// Replaces MultiHopCsrPlan::backward3 (multihop_csr_pipeline_cuda.cu:299-321).
int cign_spmm_bwd3(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* col, const float* val,
                   const int32_t* sched, const int32_t* sched_info, const void* g1, const void* g2, const void* g3,
                   void* t2, void* t1, void* gx, float* partial, int32_t* counters) {
  int rc = cign_spmm(stream, dtype, n_rows, d, col, val, sched, sched_info, g3, g2, t2, partial, counters);
  if (rc) return rc;
  rc = cign_spmm(stream, dtype, n_rows, d, col, val, sched, sched_info, t2, g1, t1, partial, counters);
  if (rc) return rc;
  return cign_spmm(stream, dtype, n_rows, d, col, val, sched, sched_info, t1, nullptr, gx, partial, counters);
}

// cign_spmm_fwd3 with its partial sums and merge counters in the library's
// own per-GPU scratch, so the call allocates nothing. The counters are
// cleared by a fill kernel on `stream` first. Calls that overlap on one GPU
// (different streams or threads) share the scratch and race.
int cign_spmm_fwd3_noalloc(void* stream, int32_t dtype, int32_t n_rows, int32_t d, const int32_t* col,
                           const float* val, const int32_t* sched, const int32_t* sched_info, const void* x,
                           void* y1, void* y2, void* y3) {
  static const char* kWhat = "cign_spmm_fwd3_noalloc";
  if (!sched_info) return set_error(kInvalid, "%s: null schedule header", kWhat);
  if (d <= 0) return set_error(kInvalid, "%s: bad dense width d=%d", kWhat, d);
  const SchedInfo info = read_info(sched_info);
  if (info.n_seg < 0 || info.n_hrow < 0) return set_error(kInvalid, "%s: corrupt schedule header", kWhat);
  const int64_t counter_ints = static_cast<int64_t>(info.n_hrow) + 1;
  const int64_t partial_bytes = cign_spmm_partial_bytes(info.n_seg, d);
  if (counter_ints > kNoAllocCounterInts || partial_bytes > kNoAllocPartialBytes) {
    return set_error(kInvalid,
                     "%s: this schedule needs %lld merge counters and %lld bytes of partial sums; the built-in "
                     "scratch holds %lld counters and %lld bytes (use cign_spmm_fwd3 with caller workspace)",
                     kWhat, static_cast<long long>(counter_ints), static_cast<long long>(partial_bytes),
                     static_cast<long long>(kNoAllocCounterInts), static_cast<long long>(kNoAllocPartialBytes));
  }
  void* base = nullptr;
  int rc = noalloc_scratch(kWhat, &base);
  if (rc) return rc;
  int32_t* counters = static_cast<int32_t*>(base);
  float* partial = reinterpret_cast<float*>(static_cast<unsigned char*>(base) + kNoAllocCounterInts * 4);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nc = static_cast<int>(counter_ints);
  hipLaunchKernelGGL(zero_i32_kernel, dim3((nc + kBlock - 1) / kBlock), dim3(kBlock), 0, st, counters, nc);
  rc = check_launch(kWhat);
  if (rc) return rc;
  return cign_spmm_fwd3(stream, dtype, n_rows, d, col, val, sched, sched_info, x, y1, y2, y3, partial, counters);
}

}  // extern "C"
