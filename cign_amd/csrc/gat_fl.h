// Collapsed GAT, feature layout: the gfx950 fast path for H <= 8 heads and C
// a multiple of the 16-byte chunk width W (4 fp32 or 8 bf16 values) with C/W
// a power of two and H*C/W <= 64 chunks. Semantics are those stated at the top
// of gat_kernels.h (reference collapsed_gat_cuda.cu:34-430).
//
// Geometry (shared with the SpMM, schedule.h built with light_max = 64 and a
// segment length that is a multiple of 256). A group of L = pow2ceil(H*C/W) lanes owns one row; lane q
// owns chunk q of a feature row, i.e. head hq = q / (C/W) and channel chunk
// cw = q % (C/W). Rows with degree <= L go one per group (64/L rows per
// wavefront), rows with degree <= 64 one per wavefront (its groups split the
// edges), heavier rows are segments (one 4-wave workgroup each, rounds of 256
// edges) whose partial results the last workgroup to finish merges in segment
// order.
//
// Every lane gathers, for each edge of its batch, the 16-byte chunk of the
// source feature row AND the source logit of its own head in the same memory
// round, right after the column index: the softmax is online (running max m,
// sum s and unnormalised accumulator rescaled per batch, flash style), so no
// lane-per-edge prologue, LDS staging or per-edge cross-lane reduction sits
// between the index load and the feature gather. A row costs one dependent
// round per level of indirection (schedule record -> column index -> source
// data). The batch size U (1..16) is the wavefront's largest per-group edge
// count rounded up to a power of two, so short rows issue few wasted loads.
//
// Backward without per-edge reductions. With g = g_pre[i] (= g_y SiLU'(pre)),
// s the softmax weight, kw = keep/(1-p) (1 without dropout), l' the
// LeakyReLU slope of the raw score and ge'_e = kw <g, x[j_e,h]>/H:
//   wsum_ih = sum_e s ge'          = <g, sum_e s kw x[j_e,h]> / H
//   A_ih    = sum_e s ge' l'       = <g, sum_e s kw l' x[j_e,h]> / H
//   grad_attn_row[i,h] = A - wsum * B,   B = sum_e s l'
// so the rows kernel accumulates two feature chunks per lane and reduces the
// dot products once per row. The columns kernel (CSC, column j) uses
//   grad_feat[j,h]     = sum_i s kw g_pre[i] / H
//   grad_attn_col[j,h] = <sum_i s l' kw g_pre[i], x[j,h]> / H - sum_i s l' wsum_i
// gathering per entry one 16-byte row record {attn_row, edge_max, 1/edge_sum,
// wsum} (written by the rows kernel) and the g_pre chunk. grad_bias is a
// deterministic two-level column sum of g_pre done by the columns kernel's
// trailing workgroups, so the rows kernel has no block barrier on light rows.
#pragma once

#include "gat_kernels.h"

namespace cign {
namespace gatk {

constexpr int kFlHeads = 8;

// Largest batch (edge slots gathered per lane before any is consumed) of
// each kernel; the cap trades loads in flight per wave for waves per SIMD.
#ifndef CIGN_FL_FWD_U
#define CIGN_FL_FWD_U 16
#endif
#ifndef CIGN_FL_ROWS_U
#define CIGN_FL_ROWS_U 16
#endif
#ifndef CIGN_FL_COLS_U
#define CIGN_FL_COLS_U 8
#endif
constexpr int kFwdU = CIGN_FL_FWD_U;
constexpr int kRowsU = CIGN_FL_ROWS_U;
constexpr int kColsU = CIGN_FL_COLS_U;

// Heavy rows are segments (one workgroup each; any multiple of 256 edges,
// chosen by the host from the graph size) processed in rounds of kSegRound =
// 4 waves x 64 edges. Longer segments mean fewer rows whose partial results
// need a cross-workgroup merge (an agent-scope release / acquire, which
// writes back and invalidates the L2 of the XCDs involved) at the cost of
// more rounds per workgroup.
constexpr int kFlLightMax = 64;
constexpr int kSegRound = kWavesPerBlock * kWave;

// grad_bias of the feature layout: the columns kernel's last
// ceil(n / 256) (at most kFlBiasBlocks) workgroups sum grad_pre rows.
constexpr int kFlBiasBlocks = 256;
inline int fl_bias_blocks(int n) { return max(1, min(kFlBiasBlocks, (n + 255) / 256)); }

template <typename T>
struct FlGeom {
  static constexpr int W = 16 / sizeof(T);
};

// Lane geometry of a group of L lanes (one row).
template <int L>
struct FlLane {
  int lane, g, gl, q, hq, cw;
  bool qv;
  __device__ __forceinline__ FlLane(int lgcq, int nq) {
    lane = lane_id();
    g = lane / L;
    gl = lane & (L - 1);
    qv = gl < nq;
    q = qv ? gl : 0;
    hq = q >> lgcq;
    cw = q & ((1 << lgcq) - 1);
  }
};

// W fp32 values from a 16-byte aligned address.
template <int W>
__device__ __forceinline__ void load_f32(const float* p, float (&v)[W]) {
#pragma unroll
  for (int k = 0; k < W; k += 4) {
    const float4 t = *reinterpret_cast<const float4*>(p + k);
    v[k] = t.x;
    v[k + 1] = t.y;
    v[k + 2] = t.z;
    v[k + 3] = t.w;
  }
}

template <int W>
__device__ __forceinline__ void store_f32(float* p, const float (&v)[W]) {
#pragma unroll
  for (int k = 0; k < W; k += 4) *reinterpret_cast<float4*>(p + k) = make_float4(v[k], v[k + 1], v[k + 2], v[k + 3]);
}

// Largest value of v over the groups of a wavefront (lane bits >= log2 L).
template <int L>
__device__ __forceinline__ int wave_group_max(int v) {
#pragma unroll
  for (int o = L; o < kWave; o <<= 1) v = max(v, shfl_xor_i(v, o));
  return v;
}

template <int L, int W>
__device__ __forceinline__ void group_sum(float (&v)[W]) {
#pragma unroll
  for (int o = L; o < kWave; o <<= 1)
#pragma unroll
    for (int w = 0; w < W; ++w) v[w] += shfl_xor(v[w], o);
}

template <int L>
__device__ __forceinline__ float group_sum1(float v) {
#pragma unroll
  for (int o = L; o < kWave; o <<= 1) v += shfl_xor(v, o);
  return v;
}

// Sum over the C/W lanes of a head (lane bits below log2(C/W)).
__device__ __forceinline__ float head_sum(float v, int cq) {
  for (int o = 1; o < cq; o <<= 1) v += shfl_xor(v, o);
  return v;
}

// ===========================================================================
// Forward
// ===========================================================================
// Online-softmax state of a lane: running max m, sum s and the unnormalised
// accumulators acc = sum p kw x, accl = sum p kw l' x, bl = sum p l' (p =
// exp(score - m)); accl and bl are the per-row aggregates the backward reads
// instead of gathering the source rows again.
template <int W>
struct FwdState {
  float m, s, bl;
  float acc[W], accl[W];
  __device__ __forceinline__ void clear() {
    m = kNegBig;
    s = 0.0f;
    bl = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) acc[w] = accl[w] = 0.0f;
  }
  __device__ __forceinline__ void scale(float f) {
    s *= f;
    bl *= f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      acc[w] *= f;
      accl[w] *= f;
    }
  }
  // state <- state (+) (m2, s2, bl2, acc2, accl2)
  __device__ __forceinline__ void merge(float m2, float s2, float bl2, const float (&acc2)[W],
                                        const float (&accl2)[W]) {
    const float mx = fmaxf(m, m2);
    const float f1 = expf(m - mx), f2 = expf(m2 - mx);
    s = s * f1 + s2 * f2;
    bl = bl * f1 + bl2 * f2;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      acc[w] = acc[w] * f1 + acc2[w] * f2;
      accl[w] = accl[w] * f1 + accl2[w] * f2;
    }
    m = mx;
  }
};

// Batches of U edge slots of a lane group: slot u = first + (k0 + k) * step,
// valid while u < cnt; its column index is held by lane (base + u) of the
// wavefront, its CSR edge id is ebase + u. DROP: edge dropout (p > 0).
template <typename T, int L, bool DROP>
struct FwdBatches {
  static constexpr int W = FlGeom<T>::W;
  const GatFwdArgs<T>& a;
  const FlLane<L>& ln;
  int jj, base, first, step, cnt, ebase;
  float ar;
  FwdState<W>& st;

  template <int U>
  __device__ __forceinline__ void run(int k0) {
    const int F = a.H * a.C;
    typename Chunk<T, W>::Raw xb[U];
    float sc[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const int j = shfl(jj, (base + (u < cnt ? u : 0)) & (kWave - 1));
      sc[k] = a.attn_col[static_cast<int64_t>(j) * a.H + ln.hq];
      xb[k] = Chunk<T, W>::load_raw(a.x + static_cast<int64_t>(j) * F + ln.q * W);
    }
    // sc[k] becomes the raw score (before LeakyReLU): its sign gives l'.
    float mx = st.m;
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      sc[k] += ar;
      if (u < cnt) mx = fmaxf(mx, leaky(sc[k], a.slope));
    }
    st.scale(expf(st.m - mx));
    st.m = mx;
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const float pk = u < cnt ? expf(leaky(sc[k], a.slope) - mx) : 0.0f;
      const float lp = sc[k] < 0.0f ? a.slope : 1.0f;
      st.s += pk;
      st.bl = fmaf(pk, lp, st.bl);
      float wk = pk;
      if constexpr (DROP) {
        bool keep = false;
        if (u < cnt) {
          const int64_t idx = static_cast<int64_t>(ebase + u) * a.H + ln.hq;
          keep = gat_keep(a.seed, static_cast<uint64_t>(idx), a.p);
          if (ln.qv && ln.cw == 0) a.mask[idx] = keep ? 1 : 0;
        }
        wk = keep ? pk / (1.0f - a.p) : 0.0f;
      }
      const float wl = wk * lp;
      float xv[W];
      Chunk<T, W>::unpack(xb[k], xv);
#pragma unroll
      for (int w = 0; w < W; ++w) {
        st.acc[w] = fmaf(wk, xv[w], st.acc[w]);
        st.accl[w] = fmaf(wl, xv[w], st.accl[w]);
      }
    }
  }
};

// All edge slots of a lane group: `need` (wave-uniform) slots per group.
template <typename T, int L, bool DROP>
__device__ __forceinline__ void fwd_edges(const GatFwdArgs<T>& a, const FlLane<L>& ln, int jj, int base, int first,
                                          int step, int cnt, int need, int ebase, float ar,
                                          FwdState<FlGeom<T>::W>& st) {
  FwdBatches<T, L, DROP> fb{a, ln, jj, base, first, step, cnt, ebase, ar, st};
  for_batches<kFwdU>(need, fb);
}

template <int L, int W>
__device__ __forceinline__ void fwd_merge_groups(FwdState<W>& st) {
#pragma unroll
  for (int o = L; o < kWave; o <<= 1) {
    float a2[W], l2[W];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      a2[w] = shfl_xor(st.acc[w], o);
      l2[w] = shfl_xor(st.accl[w], o);
    }
    const float m2 = shfl_xor(st.m, o), s2 = shfl_xor(st.s, o), b2 = shfl_xor(st.bl, o);
    st.merge(m2, s2, b2, a2, l2);
  }
}

// Head mean + bias + SiLU of a row; every lane of the wavefront calls this
// (the head sum is a butterfly inside the group), `write` selects the group
// that stores. Lane q of head 0 writes channels [cw*W, cw*W + W) of pre/out;
// lane cw = 0 of each head writes edge_max / edge_sum. With a.agg, lane q
// also writes its normalised chunks of the two aggregates and lane cw = 0 the
// head's sum_e s l'.
template <typename T, int L>
__device__ __forceinline__ void fwd_emit(const GatFwdArgs<T>& a, const FlLane<L>& ln, int cq, int row, bool write,
                                         const FwdState<FlGeom<T>::W>& st) {
  constexpr int W = FlGeom<T>::W;
  const float inv = st.s > 0.0f ? 1.0f / st.s : 0.0f;
  float y[W];
#pragma unroll
  for (int w = 0; w < W; ++w) y[w] = ln.qv ? st.acc[w] * inv : 0.0f;
  if (a.agg && write && ln.qv) {
    const int F = a.H * a.C;
    const int64_t nF = static_cast<int64_t>(a.n) * F;
    float yl[W];
#pragma unroll
    for (int w = 0; w < W; ++w) yl[w] = st.accl[w] * inv;
    store_f32<W>(a.agg + static_cast<int64_t>(row) * F + ln.q * W, y);
    store_f32<W>(a.agg + nF + static_cast<int64_t>(row) * F + ln.q * W, yl);
    if (ln.cw == 0) a.agg[2 * nF + static_cast<int64_t>(row) * a.H + ln.hq] = st.bl * inv;
  }
  for (int o = cq; o < L; o <<= 1)
#pragma unroll
    for (int w = 0; w < W; ++w) y[w] += shfl_xor(y[w], o);
  if (!write || !ln.qv) return;
  if (ln.hq == 0) {
    const int64_t base = static_cast<int64_t>(row) * a.C + ln.cw * W;
    float pr[W], o[W];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      pr[w] = y[w] / static_cast<float>(a.H) + a.bias[ln.cw * W + w];
      o[w] = silu(pr[w]);
    }
    store_f32<W>(a.pre + base, pr);
    Chunk<T, W>::store(a.out + base, o);
  }
  if (ln.cw == 0) {
    a.emax[static_cast<int64_t>(row) * a.H + ln.hq] = st.m;
    a.esum[static_cast<int64_t>(row) * a.H + ln.hq] = st.s;
  }
}

template <typename T, int L, bool DROP>
__global__ __launch_bounds__(kBlock) void gat_fwd_fl_kernel(GatFwdArgs<T> a, Sched s, int n_mid, int mid_blocks,
                                                            int lgcq) {
  constexpr int W = FlGeom<T>::W;
  constexpr int G = kWave / L;
  const int cq = 1 << lgcq;
  const int nq = a.H * cq;
  const int F = a.H * a.C;
  const FlLane<L> ln(lgcq, nq);
  const int wave = wave_id();
  FwdState<W> st;
  st.clear();
  int b = blockIdx.x;

  if (b >= s.n_seg) {
    b -= s.n_seg;
    if (b >= mid_blocks) {
      // Tiny rows (degree <= L): one per lane group.
      const int li = n_mid + ((b - mid_blocks) * kWavesPerBlock + wave) * G + ln.g;
      const bool has = li < s.n_light;
      const int4 r = has ? s.light[li] : make_int4(0, 0, 0, 0);
      const int deg = r.z - r.y;
      const int jj = ln.gl < deg ? a.col[r.y + ln.gl] : 0;
      const float ar = a.attn_row[static_cast<int64_t>(r.x) * a.H + ln.hq];
      const int need = wave_group_max<L>(deg);
      fwd_edges<T, L, DROP>(a, ln, jj, ln.g * L, 0, 1, deg, need, r.y, ar, st);
      fwd_emit<T, L>(a, ln, cq, r.x, has, st);
      return;
    }
    // Medium rows (L < degree <= 64): one per wavefront, group g takes edges
    // g, g + G, ...
    const int li = b * kWavesPerBlock + wave;
    if (li >= n_mid) return;  // wave-uniform; no block barrier follows
    const int4 r = s.light[li];
    const int deg = r.z - r.y;
    const int jj = ln.lane < deg ? a.col[r.y + ln.lane] : 0;
    const float ar = a.attn_row[static_cast<int64_t>(r.x) * a.H + ln.hq];
    fwd_edges<T, L, DROP>(a, ln, jj, 0, ln.g, G, deg, (deg + G - 1) / G, r.y, ar, st);
    fwd_merge_groups<L, W>(st);
    fwd_emit<T, L>(a, ln, cq, r.x, ln.g == 0, st);
    return;
  }

  // Heavy-row segment: wave w takes edges [64w, 64w + 64) of every 256-edge
  // round of the segment.
  __shared__ float hm[kWavesPerBlock][kWave], hs[kWavesPerBlock][kWave], hb[kWavesPerBlock][kWave];
  __shared__ float hacc[kWavesPerBlock][kWave * W], haccl[kWavesPerBlock][kWave * W];
  __shared__ int flag;
  const int4 sg = s.seg[b];
  const int row = sg.x;
  const int2 hr = s.hrow[sg.w];
  const float ar = a.attn_row[static_cast<int64_t>(row) * a.H + ln.hq];
  for (int tb = sg.y + wave * kWave; tb < sg.z; tb += kSegRound) {
    const int cnt = min(kWave, sg.z - tb);
    const int jj = ln.lane < cnt ? a.col[tb + ln.lane] : 0;
    fwd_edges<T, L, DROP>(a, ln, jj, 0, ln.g, G, cnt, (cnt + G - 1) / G, tb, ar, st);
  }
  fwd_merge_groups<L, W>(st);
  if (ln.g == 0) {
    hm[wave][ln.gl] = st.m;
    hs[wave][ln.gl] = st.s;
    hb[wave][ln.gl] = st.bl;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      hacc[wave][ln.gl * W + w] = st.acc[w];
      haccl[wave][ln.gl * W + w] = st.accl[w];
    }
  }
  __syncthreads();
  // Every wave forms the merged state of its lane slot gl (identical copies).
  st.m = hm[0][ln.gl];
  st.s = hs[0][ln.gl];
  st.bl = hb[0][ln.gl];
#pragma unroll
  for (int w = 0; w < W; ++w) {
    st.acc[w] = hacc[0][ln.gl * W + w];
    st.accl[w] = haccl[0][ln.gl * W + w];
  }
#pragma unroll
  for (int v = 1; v < kWavesPerBlock; ++v) {
    float a2[W], l2[W];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      a2[w] = hacc[v][ln.gl * W + w];
      l2[w] = haccl[v][ln.gl * W + w];
    }
    st.merge(hm[v][ln.gl], hs[v][ln.gl], hb[v][ln.gl], a2, l2);
  }
  if (hr.y == 1) {
    if (wave == 0) fwd_emit<T, L>(a, ln, cq, row, ln.g == 0, st);
    return;
  }
  // Segment partial: acc [F], accl [F], then m, s, bl per head.
  const int stride = 2 * F + 3 * a.H;
  float* mine = a.partial + static_cast<int64_t>(b) * stride;
  if (wave == 0 && ln.g == 0 && ln.qv) {
    store_f32<W>(mine + ln.q * W, st.acc);
    store_f32<W>(mine + F + ln.q * W, st.accl);
    if (ln.cw == 0) {
      mine[2 * F + ln.hq] = st.m;
      mine[2 * F + a.H + ln.hq] = st.s;
      mine[2 * F + 2 * a.H + ln.hq] = st.bl;
    }
  }
  if (!arrive_last(a.counters + sg.w, hr.y, &flag)) return;
  if (wave != 0) return;
  // Last segment to finish: merge every segment's partial in segment order.
  st.clear();
  for (int z = 0; z < hr.y; ++z) {
    const float* pz = a.partial + static_cast<int64_t>(hr.x + z) * stride;
    float a2[W], l2[W];
    load_f32<W>(pz + ln.q * W, a2);
    load_f32<W>(pz + F + ln.q * W, l2);
    st.merge(pz[2 * F + ln.hq], pz[2 * F + a.H + ln.hq], pz[2 * F + 2 * a.H + ln.hq], a2, l2);
  }
  fwd_emit<T, L>(a, ln, cq, row, ln.g == 0, st);
}

template <typename T, int L>
struct FwdFlLauncher {
  static int run(hipStream_t st, const GatFwdArgs<T>& a, const Sched& s, const int32_t* hdr, int lgcq) {
    constexpr int G = kWave / L;
    const int n_mid = G > 1 ? sched_count_gt(hdr, L) : s.n_light;
    const int mid_blocks = (n_mid + kWavesPerBlock - 1) / kWavesPerBlock;
    const int n_tiny = s.n_light - n_mid;
    const int blocks = s.n_seg + mid_blocks + (n_tiny + kWavesPerBlock * G - 1) / (kWavesPerBlock * G);
    if (blocks > 0) {
      if (a.p > 0.0f)
        hipLaunchKernelGGL((gat_fwd_fl_kernel<T, L, true>), dim3(blocks), dim3(kBlock), 0, st, a, s, n_mid,
                           mid_blocks, lgcq);
      else
        hipLaunchKernelGGL((gat_fwd_fl_kernel<T, L, false>), dim3(blocks), dim3(kBlock), 0, st, a, s, n_mid,
                           mid_blocks, lgcq);
    }
    return check_launch("cign_gat_fwd (feature layout)");
  }
};

// ===========================================================================
// Backward, rows (CSR)
// ===========================================================================
template <int W>
struct RowAcc {
  float vs[W], vsl[W];
  float B;
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int w = 0; w < W; ++w) vs[w] = vsl[w] = 0.0f;
    B = 0.0f;
  }
};

// Per-row constants of a lane's head.
struct RowHead {
  float ar, em, ies;  // attn_row, edge_max, 1 / edge_sum (0 for an empty row)
};

template <typename T>
__device__ __forceinline__ RowHead row_head(const GatBwdArgs<T>& a, int row, int hq) {
  const int64_t rh = static_cast<int64_t>(row) * a.H + hq;
  RowHead h;
  h.ar = a.attn_row[rh];
  h.em = a.emax[rh];
  const float es = a.esum[rh];
  h.ies = es > 0.0f ? 1.0f / es : 0.0f;
  return h;
}

template <typename T, int L, bool DROP>
struct RowBatches {
  static constexpr int W = FlGeom<T>::W;
  const GatBwdArgs<T>& a;
  const FlLane<L>& ln;
  int jj, base, first, step, cnt, ebase;
  const RowHead& rh;
  RowAcc<W>& st;

  template <int U>
  __device__ __forceinline__ void run(int k0) {
    const int F = a.H * a.C;
    typename Chunk<T, W>::Raw xb[U];
    float ab[U];
    float kw[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const int j = shfl(jj, (base + (u < cnt ? u : 0)) & (kWave - 1));
      ab[k] = a.attn_col[static_cast<int64_t>(j) * a.H + ln.hq];
      xb[k] = Chunk<T, W>::load_raw(a.x + static_cast<int64_t>(j) * F + ln.q * W);
      if constexpr (DROP) kw[k] = (u < cnt && a.mask[static_cast<int64_t>(ebase + u) * a.H + ln.hq]) ? 1.0f : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const float raw = rh.ar + ab[k];
      const float lp = raw < 0.0f ? a.slope : 1.0f;
      const float sm = u < cnt ? expf(leaky(raw, a.slope) - rh.em) * rh.ies : 0.0f;
      float sk = sm;
      if constexpr (DROP) sk = kw[k] != 0.0f ? sm / (1.0f - a.p) : 0.0f;
      const float skl = sk * lp;
      st.B = fmaf(sm, lp, st.B);
      float xv[W];
      Chunk<T, W>::unpack(xb[k], xv);
#pragma unroll
      for (int w = 0; w < W; ++w) {
        st.vs[w] = fmaf(sk, xv[w], st.vs[w]);
        st.vsl[w] = fmaf(skl, xv[w], st.vsl[w]);
      }
    }
  }
};

template <typename T, int L, bool DROP>
__device__ __forceinline__ void rows_edges(const GatBwdArgs<T>& a, const FlLane<L>& ln, int jj, int base, int first,
                                           int step, int cnt, int need, int ebase, const RowHead& rh,
                                           RowAcc<FlGeom<T>::W>& st) {
  RowBatches<T, L, DROP> rb{a, ln, jj, base, first, step, cnt, ebase, rh, st};
  for_batches<kRowsU>(need, rb);
}

// g_pre chunk cw of a row: g_y * SiLU'(pre).
template <typename T>
__device__ __forceinline__ void grad_pre_chunk(const GatBwdArgs<T>& a, int row, int cw,
                                               float (&gp)[FlGeom<T>::W]) {
  constexpr int W = FlGeom<T>::W;
  const int64_t base = static_cast<int64_t>(row) * a.C + cw * W;
  float gy[W], pr[W];
  Chunk<T, W>::load(a.grad_y + base, gy);
  load_f32<W>(a.pre + base, pr);
#pragma unroll
  for (int w = 0; w < W; ++w) gp[w] = gy[w] * silu_grad(pr[w]);
}

// (wsum, A) of the lane's head from the accumulated chunks: dot with g_pre,
// summed over the head's C/W lanes, divided by H.
template <int W>
__device__ __forceinline__ void rows_dots(const RowAcc<W>& st, const float (&gp)[W], int cq, float inv_h, float& wsum,
                                          float& A) {
  float d1 = 0.0f, d2 = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    d1 = fmaf(gp[w], st.vs[w], d1);
    d2 = fmaf(gp[w], st.vsl[w], d2);
  }
  wsum = head_sum(d1, cq) * inv_h;
  A = head_sum(d2, cq) * inv_h;
}

template <typename T>
__device__ __forceinline__ void rows_store(const GatBwdArgs<T>& a, int row, int hq, const RowHead& rh, float wsum,
                                           float A, float B) {
  const int64_t idx = static_cast<int64_t>(row) * a.H + hq;
  a.grad_attn_row[idx] = A - wsum * B;
  a.rowstat[idx] = make_float4(rh.ar, rh.em, rh.ies, wsum);
}

template <typename T, int L, bool DROP>
__global__ __launch_bounds__(kBlock) void gat_bwd_rows_fl_kernel(GatBwdArgs<T> a, Sched s, int n_mid, int mid_blocks,
                                                                 int lgcq) {
  constexpr int W = FlGeom<T>::W;
  constexpr int G = kWave / L;
  const int cq = 1 << lgcq;
  const int nq = a.H * cq;
  const FlLane<L> ln(lgcq, nq);
  const int wave = wave_id();
  __shared__ float red[kWavesPerBlock][3][kFlHeads];
  __shared__ int flag;
  RowAcc<W> st;
  st.clear();
  float gp[W];
  int b = blockIdx.x;

  if (b >= s.n_seg) {
    b -= s.n_seg;
    const bool tiny = b >= mid_blocks;
    int4 r = make_int4(0, 0, 0, 0);
    bool has;
    if (tiny) {
      const int li = n_mid + ((b - mid_blocks) * kWavesPerBlock + wave) * G + ln.g;
      has = li < s.n_light;
      if (has) r = s.light[li];
    } else {
      const int li = b * kWavesPerBlock + wave;
      has = li < n_mid;
      if (has) r = s.light[li];
    }
    const int row = r.x;
    const int deg = r.z - r.y;
    const int slot = tiny ? ln.gl : ln.lane;
    const int jj = slot < deg ? a.col[r.y + slot] : 0;
    const RowHead rh = row_head(a, row, ln.hq);
    grad_pre_chunk(a, row, ln.cw, gp);
    if (tiny) {
      rows_edges<T, L, DROP>(a, ln, jj, ln.g * L, 0, 1, deg, wave_group_max<L>(deg), r.y, rh, st);
    } else {
      rows_edges<T, L, DROP>(a, ln, jj, 0, ln.g, G, deg, (deg + G - 1) / G, r.y, rh, st);
      group_sum<L, W>(st.vs);
      group_sum<L, W>(st.vsl);
      st.B = group_sum1<L>(st.B);
    }
    float wsum, A;
    rows_dots<W>(st, gp, cq, a.inv_h, wsum, A);
    const bool write = has && (tiny || ln.g == 0) && ln.qv;
    if (write && ln.cw == 0) rows_store(a, row, ln.hq, rh, wsum, A, st.B);
    if (write && ln.hq == 0) store_f32<W>(a.grad_pre + static_cast<int64_t>(row) * a.C + ln.cw * W, gp);
    return;
  }

  // Heavy-row segment: the four waves' (wsum, A, B) per head, then across the
  // row's segments (last to finish, in segment order).
  const int4 sg = s.seg[b];
  const int row = sg.x;
  const int2 hr = s.hrow[sg.w];
  const RowHead rh = row_head(a, row, ln.hq);
  grad_pre_chunk(a, row, ln.cw, gp);
  for (int tb = sg.y + wave * kWave; tb < sg.z; tb += kSegRound) {
    const int cnt = min(kWave, sg.z - tb);
    const int jj = ln.lane < cnt ? a.col[tb + ln.lane] : 0;
    rows_edges<T, L, DROP>(a, ln, jj, 0, ln.g, G, cnt, (cnt + G - 1) / G, tb, rh, st);
  }
  group_sum<L, W>(st.vs);
  group_sum<L, W>(st.vsl);
  st.B = group_sum1<L>(st.B);
  float wsum, A;
  rows_dots<W>(st, gp, cq, a.inv_h, wsum, A);
  if (ln.g == 0 && ln.qv && ln.cw == 0) {
    red[wave][0][ln.hq] = wsum;
    red[wave][1][ln.hq] = A;
    red[wave][2][ln.hq] = st.B;
  }
  // The row's g_pre is published once, by its first segment.
  if (b == hr.x && wave == 0 && ln.g == 0 && ln.qv && ln.hq == 0)
    store_f32<W>(a.grad_pre + static_cast<int64_t>(row) * a.C + ln.cw * W, gp);
  __syncthreads();
  if (threadIdx.x < 3 * kFlHeads) {
    const int k = threadIdx.x / kFlHeads, h = threadIdx.x % kFlHeads;
    red[0][k][h] = red[0][k][h] + red[1][k][h] + red[2][k][h] + red[3][k][h];
  }
  __syncthreads();
  if (hr.y == 1) {
    if (threadIdx.x < a.H) {
      const int h = threadIdx.x;
      rows_store(a, row, h, row_head(a, row, h), red[0][0][h], red[0][1][h], red[0][2][h]);
    }
    return;
  }
  float* mine = a.part_row + static_cast<int64_t>(b) * 3 * a.H;
  if (threadIdx.x < 3 * a.H) mine[threadIdx.x] = red[0][threadIdx.x / a.H][threadIdx.x % a.H];
  if (!arrive_last(a.row_counters + sg.w, hr.y, &flag)) return;
  if (threadIdx.x < a.H) {
    const int h = threadIdx.x;
    float w = 0.0f, AA = 0.0f, BB = 0.0f;
    for (int z = 0; z < hr.y; ++z) {
      const float* pz = a.part_row + static_cast<int64_t>(hr.x + z) * 3 * a.H;
      w += pz[h];
      AA += pz[a.H + h];
      BB += pz[2 * a.H + h];
    }
    rows_store(a, row, h, row_head(a, row, h), w, AA, BB);
  }
}

// Rows pass from the forward's per-row aggregates (a.agg): the same
// (wsum, A, B) as gat_bwd_rows_fl_kernel without gathering any source row, a
// stream over the rows. A group of L lanes per row, G rows per wavefront.
template <typename T, int L>
__global__ __launch_bounds__(kBlock) void gat_bwd_rows_agg_kernel(GatBwdArgs<T> a, int lgcq) {
  constexpr int W = FlGeom<T>::W;
  constexpr int G = kWave / L;
  const int cq = 1 << lgcq;
  const FlLane<L> ln(lgcq, a.H * cq);
  const int row = (blockIdx.x * kWavesPerBlock + wave_id()) * G + ln.g;
  if (row >= a.n) return;  // no barrier follows
  const int F = a.H * a.C;
  const int64_t nF = static_cast<int64_t>(a.n) * F;
  RowAcc<W> st;
  load_f32<W>(a.agg + static_cast<int64_t>(row) * F + ln.q * W, st.vs);
  load_f32<W>(a.agg + nF + static_cast<int64_t>(row) * F + ln.q * W, st.vsl);
  st.B = a.agg[2 * nF + static_cast<int64_t>(row) * a.H + ln.hq];
  float gp[W];
  grad_pre_chunk(a, row, ln.cw, gp);
  float wsum, A;
  rows_dots<W>(st, gp, cq, a.inv_h, wsum, A);
  if (!ln.qv) return;
  if (ln.cw == 0) rows_store(a, row, ln.hq, row_head(a, row, ln.hq), wsum, A, st.B);
  if (ln.hq == 0) store_f32<W>(a.grad_pre + static_cast<int64_t>(row) * a.C + ln.cw * W, gp);
}

// ===========================================================================
// Backward, columns (CSC)
// ===========================================================================
template <int W>
struct ColAcc {
  float ug[W], ua[W];
  float t;
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int w = 0; w < W; ++w) ug[w] = ua[w] = 0.0f;
    t = 0.0f;
  }
};

// Batches of CSC entries of column j: slot u's destination row is held by
// lane (base + u) in ii, its CSR edge id (used only with dropout) in ee.
template <typename T, int L, bool DROP>
struct ColBatches {
  static constexpr int W = FlGeom<T>::W;
  const GatBwdArgs<T>& a;
  const FlLane<L>& ln;
  int ii, ee, base, first, step, cnt;
  float ac;
  ColAcc<W>& st;

  template <int U>
  __device__ __forceinline__ void run(int k0) {
    float gb[U][W];
    float4 rs[U];
    float kw[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const int src = (base + (u < cnt ? u : 0)) & (kWave - 1);
      const int i = shfl(ii, src);
      rs[k] = a.rowstat[static_cast<int64_t>(i) * a.H + ln.hq];
      load_f32<W>(a.grad_pre + static_cast<int64_t>(i) * a.C + ln.cw * W, gb[k]);
      if constexpr (DROP) {
        const int e = shfl(ee, src);
        kw[k] = (u < cnt && a.mask[static_cast<int64_t>(e) * a.H + ln.hq]) ? 1.0f : 0.0f;
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const float raw = rs[k].x + ac;
      const float lp = raw < 0.0f ? a.slope : 1.0f;
      const float sm = u < cnt ? expf(leaky(raw, a.slope) - rs[k].y) * rs[k].z : 0.0f;
      float w = sm;
      if constexpr (DROP) w = kw[k] != 0.0f ? sm / (1.0f - a.p) : 0.0f;
      const float wl = w * lp;
      st.t = fmaf(sm * lp, rs[k].w, st.t);
#pragma unroll
      for (int q = 0; q < W; ++q) {
        st.ug[q] = fmaf(w, gb[k][q], st.ug[q]);
        st.ua[q] = fmaf(wl, gb[k][q], st.ua[q]);
      }
    }
  }
};

template <typename T, int L, bool DROP>
__device__ __forceinline__ void cols_edges(const GatBwdArgs<T>& a, const FlLane<L>& ln, int ii, int ee, int base,
                                           int first, int step, int cnt, int need, float ac,
                                           ColAcc<FlGeom<T>::W>& st) {
  ColBatches<T, L, DROP> cb{a, ln, ii, ee, base, first, step, cnt, ac, st};
  for_batches<kColsU>(need, cb);
}

// The lane's part of grad_attn_col[j, hq]: <ua, x[j] chunk> summed over the
// head's lanes / H, minus t.
template <typename T>
__device__ __forceinline__ float cols_gac(const GatBwdArgs<T>& a, const ColAcc<FlGeom<T>::W>& st,
                                          const float (&xj)[FlGeom<T>::W], int cq) {
  constexpr int W = FlGeom<T>::W;
  float d = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) d = fmaf(st.ua[w], xj[w], d);
  return head_sum(d, cq) * a.inv_h - st.t;
}

template <typename T, int L, bool DROP>
__global__ __launch_bounds__(kBlock) void gat_bwd_cols_fl_kernel(GatBwdArgs<T> a, Sched s, int n_mid, int mid_blocks,
                                                                 int lgcq) {
  constexpr int W = FlGeom<T>::W;
  constexpr int G = kWave / L;
  const int cq = 1 << lgcq;
  const int nq = a.H * cq;
  const int F = a.H * a.C;
  const FlLane<L> ln(lgcq, nq);
  const int wave = wave_id();
  __shared__ float red[kWavesPerBlock][kWave * W];
  __shared__ float gred[kWavesPerBlock][kFlHeads];
  __shared__ int flag;
  int b = blockIdx.x;
  const int nsched = s.n_seg + mid_blocks + (s.n_light - n_mid + kWavesPerBlock * G - 1) / (kWavesPerBlock * G);
  if (b >= nsched) {
    bias_from_grad_pre(a, b - nsched, a.col_counters + s.n_hrow, &flag);
    return;
  }
  ColAcc<W> st;
  st.clear();

  if (b >= s.n_seg) {
    b -= s.n_seg;
    const bool tiny = b >= mid_blocks;
    int4 r = make_int4(0, 0, 0, 0);
    bool has;
    if (tiny) {
      const int li = n_mid + ((b - mid_blocks) * kWavesPerBlock + wave) * G + ln.g;
      has = li < s.n_light;
      if (has) r = s.light[li];
    } else {
      const int li = b * kWavesPerBlock + wave;
      has = li < n_mid;
      if (!has) return;  // wave-uniform; no block barrier follows
      r = s.light[li];
    }
    const int j = r.x;
    const int deg = r.z - r.y;
    const int slot = tiny ? ln.gl : ln.lane;
    const bool own = slot < deg;
    const int ii = own ? a.rowind[r.y + slot] : 0;
    const int ee = (DROP && own) ? a.perm[r.y + slot] : 0;
    const float ac = a.attn_col[static_cast<int64_t>(j) * a.H + ln.hq];
    float xj[W];
    Chunk<T, W>::load(a.x + static_cast<int64_t>(j) * F + ln.q * W, xj);
    if (tiny) {
      cols_edges<T, L, DROP>(a, ln, ii, ee, ln.g * L, 0, 1, deg, wave_group_max<L>(deg), ac, st);
    } else {
      cols_edges<T, L, DROP>(a, ln, ii, ee, 0, ln.g, G, deg, (deg + G - 1) / G, ac, st);
      group_sum<L, W>(st.ug);
      group_sum<L, W>(st.ua);
      st.t = group_sum1<L>(st.t);
    }
    const float gac = cols_gac(a, st, xj, cq);
    if (!(has && (tiny || ln.g == 0) && ln.qv)) return;
    float o[W];
#pragma unroll
    for (int w = 0; w < W; ++w) o[w] = st.ug[w] * a.inv_h;
    Chunk<T, W>::store(a.grad_feat + static_cast<int64_t>(j) * F + ln.q * W, o);
    if (ln.cw == 0) a.grad_attn_col[static_cast<int64_t>(j) * a.H + ln.hq] = gac;
    return;
  }

  // Heavy column segment: wave w takes entries [64w, 64w + 64) of every
  // 256-entry round of the segment.
  const int4 sg = s.seg[b];
  const int j = sg.x;
  const int2 hr = s.hrow[sg.w];
  const float ac = a.attn_col[static_cast<int64_t>(j) * a.H + ln.hq];
  float xj[W];
  Chunk<T, W>::load(a.x + static_cast<int64_t>(j) * F + ln.q * W, xj);
  for (int tb = sg.y + wave * kWave; tb < sg.z; tb += kSegRound) {
    const int cnt = min(kWave, sg.z - tb);
    const bool own = ln.lane < cnt;
    const int ii = own ? a.rowind[tb + ln.lane] : 0;
    const int ee = (DROP && own) ? a.perm[tb + ln.lane] : 0;
    cols_edges<T, L, DROP>(a, ln, ii, ee, 0, ln.g, G, cnt, (cnt + G - 1) / G, ac, st);
  }
  group_sum<L, W>(st.ug);
  group_sum<L, W>(st.ua);
  st.t = group_sum1<L>(st.t);
  const float gac = cols_gac(a, st, xj, cq);
  if (ln.g == 0 && ln.qv) {
#pragma unroll
    for (int w = 0; w < W; ++w) red[wave][ln.q * W + w] = st.ug[w];
    if (ln.cw == 0) gred[wave][ln.hq] = gac;
  }
  __syncthreads();
  const bool single = hr.y == 1;
  const int stride = F + a.H;
  float* mine = a.part_col + static_cast<int64_t>(b) * stride;
  for (int k = threadIdx.x; k < F; k += kBlock) {
    const float v = red[0][k] + red[1][k] + red[2][k] + red[3][k];
    if (single) a.grad_feat[static_cast<int64_t>(j) * F + k] = from_f32<T>(v * a.inv_h);
    else mine[k] = v;
  }
  if (threadIdx.x < a.H) {
    const int h = threadIdx.x;
    const float v = gred[0][h] + gred[1][h] + gred[2][h] + gred[3][h];
    if (single) a.grad_attn_col[static_cast<int64_t>(j) * a.H + h] = v;
    else mine[F + h] = v;
  }
  if (single) return;
  if (!arrive_last(a.col_counters + sg.w, hr.y, &flag)) return;
  for (int k = threadIdx.x; k < stride; k += kBlock) {
    float v = 0.0f;
    for (int z = 0; z < hr.y; ++z) v += a.part_col[static_cast<int64_t>(hr.x + z) * stride + k];
    if (k < F) a.grad_feat[static_cast<int64_t>(j) * F + k] = from_f32<T>(v * a.inv_h);
    else a.grad_attn_col[static_cast<int64_t>(j) * a.H + (k - F)] = v;
  }
}

template <typename T, int L>
struct BwdFlLauncher {
  static int row_blocks(const Sched& rs, const int32_t* rhdr) {
    constexpr int G = kWave / L;
    const int r_mid = G > 1 ? sched_count_gt(rhdr, L) : rs.n_light;
    return rs.n_seg + (r_mid + kWavesPerBlock - 1) / kWavesPerBlock +
           (rs.n_light - r_mid + kWavesPerBlock * G - 1) / (kWavesPerBlock * G);
  }

  static int run(hipStream_t st, const GatBwdArgs<T>& a, const Sched& rs, const int32_t* rhdr, const Sched& cs,
                 const int32_t* chdr, int lgcq) {
    constexpr int G = kWave / L;
    const int r_mid = G > 1 ? sched_count_gt(rhdr, L) : rs.n_light;
    const int r_mid_blocks = (r_mid + kWavesPerBlock - 1) / kWavesPerBlock;
    const int rb = row_blocks(rs, rhdr);
    if (a.agg) {
      const int ab = (a.n + kWavesPerBlock * G - 1) / (kWavesPerBlock * G);
      if (ab > 0) {
        hipLaunchKernelGGL((gat_bwd_rows_agg_kernel<T, L>), dim3(ab), dim3(kBlock), 0, st, a, lgcq);
        const int rc = check_launch("cign_gat_bwd (rows from aggregates, feature layout)");
        if (rc) return rc;
      }
    } else if (rb > 0) {
      if (a.p > 0.0f)
        hipLaunchKernelGGL((gat_bwd_rows_fl_kernel<T, L, true>), dim3(rb), dim3(kBlock), 0, st, a, rs, r_mid,
                           r_mid_blocks, lgcq);
      else
        hipLaunchKernelGGL((gat_bwd_rows_fl_kernel<T, L, false>), dim3(rb), dim3(kBlock), 0, st, a, rs, r_mid,
                           r_mid_blocks, lgcq);
      const int rc = check_launch("cign_gat_bwd (rows, feature layout)");
      if (rc) return rc;
    }
    const int c_mid = G > 1 ? sched_count_gt(chdr, L) : cs.n_light;
    const int c_mid_blocks = (c_mid + kWavesPerBlock - 1) / kWavesPerBlock;
    const int cb = cs.n_seg + c_mid_blocks + (cs.n_light - c_mid + kWavesPerBlock * G - 1) / (kWavesPerBlock * G) +
                   a.n_l2;
    if (cb > 0) {
      if (a.p > 0.0f)
        hipLaunchKernelGGL((gat_bwd_cols_fl_kernel<T, L, true>), dim3(cb), dim3(kBlock), 0, st, a, cs, c_mid,
                           c_mid_blocks, lgcq);
      else
        hipLaunchKernelGGL((gat_bwd_cols_fl_kernel<T, L, false>), dim3(cb), dim3(kBlock), 0, st, a, cs, c_mid,
                           c_mid_blocks, lgcq);
    }
    return check_launch("cign_gat_bwd (cols, feature layout)");
  }
};

#define CIGN_GAT_FL_INSTANTIATE(T)                       \
  template struct ::cign::gatk::BwdFlLauncher<T, 1>;     \
  template struct ::cign::gatk::BwdFlLauncher<T, 2>;     \
  template struct ::cign::gatk::BwdFlLauncher<T, 4>;     \
  template struct ::cign::gatk::BwdFlLauncher<T, 8>;     \
  template struct ::cign::gatk::BwdFlLauncher<T, 16>;    \
  template struct ::cign::gatk::BwdFlLauncher<T, 32>;    \
  template struct ::cign::gatk::BwdFlLauncher<T, 64>;    \
  template struct ::cign::gatk::FwdFlLauncher<T, 1>;     \
  template struct ::cign::gatk::FwdFlLauncher<T, 2>;     \
  template struct ::cign::gatk::FwdFlLauncher<T, 4>;     \
  template struct ::cign::gatk::FwdFlLauncher<T, 8>;     \
  template struct ::cign::gatk::FwdFlLauncher<T, 16>;    \
  template struct ::cign::gatk::FwdFlLauncher<T, 32>;    \
  template struct ::cign::gatk::FwdFlLauncher<T, 64>;

#define CIGN_GAT_FL_DECLARE(T)                                  \
  extern template struct ::cign::gatk::BwdFlLauncher<T, 1>;     \
  extern template struct ::cign::gatk::BwdFlLauncher<T, 2>;     \
  extern template struct ::cign::gatk::BwdFlLauncher<T, 4>;     \
  extern template struct ::cign::gatk::BwdFlLauncher<T, 8>;     \
  extern template struct ::cign::gatk::BwdFlLauncher<T, 16>;    \
  extern template struct ::cign::gatk::BwdFlLauncher<T, 32>;    \
  extern template struct ::cign::gatk::BwdFlLauncher<T, 64>;    \
  extern template struct ::cign::gatk::FwdFlLauncher<T, 1>;     \
  extern template struct ::cign::gatk::FwdFlLauncher<T, 2>;     \
  extern template struct ::cign::gatk::FwdFlLauncher<T, 4>;     \
  extern template struct ::cign::gatk::FwdFlLauncher<T, 8>;     \
  extern template struct ::cign::gatk::FwdFlLauncher<T, 16>;    \
  extern template struct ::cign::gatk::FwdFlLauncher<T, 32>;    \
  extern template struct ::cign::gatk::FwdFlLauncher<T, 64>;

}  // namespace gatk
}  // namespace cign
