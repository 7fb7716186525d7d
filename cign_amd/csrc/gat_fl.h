// Collapsed GAT, feature layout: the gfx950 fast path for H <= 8 heads and C
// a multiple of the 16-byte chunk width W (4 fp32 or 8 bf16 values) with
// cq = C/W a power of two, and either H*cq <= 64 chunks (narrow rows) or cq <=
// 64 with V = H*cq/64 in {2, 3, 4, 6, 8} chunks per lane (wide rows, e.g. the
// production H=6 x C=256). Semantics are those stated at the top of
// gat_kernels.h (reference collapsed_gat_cuda.cu:34-430).
//
// Geometry (shared with the SpMM, schedule.h built with light_max = 64 and a
// segment length that is a multiple of 256). A group of L lanes owns one row;
// lane gl owns the V chunks q = v*L + gl (v < V) of a feature row, chunk q
// being head hq = q / cq, channel chunk cw = q % cq. Narrow rows have V = 1
// and L = pow2ceil(H*cq); wide rows have L = 64 and, as cq divides 64, every
// chunk of a lane has the same channel chunk cw = gl % cq and its own head.
// Rows with degree <= L go one per group (64/L rows per wavefront), rows
// with degree <= 64 one per wavefront (its groups split the edges), heavier
// rows are segments (one 4-wave workgroup each, rounds of 256 edges) whose
// partial results the last workgroup to finish merges in segment order.
//
// Every lane gathers, for each edge of its batch, the 16-byte chunks of the
// source feature row AND the source logits of its own heads in the same
// memory round, right after the column index: the softmax is online (running
// max m, sum s and unnormalised accumulators rescaled per batch, flash
// style), so no lane-per-edge prologue, LDS staging or per-edge cross-lane
// reduction sits between the index load and the feature gather. A row costs
// one dependent round per level of indirection (schedule record -> column
// index -> source data). The batch size U is the wavefront's largest
// per-group edge count rounded up to a power of two, capped so that a lane
// keeps at most 16 (forward, rows) or 8 (columns) edge slots x V chunks in
// flight.
//
// Backward without per-edge reductions. With g = g_pre[i] (= g_y SiLU'(pre)),
// s the softmax weight, kw = keep/(1-p) (1 without dropout), l' the
// LeakyReLU slope of the raw score and ge'_e = kw <g, x[j_e,h]>/H:
//   wsum_ih = sum_e s ge'          = <g, sum_e s kw x[j_e,h]> / H
//   A_ih    = sum_e s ge' l'       = <g, sum_e s kw l' x[j_e,h]> / H
//   grad_attn_row[i,h] = A - wsum * B,   B = sum_e s l'
// so the rows pass needs two feature sums per (row, head) and one dot product
// per row. The forward can save those sums (the per-row aggregates, a.agg);
// the rows pass then streams them (gat_bwd_rows_agg_kernel), otherwise it
// gathers the source rows again (gat_bwd_rows_fl_kernel). The columns kernel
// (CSC, column j) uses
//   grad_feat[j,h]     = sum_i s kw g_pre[i] / H
//   grad_attn_col[j,h] = <sum_i s l' kw g_pre[i], x[j,h]> / H - sum_i s l' wsum_i
// gathering per entry one 16-byte row record {attn_row, edge_max, 1/edge_sum,
// wsum} per head (written by the rows pass) and the g_pre chunk. grad_bias is
// a deterministic two-level column sum of g_pre done by the columns kernel's
// trailing workgroups, so the rows pass has no block barrier on light rows.
#pragma once

#include <cstdlib>
#include <utility>

#include "gat_kernels.h"

namespace cign {
namespace gatk {

constexpr int kFlHeads = 8;

// Largest batch (edge slots gathered per lane before any is consumed, times
// the chunks per lane) of each kernel; the cap trades loads in flight per
// wave for waves per SIMD.
// The forward has two caps: 16 edge slots for graphs below kFwdBigGraph
// edges, where a launch is a few dependent memory rounds and more loads per
// round shorten it, and 8 above, where the smaller register footprint (one
// more wavefront per SIMD) keeps more bytes in flight: at 62.4M edges (bf16,
// 4 x 32) the forward took 3.43 ms with 8 against 4.84 ms with 16, at 211K
// edges (fp32, 4 x 16) 14.7 us against 13.5 us.
#ifndef CIGN_FL_FWD_U
#define CIGN_FL_FWD_U 16
#endif
#ifndef CIGN_FL_FWD_U_BIG
#define CIGN_FL_FWD_U_BIG 8
#endif
constexpr int64_t kFwdBigGraph = 1 << 22;

// Edge count from which the large-graph variants run: kFwdBigGraph, or the
// value of CIGN_GAT_BIG_GRAPH_EDGES (read at every launch; the tests set it to
// 0 to run every shape through the large-graph variants at small sizes).
inline int64_t big_graph_edges() {
  const char* e = getenv("CIGN_GAT_BIG_GRAPH_EDGES");
  return (e && *e) ? atoll(e) : kFwdBigGraph;
}
#ifndef CIGN_FL_ROWS_U
#define CIGN_FL_ROWS_U 16
#endif
#ifndef CIGN_FL_COLS_U
#define CIGN_FL_COLS_U 8
#endif
// Wide columns gather only grad_pre chunks (W floats each) per slot; this is
// the number of gathered floats a lane holds per batch.
#ifndef CIGN_FL_COLS_PAIR_FLOATS
#define CIGN_FL_COLS_PAIR_FLOATS 16
#endif
constexpr int kFwdU = CIGN_FL_FWD_U;
constexpr int kFwdUBig = CIGN_FL_FWD_U_BIG;
// fp32 rows of one chunk per lane (V = 1: the c2 GAT's 4 x 16) take 8 slots
// on small graphs too since their hub rows split into 512-edge segments with
// write-through merges: c2 forward 12.2 -> 11.6 us. bf16 rows (11.3 -> 11.9 us)
// and wide rows (production block, bf16 96 -> 106 us, fp32 237 -> 301 us)
// keep 16.
constexpr int kFwdUNarrowF32 = 8;
constexpr int kRowsU = CIGN_FL_ROWS_U;
constexpr int kColsU = CIGN_FL_COLS_U;
// Batch cap of the shared-weight columns batches (large graphs): 4 slots
// measured 3.54 ms at 62.4M edges against 3.90 ms for 8 and 5.55 ms for 16.
constexpr int kColsUShared = 4;
constexpr int kColsPairFloats = CIGN_FL_COLS_PAIR_FLOATS;

// Batch cap for V chunks per lane: the largest power of two <= umax / V.
constexpr int batch_cap(int umax, int v) {
  return umax / v >= 16 ? 16 : umax / v >= 8 ? 8 : umax / v >= 4 ? 4 : umax / v >= 2 ? 2 : 1;
}

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
template <>
struct FlGeom<bf16h> {
  static constexpr int W = 4;
};

// Lane geometry of a group of L lanes (one row) owning V chunks per lane.
template <int L, int V>
struct FlLane {
  static_assert(V == 1 || L == kWave, "several chunks per lane need a full wavefront per row");
  int lane, g, gl, cw;
  int q[V], hq[V];
  bool qv[V];
  __device__ __forceinline__ FlLane(int lgcq, int nq) {
    lane = lane_id();
    g = lane / L;
    gl = lane & (L - 1);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int qq = v * L + gl;
      qv[v] = qq < nq;
      q[v] = qv[v] ? qq : 0;
      hq[v] = q[v] >> lgcq;
    }
    cw = V == 1 ? (q[0] & ((1 << lgcq) - 1)) : (gl & ((1 << lgcq) - 1));
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
  for_offsets<L, kWave>([&](auto OC) {
#pragma unroll
    for (int w = 0; w < W; ++w) v[w] += xor_shfl<decltype(OC)::value>(v[w]);
  });
}

template <int L>
__device__ __forceinline__ float group_sum1(float v) {
  for_offsets<L, kWave>([&](auto OC) { v += xor_shfl<decltype(OC)::value>(v); });
  return v;
}

// Sums each of N values over the cq lanes of a head (lane bits below
// log2(cq)). The N butterflies are interleaved step by step, so their
// shuffles are in flight together; one value at a time made every shuffle
// wait for the previous one (72 dependent round trips per row for the six
// heads' two sums of a 6 x 256 row).
template <int N>
__device__ __forceinline__ void head_sum_n(float (&v)[N], int cq) {
  for_offsets<1, kWave>([&](auto OC) {
    constexpr int o = decltype(OC)::value;
    if (o < cq)
#pragma unroll
      for (int i = 0; i < N; ++i) v[i] += xor_shfl<o>(v[i]);
  });
}

// Dropout keep bits of a batch's U x H (edge slot k, head h) pairs, each
// computed once. Slots are laid out S = min(L, 8) >= H bits apart, SPR = L / S
// slots per round: pair (k, h) belongs to lane (k % SPR) * S + h of its group
// in round k / SPR, and the round's ballot holds it at bit g*L + (k % SPR)*S
// + h for group g, so a lookup indexes the ballot array with a compile-time
// round. keep_of(k, h, own) is called by every lane of every round (with a
// valid (k, h) even when the lane owns no pair, own = false) and returns the
// pair's bit (false when !own), so shuffles inside it see the whole
// wavefront.
template <int U, int L>
struct PairBits {
  static constexpr int S = L < 8 ? L : 8;
  static constexpr int SPR = L / S;
  static constexpr int R = (U + SPR - 1) / SPR;
  uint64_t w[R];

  template <typename Fn>
  __device__ __forceinline__ void compute(int H, int gl, Fn&& keep_of) {
    const int h = gl % S;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = r * SPR + gl / S;
      const bool own = h < H && k < U;
      const bool keep = keep_of(k < U ? k : U - 1, h < H ? h : H - 1, own);
      w[r] = __ballot(keep);
    }
  }
  __device__ __forceinline__ bool get(int k, int h, int g) const {
    return (w[k / SPR] >> (g * L + (k % SPR) * S + h)) & 1ull;
  }
};

// ===========================================================================
// Forward
// ===========================================================================
// Online-softmax state of a lane, per owned chunk v: running max m, sum s and
// the unnormalised accumulators acc = sum p kw x, accl = sum p kw l' x, bl =
// sum p l' (p = exp(score - m)); accl and bl are the per-row aggregates the
// backward reads instead of gathering the source rows again.
template <int W, int V>
struct FwdState {
  float m[V], s[V], bl[V];
  float acc[V][W], accl[V][W];
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      m[v] = kNegBig;
      s[v] = 0.0f;
      bl[v] = 0.0f;
#pragma unroll
      for (int w = 0; w < W; ++w) acc[v][w] = accl[v][w] = 0.0f;
    }
  }
  __device__ __forceinline__ void scale(int v, float f) {
    s[v] *= f;
    bl[v] *= f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      acc[v][w] *= f;
      accl[v][w] *= f;
    }
  }
  // chunk v's state <- state (+) (m2, s2, bl2, acc2, accl2)
  __device__ __forceinline__ void merge(int v, float m2, float s2, float bl2, const float (&acc2)[W],
                                        const float (&accl2)[W]) {
    const float mx = fmaxf(m[v], m2);
    const float f1 = softmax_exp(m[v] - mx), f2 = softmax_exp(m2 - mx);
    s[v] = s[v] * f1 + s2 * f2;
    bl[v] = bl[v] * f1 + bl2 * f2;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      acc[v][w] = acc[v][w] * f1 + acc2[w] * f2;
      accl[v][w] = accl[v][w] * f1 + accl2[w] * f2;
    }
    m[v] = mx;
  }
};

// The R lanes of a quad (R = 4) or pair (R = 2) that hold chunks of one
// head split the per-(edge, head) work of a batch and exchange its results
// through DPP: broadcast of lane S, max and sum over the R lanes.
template <int R, int S>
__device__ __forceinline__ float quad_bcast(float v) {
  if constexpr (R == 1) return v;
  else if constexpr (R == 2) return dpp<(S == 0 ? 0xA0 : 0xF5)>(v);  // [S, S, 2 + S, 2 + S]
  else return dpp<0x55 * S>(v);                                        // [S, S, S, S]
}
// f(integral_constant<int, i>) for i = 0 .. N-1 (compile-time indices).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}
template <int R>
__device__ __forceinline__ float quad_max(float v) {
  if constexpr (R >= 2) v = fmaxf(v, dpp<0xB1>(v));  // xor 1
  if constexpr (R >= 4) v = fmaxf(v, dpp<0x4E>(v));  // xor 2
  return v;
}
template <int R>
__device__ __forceinline__ float quad_sum(float v) {
  if constexpr (R >= 2) v += dpp<0xB1>(v);
  if constexpr (R >= 4) v += dpp<0x4E>(v);
  return v;
}

// Batches of U edge slots of a lane group: slot u = first + (k0 + k) * step,
// valid while u < cnt; its column index is held by lane (base + u) of the
// wavefront, its CSR edge id is ebase + u. DROP: edge dropout (p > 0).
// Every lane gathers its chunks of all U source rows. The softmax work of
// each (edge, head) pair -- the source logit, LeakyReLU, exponential, slope,
// dropout bit and mask byte -- is done once per R lanes of the head: lane r of
// an R-lane set takes slots r, r + R, ...; the weights of slot k then come
// from lane k % R by a DPP broadcast. The running max is shared by the R
// lanes; the sums s and bl are per-lane partials until quad_reduce().
template <typename T, int L, int V, bool DROP, int R>
struct FwdBatches {
  static constexpr int W = FlGeom<T>::W;
  const GatFwdArgs<T>& a;
  const FlLane<L, V>& ln;
  int jj, base, first, step, cnt, ebase;
  const float (&ar)[V];
  FwdState<W, V>& st;

  template <int U>
  __device__ __forceinline__ void run(int k0) {
    constexpr int NT = (U + R - 1) / R;  // slots whose weights this lane computes
    const uint32_t rowB = static_cast<uint32_t>(a.H * a.C) * sizeof(T);
    typename Chunk<T, W>::Raw xb[U][V];
    // Slot u's index is held by lane (base + u) mod 64. Every lane holds a
    // valid column index (0 where it has no edge), so a slot past cnt reads
    // some valid row, weighted 0, and needs no clamp.
    const int ub = base + first + k0 * step;
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const uint64_t j = static_cast<uint32_t>(shfl(jj, (ub + k * step) & (kWave - 1)));
#pragma unroll
      for (int v = 0; v < V; ++v)
        xb[k][v] = *reinterpret_cast<const typename Chunk<T, W>::Raw*>(
            reinterpret_cast<const char*>(a.x + ln.q[v] * W) + j * rowB);
    }
    const int r = ln.gl & (R - 1);
    float sc[NT][V];
    bool own[NT];
    int uo[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int kk = R * t + r;
      uo[t] = first + (k0 + kk) * step;
      own[t] = kk < U && uo[t] < cnt;
      const uint64_t j = static_cast<uint32_t>(shfl(jj, (base + uo[t]) & (kWave - 1)));
#pragma unroll
      for (int v = 0; v < V; ++v) sc[t][v] = a.attn_col[j * a.H + ln.hq[v]] + ar[v];  // raw score
    }
    float wk[NT][V], wl[NT][V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float mx = st.m[v];
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (own[t]) mx = fmaxf(mx, leaky(sc[t][v], a.slope));
      mx = quad_max<R>(mx);
      if (__any(mx != st.m[v])) st.scale(v, softmax_exp(st.m[v] - mx));
      st.m[v] = mx;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float pk = own[t] ? softmax_exp(leaky(sc[t][v], a.slope) - mx) : 0.0f;
        const float lp = sc[t][v] < 0.0f ? a.slope : 1.0f;
        st.s[v] += pk;
        st.bl[v] = fmaf(pk, lp, st.bl[v]);
        float w = pk;
        if constexpr (DROP) {
          const int64_t idx = static_cast<int64_t>(ebase + uo[t]) * a.H + ln.hq[v];
          const bool keep = gat_keep(a.seed, static_cast<uint64_t>(idx + a.mask_base), a.p);
          if (own[t] && ln.qv[v]) a.mask[idx] = keep ? 1 : 0;
          w = keep ? pk * (1.0f / (1.0f - a.p)) : 0.0f;
        }
        wk[t][v] = w;
        wl[t][v] = w * lp;
      }
    }
    static_for<U>([&](auto KC) {
      constexpr int k = decltype(KC)::value;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float w = quad_bcast<R, k % R>(wk[k / R][v]);
        const float wlk = quad_bcast<R, k % R>(wl[k / R][v]);
        float xv[W];
        Chunk<T, W>::unpack(xb[k][v], xv);
#pragma unroll
        for (int q = 0; q < W; ++q) {
          st.acc[v][q] = fmaf(w, xv[q], st.acc[v][q]);
          st.accl[v][q] = fmaf(wlk, xv[q], st.accl[v][q]);
        }
      }
    });
  }
};

// All edge slots of a lane group: `need` (wave-uniform) slots per group.
template <typename T, int L, int V, bool DROP, int R, int UM>
__device__ __forceinline__ void fwd_edges(const GatFwdArgs<T>& a, const FlLane<L, V>& ln, int jj, int base, int first,
                                          int step, int cnt, int need, int ebase, const float (&ar)[V],
                                          FwdState<FlGeom<T>::W, V>& st) {
  FwdBatches<T, L, V, DROP, R> fb{a, ln, jj, base, first, step, cnt, ebase, ar, st};
  for_batches<batch_cap(UM, V)>(need, fb);
}

// The per-lane partial sums s, bl of each R-lane set, summed (after a row's
// or segment's last batch).
template <int R, int W, int V>
__device__ __forceinline__ void quad_reduce(FwdState<W, V>& st) {
#pragma unroll
  for (int v = 0; v < V; ++v) {
    st.s[v] = quad_sum<R>(st.s[v]);
    st.bl[v] = quad_sum<R>(st.bl[v]);
  }
}

template <int L, int W, int V>
__device__ __forceinline__ void fwd_merge_groups(FwdState<W, V>& st) {
  for_offsets<L, kWave>([&](auto OC) {
    constexpr int o = decltype(OC)::value;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float a2[W], l2[W];
#pragma unroll
      for (int w = 0; w < W; ++w) {
        a2[w] = xor_shfl<o>(st.acc[v][w]);
        l2[w] = xor_shfl<o>(st.accl[v][w]);
      }
      const float m2 = xor_shfl<o>(st.m[v]), s2 = xor_shfl<o>(st.s[v]), b2 = xor_shfl<o>(st.bl[v]);
      st.merge(v, m2, s2, b2, a2, l2);
    }
  });
}

template <typename T, int L, int V>
__device__ __forceinline__ void load_attn_row(const GatFwdArgs<T>& a, const FlLane<L, V>& ln, int row,
                                              float (&ar)[V]) {
#pragma unroll
  for (int v = 0; v < V; ++v) ar[v] = a.attn_row[static_cast<int64_t>(row) * a.H + ln.hq[v]];
}

// Head mean + bias + SiLU of a row; every lane of the wavefront calls this
// (the head sum is an in-lane sum over the chunks plus a butterfly inside the
// group), `write` selects the group that stores. Lanes of head 0 write
// channels [cw*W, cw*W + W) of pre/out; lane cw = 0 of each head writes
// edge_max / edge_sum. With a.agg, a lane also writes its normalised chunks
// of the two aggregates and lane cw = 0 the head's sum_e s l'.
template <typename T, int L, int V>
__device__ __forceinline__ void fwd_emit(const GatFwdArgs<T>& a, const FlLane<L, V>& ln, int cq, int row, bool write,
                                         const FwdState<FlGeom<T>::W, V>& st) {
  constexpr int W = FlGeom<T>::W;
  const int F = a.H * a.C;
  const int64_t nF = static_cast<int64_t>(a.n) * F;
  float y[W];
#pragma unroll
  for (int w = 0; w < W; ++w) y[w] = 0.0f;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const float inv = st.s[v] > 0.0f ? 1.0f / st.s[v] : 0.0f;
    float yv[W];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      yv[w] = ln.qv[v] ? st.acc[v][w] * inv : 0.0f;
      y[w] += yv[w];
    }
    if (a.agg && write && ln.qv[v]) {
      float yl[W];
#pragma unroll
      for (int w = 0; w < W; ++w) yl[w] = st.accl[v][w] * inv;
      store_f32<W>(a.agg + static_cast<int64_t>(row) * F + ln.q[v] * W, yv);
      store_f32<W>(a.agg + nF + static_cast<int64_t>(row) * F + ln.q[v] * W, yl);
      if (ln.cw == 0) a.agg[2 * nF + static_cast<int64_t>(row) * a.H + ln.hq[v]] = st.bl[v] * inv;
    }
  }
  for_offsets<1, L>([&](auto OC) {
    constexpr int o = decltype(OC)::value;
    if (o >= cq)
#pragma unroll
      for (int w = 0; w < W; ++w) y[w] += xor_shfl<o>(y[w]);
  });
  if (!write) return;
  if (ln.qv[0] && ln.hq[0] == 0) {
    const int64_t base = static_cast<int64_t>(row) * a.C + ln.cw * W;
    const float inv_h = 1.0f / static_cast<float>(a.H);
    float pr[W], o[W];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      pr[w] = y[w] * inv_h + a.bias[ln.cw * W + w];
      o[w] = silu(pr[w]);
    }
    store_f32<W>(a.pre + base, pr);
    Chunk<GatOut<T>, W>::store(a.out + base, o);
  }
  if (ln.cw == 0)
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (ln.qv[v]) {
        a.emax[static_cast<int64_t>(row) * a.H + ln.hq[v]] = st.m[v];
        a.esum[static_cast<int64_t>(row) * a.H + ln.hq[v]] = st.s[v];
      }
}

// Heavy-segment merge of the four waves' states into wave 0, one wave at a
// time through one LDS slot of V * 64 * (2W + 3) floats.
template <int W, int V>
__device__ __forceinline__ void fwd_merge_waves(FwdState<W, V>& st, float* slot, int wave, int gl, bool publish) {
  constexpr int S = 2 * W + 3;
  for (int src = 1; src < kWavesPerBlock; ++src) {
    if (wave == src && publish)
#pragma unroll
      for (int v = 0; v < V; ++v) {
        float* d = slot + (v * kWave + gl) * S;
        d[0] = st.m[v];
        d[1] = st.s[v];
        d[2] = st.bl[v];
#pragma unroll
        for (int w = 0; w < W; ++w) {
          d[3 + w] = st.acc[v][w];
          d[3 + W + w] = st.accl[v][w];
        }
      }
    __syncthreads();
    if (wave == 0)
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float* d = slot + (v * kWave + gl) * S;
        float a2[W], l2[W];
#pragma unroll
        for (int w = 0; w < W; ++w) {
          a2[w] = d[3 + w];
          l2[w] = d[3 + W + w];
        }
        st.merge(v, d[0], d[1], d[2], a2, l2);
      }
    __syncthreads();
  }
}

template <typename T, int L, int V, bool DROP, int R, int UM>
__global__ __launch_bounds__(kBlock) void gat_fwd_fl_kernel(GatFwdArgs<T> a, Sched s, int n_mid, int mid_blocks,
                                                            int lgcq) {
  constexpr int W = FlGeom<T>::W;
  constexpr int G = kWave / L;
  const int cq = 1 << lgcq;
  const int nq = a.H * cq;
  const int F = a.H * a.C;
  const FlLane<L, V> ln(lgcq, nq);
  const int wave = wave_id();
  FwdState<W, V> st;
  st.clear();
  float ar[V];
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
      load_attn_row(a, ln, r.x, ar);
      const int need = wave_group_max<L>(deg);
      fwd_edges<T, L, V, DROP, R, UM>(a, ln, jj, ln.g * L, 0, 1, deg, need, r.y, ar, st);
      quad_reduce<R>(st);
      fwd_emit<T, L, V>(a, ln, cq, r.x, has, st);
      return;
    }
    // Medium rows (L < degree <= 64): one per wavefront, group g takes edges
    // g, g + G, ...
    const int li = b * kWavesPerBlock + wave;
    if (li >= n_mid) return;  // wave-uniform; no block barrier follows
    const int4 r = s.light[li];
    const int deg = r.z - r.y;
    const int jj = ln.lane < deg ? a.col[r.y + ln.lane] : 0;
    load_attn_row(a, ln, r.x, ar);
    fwd_edges<T, L, V, DROP, R, UM>(a, ln, jj, 0, ln.g, G, deg, (deg + G - 1) / G, r.y, ar, st);
    quad_reduce<R>(st);
    fwd_merge_groups<L, W, V>(st);
    fwd_emit<T, L, V>(a, ln, cq, r.x, ln.g == 0, st);
    return;
  }

  // Heavy-row segment: wave w takes edges [64w, 64w + 64) of every 256-edge
  // round of the segment.
  __shared__ float slot[V * kWave * (2 * W + 3)];
  __shared__ int flag;
  const int4 sg = s.seg[b];
  const int row = sg.x;
  const int2 hr = s.hrow[sg.w];
  load_attn_row(a, ln, row, ar);
  // The next round's column indices are loaded before this round's gathers,
  // so a round waits on one memory latency (the gathers) instead of two.
  int tb = sg.y + wave * kWave;
  int jj = tb + ln.lane < sg.z ? a.col[tb + ln.lane] : 0;
  for (; tb < sg.z; tb += kSegRound) {
    const int cnt = min(kWave, sg.z - tb);
    const int tn = tb + kSegRound + ln.lane;
    const int jn = tn < sg.z ? a.col[tn] : 0;
    fwd_edges<T, L, V, DROP, R, UM>(a, ln, jj, 0, ln.g, G, cnt, (cnt + G - 1) / G, tb, ar, st);
    jj = jn;
  }
  quad_reduce<R>(st);
  fwd_merge_groups<L, W, V>(st);
  fwd_merge_waves<W, V>(st, slot, wave, ln.gl, ln.g == 0);
  if (hr.y == 1) {
    if (wave == 0) fwd_emit<T, L, V>(a, ln, cq, row, ln.g == 0, st);
    return;
  }
  // Segment partial: acc [F], accl [F], then m, s, bl per head.
  const int stride = 2 * F + 3 * a.H;
  float* mine = a.partial + static_cast<int64_t>(b) * stride;
  if (wave == 0 && ln.g == 0)
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (ln.qv[v]) {
        st_agent_n<W>(mine + ln.q[v] * W, st.acc[v]);
        st_agent_n<W>(mine + F + ln.q[v] * W, st.accl[v]);
        if (ln.cw == 0) {
          st_agent(mine + 2 * F + ln.hq[v], st.m[v]);
          st_agent(mine + 2 * F + a.H + ln.hq[v], st.s[v]);
          st_agent(mine + 2 * F + 2 * a.H + ln.hq[v], st.bl[v]);
        }
      }
  if (!arrive_last(a.counters + sg.w, hr.y, &flag)) return;
  if (wave != 0) return;
  // Last segment to finish: merge every segment's partial in segment order.
  st.clear();
  for (int z = 0; z < hr.y; ++z) {
    const float* pz = a.partial + static_cast<int64_t>(hr.x + z) * stride;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float a2[W], l2[W];
      ld_agent_n<W>(pz + ln.q[v] * W, a2);
      ld_agent_n<W>(pz + F + ln.q[v] * W, l2);
      st.merge(v, ld_agent(pz + 2 * F + ln.hq[v]), ld_agent(pz + 2 * F + a.H + ln.hq[v]),
               ld_agent(pz + 2 * F + 2 * a.H + ln.hq[v]), a2, l2);
    }
  }
  fwd_emit<T, L, V>(a, ln, cq, row, ln.g == 0, st);
}

template <typename T, int L, int V>
struct FwdFlLauncher {
  static int run(hipStream_t st, const GatFwdArgs<T>& a, const Sched& s, const int32_t* hdr, int lgcq);
};

// Out of class, so that the extern template declarations of the
// translation units that only call a launcher also suppress its kernels.
template <typename T, int L, int V>
int FwdFlLauncher<T, L, V>::run(hipStream_t st, const GatFwdArgs<T>& a, const Sched& s, const int32_t* hdr, int lgcq) {
  constexpr int G = kWave / L;
  const int n_mid = G > 1 ? sched_count_gt(hdr, L) : s.n_light;
  const int mid_blocks = (n_mid + kWavesPerBlock - 1) / kWavesPerBlock;
  const int n_tiny = s.n_light - n_mid;
  const int blocks = s.n_seg + mid_blocks + (n_tiny + kWavesPerBlock * G - 1) / (kWavesPerBlock * G);
  if (blocks <= 0) return kOk;
  // R lanes per head share the softmax work: min(cq, 4) (cq <= L).
  const bool big = a.graph_nnz >= big_graph_edges();
  constexpr int kU = std::is_same_v<T, float> && V == 1 ? kFwdUNarrowF32 : kFwdU;
  auto launch = [&](auto RC) {
    constexpr int R = decltype(RC)::value;
    if (a.p > 0.0f) {
      if (big)
        hipLaunchKernelGGL((gat_fwd_fl_kernel<T, L, V, true, R, kFwdUBig>), dim3(blocks), dim3(kBlock), 0, st, a, s,
                           n_mid, mid_blocks, lgcq);
      else
        hipLaunchKernelGGL((gat_fwd_fl_kernel<T, L, V, true, R, kU>), dim3(blocks), dim3(kBlock), 0, st, a, s,
                           n_mid, mid_blocks, lgcq);
    } else {
      if (big)
        hipLaunchKernelGGL((gat_fwd_fl_kernel<T, L, V, false, R, kFwdUBig>), dim3(blocks), dim3(kBlock), 0, st, a, s,
                           n_mid, mid_blocks, lgcq);
      else
        hipLaunchKernelGGL((gat_fwd_fl_kernel<T, L, V, false, R, kU>), dim3(blocks), dim3(kBlock), 0, st, a, s,
                           n_mid, mid_blocks, lgcq);
    }
  };
  if constexpr (L >= 4) {
    if (lgcq >= 2) launch(std::integral_constant<int, 4>());
    else if (lgcq == 1) launch(std::integral_constant<int, 2>());
    else launch(std::integral_constant<int, 1>());
  } else if constexpr (L == 2) {
    if (lgcq >= 1) launch(std::integral_constant<int, 2>());
    else launch(std::integral_constant<int, 1>());
  } else {
    launch(std::integral_constant<int, 1>());
  }
  return check_launch("cign_gat_fwd (feature layout)");
}

// ===========================================================================
// Backward, rows (CSR)
// ===========================================================================
template <int W, int V>
struct RowAcc {
  float vs[V][W], vsl[V][W];
  float B[V];
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int v = 0; v < V; ++v) {
#pragma unroll
      for (int w = 0; w < W; ++w) vs[v][w] = vsl[v][w] = 0.0f;
      B[v] = 0.0f;
    }
  }
};

// Per-row constants of a lane's heads: attn_row, edge_max, 1 / edge_sum (0
// for an empty row).
template <int V>
struct RowHead {
  float ar[V], em[V], ies[V];
};

template <typename T>
__device__ __forceinline__ void row_head1(const GatBwdArgs<T>& a, int row, int hq, float& ar, float& em,
                                          float& ies) {
  const int64_t rh = static_cast<int64_t>(row) * a.H + hq;
  ar = a.attn_row[rh];
  em = a.emax[rh];
  const float es = a.esum[rh];
  ies = es > 0.0f ? 1.0f / es : 0.0f;
}

template <typename T, int L, int V>
__device__ __forceinline__ RowHead<V> row_head(const GatBwdArgs<T>& a, int row, const FlLane<L, V>& ln) {
  RowHead<V> h;
#pragma unroll
  for (int v = 0; v < V; ++v) row_head1(a, row, ln.hq[v], h.ar[v], h.em[v], h.ies[v]);
  return h;
}

template <typename T, int L, int V, bool DROP>
struct RowBatches {
  static constexpr int W = FlGeom<T>::W;
  const GatBwdArgs<T>& a;
  const FlLane<L, V>& ln;
  int jj, base, first, step, cnt, ebase;
  const RowHead<V>& rh;
  RowAcc<W, V>& st;

  template <int U>
  __device__ __forceinline__ void run(int k0) {
    const int F = a.H * a.C;
    typename Chunk<T, W>::Raw xb[U][V];
    float ab[U][V];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const int j = shfl(jj, (base + u) & (kWave - 1));
#pragma unroll
      for (int v = 0; v < V; ++v) {
        ab[k][v] = a.attn_col[static_cast<int64_t>(j) * a.H + ln.hq[v]];
        xb[k][v] = Chunk<T, W>::load_raw(a.x + static_cast<int64_t>(j) * F + ln.q[v] * W);
      }
    }
    // Dropout mask bytes: each (edge, head) pair loaded once.
    PairBits<(DROP ? U : 1), L> kb;
    if constexpr (DROP)
      kb.compute(a.H, ln.gl, [&](int k, int h, bool own) {
        const int u = first + (k0 + k) * step;
        return own && u < cnt && a.mask[static_cast<int64_t>(ebase + u) * a.H + h] != 0;
      });
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float raw = rh.ar[v] + ab[k][v];
        const float lp = raw < 0.0f ? a.slope : 1.0f;
        const float sm = u < cnt ? softmax_exp(leaky(raw, a.slope) - rh.em[v]) * rh.ies[v] : 0.0f;
        float sk = sm;
        if constexpr (DROP) sk = kb.get(k, ln.hq[v], ln.g) ? sm * (1.0f / (1.0f - a.p)) : 0.0f;
        const float skl = sk * lp;
        st.B[v] = fmaf(sm, lp, st.B[v]);
        float xv[W];
        Chunk<T, W>::unpack(xb[k][v], xv);
#pragma unroll
        for (int w = 0; w < W; ++w) {
          st.vs[v][w] = fmaf(sk, xv[w], st.vs[v][w]);
          st.vsl[v][w] = fmaf(skl, xv[w], st.vsl[v][w]);
        }
      }
    }
  }
};

template <typename T, int L, int V, bool DROP>
__device__ __forceinline__ void rows_edges(const GatBwdArgs<T>& a, const FlLane<L, V>& ln, int jj, int base,
                                           int first, int step, int cnt, int need, int ebase, const RowHead<V>& rh,
                                           RowAcc<FlGeom<T>::W, V>& st) {
  RowBatches<T, L, V, DROP> rb{a, ln, jj, base, first, step, cnt, ebase, rh, st};
  for_batches<batch_cap(kRowsU, V)>(need, rb);
}

template <int L, int W, int V>
__device__ __forceinline__ void rows_group_sum(RowAcc<W, V>& st) {
#pragma unroll
  for (int v = 0; v < V; ++v) {
    group_sum<L, W>(st.vs[v]);
    group_sum<L, W>(st.vsl[v]);
    st.B[v] = group_sum1<L>(st.B[v]);
  }
}

// g_pre chunk cw of a row: g_y * SiLU'(pre).
template <typename T>
__device__ __forceinline__ void grad_pre_chunk(const GatBwdArgs<T>& a, int row, int cw,
                                               float (&gp)[FlGeom<T>::W]) {
  constexpr int W = FlGeom<T>::W;
  const int64_t base = static_cast<int64_t>(row) * a.C + cw * W;
  float gy[W], pr[W];
  Chunk<GatOut<T>, W>::load(a.grad_y + base, gy);
  load_f32<W>(a.pre + base, pr);
#pragma unroll
  for (int w = 0; w < W; ++w) gp[w] = gy[w] * silu_grad(pr[w]);
}

// (wsum, A) of each of the lane's heads from the accumulated chunks: dot with
// g_pre, summed over the head's cq lanes, divided by H.
template <int W, int V>
__device__ __forceinline__ void rows_dots(const RowAcc<W, V>& st, const float (&gp)[W], int cq, float inv_h,
                                          float (&wsum)[V], float (&A)[V]) {
  float d[2 * V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    float d1 = 0.0f, d2 = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      d1 = fmaf(gp[w], st.vs[v][w], d1);
      d2 = fmaf(gp[w], st.vsl[v][w], d2);
    }
    d[v] = d1;
    d[V + v] = d2;
  }
  head_sum_n<2 * V>(d, cq);
#pragma unroll
  for (int v = 0; v < V; ++v) {
    wsum[v] = d[v] * inv_h;
    A[v] = d[V + v] * inv_h;
  }
}

template <typename T>
__device__ __forceinline__ void rows_store(const GatBwdArgs<T>& a, int row, int hq, float ar, float em, float ies,
                                           float wsum, float A, float B) {
  a.grad_attn_row[static_cast<int64_t>(row) * a.H + hq] = A - wsum * B;
  a.rowstat[static_cast<int64_t>(row) * a.rs_stride + hq] = make_float4(ar, em, ies, wsum);
}

// Lane stores of a finished light row: grad_attn_row / rowstat of its heads
// (lanes cw = 0) and the g_pre chunk (head-0 lanes).
template <typename T, int L, int V>
__device__ __forceinline__ void rows_emit(const GatBwdArgs<T>& a, const FlLane<L, V>& ln, int row,
                                          const RowHead<V>& rh, const float (&wsum)[V], const float (&A)[V],
                                          const float (&B)[V], const float (&gp)[FlGeom<T>::W]) {
  constexpr int W = FlGeom<T>::W;
  if (ln.cw == 0)
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (ln.qv[v]) rows_store(a, row, ln.hq[v], rh.ar[v], rh.em[v], rh.ies[v], wsum[v], A[v], B[v]);
  if (ln.qv[0] && ln.hq[0] == 0) store_f32<W>(a.grad_pre + static_cast<int64_t>(row) * a.gp_stride + ln.cw * W, gp);
}

template <typename T, int L, int V, bool DROP>
__global__ __launch_bounds__(kBlock) void gat_bwd_rows_fl_kernel(GatBwdArgs<T> a, Sched s, int n_mid, int mid_blocks,
                                                                 int lgcq) {
  constexpr int W = FlGeom<T>::W;
  constexpr int G = kWave / L;
  const int cq = 1 << lgcq;
  const int nq = a.H * cq;
  const FlLane<L, V> ln(lgcq, nq);
  const int wave = wave_id();
  __shared__ float red[kWavesPerBlock][3][kFlHeads];
  __shared__ int flag;
  RowAcc<W, V> st;
  st.clear();
  float gp[W];
  float wsum[V], A[V];
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
    const RowHead<V> rh = row_head(a, row, ln);
    grad_pre_chunk(a, row, ln.cw, gp);
    if (tiny) {
      rows_edges<T, L, V, DROP>(a, ln, jj, ln.g * L, 0, 1, deg, wave_group_max<L>(deg), r.y, rh, st);
    } else {
      rows_edges<T, L, V, DROP>(a, ln, jj, 0, ln.g, G, deg, (deg + G - 1) / G, r.y, rh, st);
      rows_group_sum<L, W, V>(st);
    }
    rows_dots<W, V>(st, gp, cq, a.inv_h, wsum, A);
    if (has && (tiny || ln.g == 0)) rows_emit(a, ln, row, rh, wsum, A, st.B, gp);
    return;
  }

  // Heavy-row segment: the four waves' (wsum, A, B) per head, then across the
  // row's segments (last to finish, in segment order).
  const int4 sg = s.seg[b];
  const int row = sg.x;
  const int2 hr = s.hrow[sg.w];
  const RowHead<V> rh = row_head(a, row, ln);
  grad_pre_chunk(a, row, ln.cw, gp);
  // next round's indices loaded before this round's gathers, as in the forward
  int tb = sg.y + wave * kWave;
  int jj = tb + ln.lane < sg.z ? a.col[tb + ln.lane] : 0;
  for (; tb < sg.z; tb += kSegRound) {
    const int cnt = min(kWave, sg.z - tb);
    const int tn = tb + kSegRound + ln.lane;
    const int jn = tn < sg.z ? a.col[tn] : 0;
    rows_edges<T, L, V, DROP>(a, ln, jj, 0, ln.g, G, cnt, (cnt + G - 1) / G, tb, rh, st);
    jj = jn;
  }
  rows_group_sum<L, W, V>(st);
  rows_dots<W, V>(st, gp, cq, a.inv_h, wsum, A);
  if (ln.g == 0 && ln.cw == 0)
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (ln.qv[v]) {
        red[wave][0][ln.hq[v]] = wsum[v];
        red[wave][1][ln.hq[v]] = A[v];
        red[wave][2][ln.hq[v]] = st.B[v];
      }
  // The row's g_pre is published once, by its first segment.
  if (b == hr.x && wave == 0 && ln.g == 0 && ln.qv[0] && ln.hq[0] == 0)
    store_f32<W>(a.grad_pre + static_cast<int64_t>(row) * a.gp_stride + ln.cw * W, gp);
  __syncthreads();
  if (threadIdx.x < 3 * kFlHeads) {
    const int k = threadIdx.x / kFlHeads, h = threadIdx.x % kFlHeads;
    red[0][k][h] = red[0][k][h] + red[1][k][h] + red[2][k][h] + red[3][k][h];
  }
  __syncthreads();
  if (hr.y == 1) {
    if (threadIdx.x < a.H) {
      const int h = threadIdx.x;
      float ar, em, ies;
      row_head1(a, row, h, ar, em, ies);
      rows_store(a, row, h, ar, em, ies, red[0][0][h], red[0][1][h], red[0][2][h]);
    }
    return;
  }
  float* mine = a.part_row + static_cast<int64_t>(b) * 3 * a.H;
  if (threadIdx.x < 3 * a.H) st_agent(mine + threadIdx.x, red[0][threadIdx.x / a.H][threadIdx.x % a.H]);
  if (!arrive_last(a.row_counters + sg.w, hr.y, &flag)) return;
  if (threadIdx.x < a.H) {
    const int h = threadIdx.x;
    float w = 0.0f, AA = 0.0f, BB = 0.0f;
    for (int z = 0; z < hr.y; ++z) {
      const float* pz = a.part_row + static_cast<int64_t>(hr.x + z) * 3 * a.H;
      w += ld_agent(pz + h);
      AA += ld_agent(pz + a.H + h);
      BB += ld_agent(pz + 2 * a.H + h);
    }
    float ar, em, ies;
    row_head1(a, row, h, ar, em, ies);
    rows_store(a, row, h, ar, em, ies, w, AA, BB);
  }
}

// Rows pass from the forward's per-row aggregates (a.agg): the same
// (wsum, A, B) as gat_bwd_rows_fl_kernel without gathering any source row, a
// stream over the rows. A group of L lanes per row, G rows per wavefront.
template <typename T, int L, int V>
__global__ __launch_bounds__(kBlock) void gat_bwd_rows_agg_kernel(GatBwdArgs<T> a, int lgcq) {
  constexpr int W = FlGeom<T>::W;
  constexpr int G = kWave / L;
  const int cq = 1 << lgcq;
  const FlLane<L, V> ln(lgcq, a.H * cq);
  const int row = (blockIdx.x * kWavesPerBlock + wave_id()) * G + ln.g;
  if (row >= a.n) return;  // no barrier follows
  const int F = a.H * a.C;
  const int64_t nF = static_cast<int64_t>(a.n) * F;
  RowAcc<W, V> st;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    load_f32<W>(a.agg + static_cast<int64_t>(row) * F + ln.q[v] * W, st.vs[v]);
    load_f32<W>(a.agg + nF + static_cast<int64_t>(row) * F + ln.q[v] * W, st.vsl[v]);
    st.B[v] = a.agg[2 * nF + static_cast<int64_t>(row) * a.H + ln.hq[v]];
  }
  float gp[W];
  grad_pre_chunk(a, row, ln.cw, gp);
  const RowHead<V> rh = row_head(a, row, ln);  // issued with the loads above, before any use
  float wsum[V], A[V];
  rows_dots<W, V>(st, gp, cq, a.inv_h, wsum, A);
  rows_emit(a, ln, row, rh, wsum, A, st.B, gp);
}

// ===========================================================================
// Backward, columns (CSC)
// ===========================================================================
// ug = sum s kw g_pre and ua = sum s kw l' g_pre per owned chunk; t = sum s l'
// wsum per owned chunk's head. Wide columns (pair weights) accumulate t per
// pair lane in tp first and distribute it with cols_pair_t.
template <int W, int V>
struct ColAcc {
  float ug[V][W], ua[V][W];
  float t[V];
  float tp;
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int v = 0; v < V; ++v) {
#pragma unroll
      for (int w = 0; w < W; ++w) ug[v][w] = ua[v][w] = 0.0f;
      t[v] = 0.0f;
    }
    tp = 0.0f;
  }
};

// Columns whose lanes own several chunks (V > 1, a wavefront per column)
// compute each (entry, head) weight once per wavefront: with every lane
// evaluating the softmax weight of each of its heads, the exponentials, the
// row-record loads and the dropout division were repeated cq times per pair
// and bounded the kernel.
template <int V>
constexpr bool cols_pairwise() {
  return V > 1;
}

// Softmax weight e^(leaky(raw) - max) / sum of a CSC entry from its
// destination row's record rs = {attn_row, max, 1/sum, wsum}; 0 for an unused
// slot. Branch-free: an unused slot's record (some valid row's) is loaded
// like the others and the selects leave nothing to do conditionally, so the
// whole record arrives in one 16-byte load instead of a second load issued
// behind a branch once the first has returned.
__device__ __forceinline__ float col_weight(const float4& rs, float raw, float slope, bool own) {
  return softmax_exp(own ? leaky(raw, slope) - rs.y : -__builtin_inff()) * (own ? rs.z : 0.0f);
}

// Float offset of record row i (i < 2^31, stride < 2^31): one 32 x 32 -> 64
// bit multiply.
__device__ __forceinline__ uint64_t rec_off(uint32_t i, int stride) {
  return static_cast<uint64_t>(i) * static_cast<uint32_t>(stride);
}

// Batches of CSC entries of column j: slot u's destination row is held by
// lane (base + u) mod 64 in ii, its CSR edge id (used only with dropout) in
// ee. Every lane holds a valid row and edge id (0 where it has no entry), so
// a slot past cnt reads some valid record, weighted 0, without a clamp. The
// g_pre chunk of a destination row is shared by the lane's V heads.
template <typename T, int L, int V, bool DROP>
struct ColBatches {
  static constexpr int W = FlGeom<T>::W;
  const GatBwdArgs<T>& a;
  const FlLane<L, V>& ln;
  int ii, ee, base, first, step, cnt;
  const float (&ac)[V];
  ColAcc<W, V>& st;

  template <int U>
  __device__ __forceinline__ void run(int k0) {
    float gb[U][W];
    float4 rs[U][V];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const int src = (base + u) & (kWave - 1);
      const uint32_t i = shfl(ii, src);
      load_f32<W>(a.grad_pre + rec_off(i, a.gp_stride) + ln.cw * W, gb[k]);
#pragma unroll
      for (int v = 0; v < V; ++v) rs[k][v] = a.rowstat[rec_off(i, a.rs_stride) + ln.hq[v]];
    }
    // Dropout mask bytes (CSR edge id from perm): each (entry, head) pair
    // loaded once.
    PairBits<(DROP ? U : 1), L> kb;
    if constexpr (DROP)
      kb.compute(a.H, ln.gl, [&](int k, int h, bool own) {
        const int u = first + (k0 + k) * step;
        const int e = shfl(ee, (base + u) & (kWave - 1));
        return own && u < cnt && a.mask[static_cast<int64_t>(e) * a.H + h] != 0;
      });
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float raw = rs[k][v].x + ac[v];
        const float lp = raw < 0.0f ? a.slope : 1.0f;
        const float sm = col_weight(rs[k][v], raw, a.slope, u < cnt);
        float w = sm;
        if constexpr (DROP) w = kb.get(k, ln.hq[v], ln.g) ? sm * (1.0f / (1.0f - a.p)) : 0.0f;
        const float wl = w * lp;
        st.t[v] = fmaf(sm * lp, rs[k][v].w, st.t[v]);
#pragma unroll
        for (int q = 0; q < W; ++q) {
          st.ug[v][q] = fmaf(w, gb[k][q], st.ug[v][q]);
          st.ua[v][q] = fmaf(wl, gb[k][q], st.ua[v][q]);
        }
      }
    }
  }
};

template <typename T, int L, int V, bool DROP, int R>
struct ColSharedBatches {
  static constexpr int W = FlGeom<T>::W;
  const GatBwdArgs<T>& a;
  const FlLane<L, V>& ln;
  int ii, ee, base, first, step, cnt;
  const float (&ac)[V];
  ColAcc<W, V>& st;

  // Every lane gathers its g_pre chunk of all U destination rows; the row
  // record, the exponential and the dropout byte of each (entry, head) pair
  // are handled once per R lanes of the head (slots r, r + R, ... by lane r,
  // weights shared by DPP broadcast, t a per-lane partial until
  // cols_quad_reduce), as in the forward.
  template <int U>
  __device__ __forceinline__ void run(int k0) {
    constexpr int NT = (U + R - 1) / R;
    float gb[U][W];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const uint32_t i = shfl(ii, (base + u) & (kWave - 1));
      load_f32<W>(a.grad_pre + rec_off(i, a.gp_stride) + ln.cw * W, gb[k]);
    }
    const int r = ln.gl & (R - 1);
    float wk[NT][V], wl[NT][V];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int kk = R * t + r;
      const int u = first + (k0 + kk) * step;
      const bool own = kk < U && u < cnt;
      const int src = (base + u) & (kWave - 1);
      const uint32_t i = shfl(ii, src);
      int e = 0;
      if constexpr (DROP) e = shfl(ee, src);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float4 rs = a.rowstat[rec_off(i, a.rs_stride) + ln.hq[v]];
        const float raw = rs.x + ac[v];
        const float lp = raw < 0.0f ? a.slope : 1.0f;
        const float sm = col_weight(rs, raw, a.slope, own);
        float w = sm;
        // (an unused slot's e is a valid edge id: its mask byte is read and
        // ignored)
        if constexpr (DROP)
          w = (a.mask[static_cast<int64_t>(e) * a.H + ln.hq[v]] != 0) ? sm * (1.0f / (1.0f - a.p)) : 0.0f;
        st.t[v] = fmaf(sm * lp, rs.w, st.t[v]);
        wk[t][v] = w;
        wl[t][v] = w * lp;
      }
    }
    static_for<U>([&](auto KC) {
      constexpr int k = decltype(KC)::value;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float w = quad_bcast<R, k % R>(wk[k / R][v]);
        const float wlk = quad_bcast<R, k % R>(wl[k / R][v]);
#pragma unroll
        for (int q = 0; q < W; ++q) {
          st.ug[v][q] = fmaf(w, gb[k][q], st.ug[v][q]);
          st.ua[v][q] = fmaf(wlk, gb[k][q], st.ua[v][q]);
        }
      }
    });
  }
};

// t of each R-lane set summed (per-lane partials of ColBatches), after a
// column's or segment's last batch.
template <int R, int W, int V>
__device__ __forceinline__ void cols_quad_reduce(ColAcc<W, V>& st) {
  if constexpr (!cols_pairwise<V>())
#pragma unroll
    for (int v = 0; v < V; ++v) st.t[v] = quad_sum<R>(st.t[v]);
}

// Pairwise batches: pair (slot k, head h) belongs to lane (k % SPR) * S + h of
// the group in round k / SPR (the PairBits layout). The pair lane loads the
// destination row's record and the mask byte, forms w = s kw and wl = w l'
// and adds s l' wsum to its tp; every lane then reads the w, wl of its
// chunks' heads by shuffle. acp is attn_col of the column for the lane's pair
// head gl % S.
template <typename T, int L, int V, bool DROP>
struct ColPairBatches {
  static constexpr int W = FlGeom<T>::W;
  static constexpr int S = L < 8 ? L : 8;
  static constexpr int SPR = L / S;
  const GatBwdArgs<T>& a;
  const FlLane<L, V>& ln;
  int ii, ee, base, first, step, cnt;
  float acp;
  ColAcc<W, V>& st;

  template <int U>
  __device__ __forceinline__ void run(int k0) {
    constexpr int R = (U + SPR - 1) / SPR;
    float gb[U][W];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int u = first + (k0 + k) * step;
      const uint32_t i = shfl(ii, (base + u) & (kWave - 1));
      load_f32<W>(a.grad_pre + rec_off(i, a.gp_stride) + ln.cw * W, gb[k]);
    }
    const int h = ln.gl % S;
    float pw[R], pwl[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = r * SPR + ln.gl / S;
      const int u = first + (k0 + k) * step;
      const bool own = h < a.H && k < U && u < cnt;
      const int src = (base + u) & (kWave - 1);
      const uint32_t i = shfl(ii, src);
      const int hc = h < a.H ? h : a.H - 1;  // pair lanes past the heads read head H-1's record, unused
      const float4 rs = a.rowstat[rec_off(i, a.rs_stride) + hc];
      bool keep = true;
      if constexpr (DROP) {
        const int e = shfl(ee, src);
        keep = a.mask[static_cast<int64_t>(e) * a.H + hc] != 0;
      }
      const float raw = rs.x + acp;
      const float lp = raw < 0.0f ? a.slope : 1.0f;
      const float sm = col_weight(rs, raw, a.slope, own);
      float w = sm;
      if constexpr (DROP) w = keep ? sm * (1.0f / (1.0f - a.p)) : 0.0f;
      st.tp = fmaf(sm * lp, rs.w, st.tp);
      pw[r] = w;
      pwl[r] = w * lp;
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int src = ln.g * L + (k % SPR) * S + ln.hq[v];
        const float w = shfl(pw[k / SPR], src);
        const float wl = shfl(pwl[k / SPR], src);
#pragma unroll
        for (int q = 0; q < W; ++q) {
          st.ug[v][q] = fmaf(w, gb[k][q], st.ug[v][q]);
          st.ua[v][q] = fmaf(wl, gb[k][q], st.ua[v][q]);
        }
      }
    }
  }
};

// ac: attn_col of the column for the lane's chunks' heads (per-lane weights)
// or, pairwise, ac[0] for the lane's pair head.
template <typename T, int L, int V, bool DROP, int R>
__device__ __forceinline__ void cols_edges(const GatBwdArgs<T>& a, const FlLane<L, V>& ln, int ii, int ee, int base,
                                           int first, int step, int cnt, int need, const float (&ac)[V],
                                           ColAcc<FlGeom<T>::W, V>& st) {
  if constexpr (cols_pairwise<V>()) {
    ColPairBatches<T, L, V, DROP> cb{a, ln, ii, ee, base, first, step, cnt, ac[0], st};
    for_batches<batch_cap(kColsPairFloats / FlGeom<T>::W, 1)>(need, cb);
  } else if constexpr (R == 1) {
    ColBatches<T, L, V, DROP> cb{a, ln, ii, ee, base, first, step, cnt, ac, st};
    for_batches<batch_cap(kColsU, V)>(need, cb);
  } else {
    ColSharedBatches<T, L, V, DROP, R> cb{a, ln, ii, ee, base, first, step, cnt, ac, st};
    for_batches<batch_cap(kColsUShared, V)>(need, cb);
  }
}

// Pairwise t: the pair lanes' tp summed over the lanes sharing a pair head,
// within the group (whole_wave false) or the wavefront, then read by each
// owned chunk's head.
template <int L, int W, int V>
__device__ __forceinline__ void cols_pair_t(ColAcc<W, V>& st, const FlLane<L, V>& ln, bool whole_wave) {
  constexpr int S = L < 8 ? L : 8;
  float x = st.tp;
  const int top = whole_wave ? kWave : L;
  for (int o = S; o < top; o <<= 1) x += shfl_xor(x, o);
  const int b = whole_wave ? 0 : ln.g * L;
#pragma unroll
  for (int v = 0; v < V; ++v) st.t[v] = shfl(x, b + ln.hq[v]);
}

// Sums of the wavefront's groups (mid and heavy columns split a column's
// entries over the groups).
template <int L, int W, int V>
__device__ __forceinline__ void cols_group_sum(ColAcc<W, V>& st, const FlLane<L, V>& ln) {
#pragma unroll
  for (int v = 0; v < V; ++v) {
    group_sum<L, W>(st.ug[v]);
    group_sum<L, W>(st.ua[v]);
    if constexpr (!cols_pairwise<V>()) st.t[v] = group_sum1<L>(st.t[v]);
  }
  if constexpr (cols_pairwise<V>()) cols_pair_t<L, W, V>(st, ln, true);
}

// The column's own x chunks, needed after its entries: loaded before the
// entry loop (off the critical path) when a lane owns at most two chunks,
// after it otherwise (to keep registers for the entry batches).
template <typename T, int V>
struct XCol {
  static constexpr int W = FlGeom<T>::W;
  static constexpr bool kEarly = V <= 2;
  typename Chunk<T, W>::Raw raw[kEarly ? V : 1];

  template <int L>
  __device__ __forceinline__ void prefetch(const GatBwdArgs<T>& a, const FlLane<L, V>& ln, int j) {
    if constexpr (kEarly)
#pragma unroll
      for (int v = 0; v < V; ++v) raw[v] = Chunk<T, W>::load_raw(a.x + static_cast<int64_t>(j) * a.H * a.C + ln.q[v] * W);
  }
  template <int L>
  __device__ __forceinline__ void get(const GatBwdArgs<T>& a, const FlLane<L, V>& ln, int j, int v,
                                      float (&xj)[W]) const {
    if constexpr (kEarly) Chunk<T, W>::unpack(raw[v], xj);
    else Chunk<T, W>::load(a.x + static_cast<int64_t>(j) * a.H * a.C + ln.q[v] * W, xj);
  }
};

// The lane's part of grad_attn_col[j, hq[v]] for each chunk v: <ua, x[j]
// chunk> summed over the head's lanes / H, minus t.
template <typename T, int L, int V>
__device__ __forceinline__ void cols_gac(const GatBwdArgs<T>& a, const FlLane<L, V>& ln, const ColAcc<FlGeom<T>::W, V>& st,
                                         const XCol<T, V>& xc, int j, int cq, float (&gac)[V]) {
  constexpr int W = FlGeom<T>::W;
  float d[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    float xj[W];
    xc.get(a, ln, j, v, xj);
    d[v] = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) d[v] = fmaf(st.ua[v][w], xj[w], d[v]);
  }
  head_sum_n<V>(d, cq);
#pragma unroll
  for (int v = 0; v < V; ++v) gac[v] = d[v] * a.inv_h - st.t[v];
}

// attn_col[j] as cols_edges takes it.
template <typename T, int L, int V>
__device__ __forceinline__ void load_attn_col(const GatBwdArgs<T>& a, const FlLane<L, V>& ln, int j, float (&ac)[V]) {
  if constexpr (cols_pairwise<V>()) {
    constexpr int S = L < 8 ? L : 8;
    const int h = ln.gl % S;
    ac[0] = a.attn_col[static_cast<int64_t>(j) * a.H + (h < a.H ? h : a.H - 1)];
  } else {
#pragma unroll
    for (int v = 0; v < V; ++v) ac[v] = a.attn_col[static_cast<int64_t>(j) * a.H + ln.hq[v]];
  }
}

template <typename T, int L, int V, bool DROP, int R>
__global__ __launch_bounds__(kBlock) void gat_bwd_cols_fl_kernel(GatBwdArgs<T> a, Sched s, int n_mid, int mid_blocks,
                                                                 int lgcq) {
  constexpr int W = FlGeom<T>::W;
  constexpr int G = kWave / L;
  const int cq = 1 << lgcq;
  const int nq = a.H * cq;
  const int F = a.H * a.C;
  const FlLane<L, V> ln(lgcq, nq);
  const int wave = wave_id();
  __shared__ float red[V * kWave * W];
  __shared__ float gred[kWavesPerBlock][kFlHeads];
  __shared__ int flag;
  // the grad_bias workgroups first: their sums of grad_pre rows overlap the
  // columns (placed last they were the launch's tail)
  int b = blockIdx.x;
  if (b < a.n_l2) {
    bias_from_grad_pre(a, b, a.col_counters + s.n_hrow, &flag);
    return;
  }
  b -= a.n_l2;
  ColAcc<W, V> st;
  st.clear();
  float ac[V], gac[V];

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
    load_attn_col(a, ln, j, ac);
    XCol<T, V> xc;
    xc.prefetch(a, ln, j);
    if (tiny) {
      cols_edges<T, L, V, DROP, R>(a, ln, ii, ee, ln.g * L, 0, 1, deg, wave_group_max<L>(deg), ac, st);
      cols_quad_reduce<R>(st);
      if constexpr (cols_pairwise<V>()) cols_pair_t<L, W, V>(st, ln, false);
    } else {
      cols_edges<T, L, V, DROP, R>(a, ln, ii, ee, 0, ln.g, G, deg, (deg + G - 1) / G, ac, st);
      cols_quad_reduce<R>(st);
      cols_group_sum<L, W, V>(st, ln);
    }
    cols_gac(a, ln, st, xc, j, cq, gac);
    if (!(has && (tiny || ln.g == 0))) return;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      if (!ln.qv[v]) continue;
      float o[W];
#pragma unroll
      for (int w = 0; w < W; ++w) o[w] = st.ug[v][w] * a.inv_h;
      Chunk<GatOut<T>, W>::store(a.grad_feat + static_cast<int64_t>(j) * F + ln.q[v] * W, o);
      if (ln.cw == 0) a.grad_attn_col[static_cast<int64_t>(j) * a.H + ln.hq[v]] = gac[v];
    }
    return;
  }

  // Heavy column segment: wave w takes entries [64w, 64w + 64) of every
  // 256-entry round of the segment; the waves' sums meet in one LDS slot.
  const int4 sg = s.seg[b];
  const int j = sg.x;
  const int2 hr = s.hrow[sg.w];
  load_attn_col(a, ln, j, ac);
  XCol<T, V> xc;
  xc.prefetch(a, ln, j);
  // next round's entries loaded before this round's gathers, as in the forward
  int tb = sg.y + wave * kWave;
  int ii = tb + ln.lane < sg.z ? a.rowind[tb + ln.lane] : 0;
  int ee = DROP && tb + ln.lane < sg.z ? a.perm[tb + ln.lane] : 0;
  for (; tb < sg.z; tb += kSegRound) {
    const int cnt = min(kWave, sg.z - tb);
    const int tn = tb + kSegRound + ln.lane;
    const int in = tn < sg.z ? a.rowind[tn] : 0;
    const int en = DROP && tn < sg.z ? a.perm[tn] : 0;
    cols_edges<T, L, V, DROP, R>(a, ln, ii, ee, 0, ln.g, G, cnt, (cnt + G - 1) / G, ac, st);
    ii = in;
    ee = en;
  }
  cols_quad_reduce<R>(st);
  cols_group_sum<L, W, V>(st, ln);
  cols_gac(a, ln, st, xc, j, cq, gac);
  if (ln.g == 0 && ln.cw == 0)
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (ln.qv[v]) gred[wave][ln.hq[v]] = gac[v];
  // red[q * W + w] (feature order) = sum of the waves' ug, added one wave at
  // a time.
  for (int src = 0; src < kWavesPerBlock; ++src) {
    if (wave == src && ln.g == 0)
#pragma unroll
      for (int v = 0; v < V; ++v)
        if (ln.qv[v])
#pragma unroll
          for (int w = 0; w < W; ++w) {
            float& d = red[ln.q[v] * W + w];
            d = src == 0 ? st.ug[v][w] : d + st.ug[v][w];
          }
    __syncthreads();
  }
  const bool single = hr.y == 1;
  const int stride = F + a.H;
  float* mine = a.part_col + static_cast<int64_t>(b) * stride;
  for (int k = threadIdx.x; k < F; k += kBlock) {
    const float v = red[k];
    if (single) a.grad_feat[static_cast<int64_t>(j) * F + k] = from_f32<GatOut<T>>(v * a.inv_h);
    else st_agent(mine + k, v);
  }
  if (threadIdx.x < a.H) {
    const int h = threadIdx.x;
    const float v = gred[0][h] + gred[1][h] + gred[2][h] + gred[3][h];
    if (single) a.grad_attn_col[static_cast<int64_t>(j) * a.H + h] = v;
    else st_agent(mine + F + h, v);
  }
  if (single) return;
  if (!arrive_last(a.col_counters + sg.w, hr.y, &flag)) return;
  for (int k = threadIdx.x; k < stride; k += kBlock) {
    float v = 0.0f;
    for (int z = 0; z < hr.y; ++z) v += ld_agent(a.part_col + static_cast<int64_t>(hr.x + z) * stride + k);
    if (k < F) a.grad_feat[static_cast<int64_t>(j) * F + k] = from_f32<GatOut<T>>(v * a.inv_h);
    else a.grad_attn_col[static_cast<int64_t>(j) * a.H + (k - F)] = v;
  }
}

// ===========================================================================
// Backward, columns, channel-major lanes
// ===========================================================================
// Narrow rows of H = 4 heads and C = 4 LC channels (LC in {4, 8, 16}): a
// group of LC lanes owns a column and lane c the channels [4c, 4c + 4) of
// every head, so a destination row's g_pre chunk is gathered once per entry
// rather than once per head as in the head-major lanes above (at 62.4M edges
// those gathers kept the address units 78% busy and the VALU 58%). Lane r of
// the column's first quad loads head r's part of each slot's row record and
// computes its softmax weight; DPP row shifts pass the weights to the other
// quads and quad broadcasts to every lane. Light columns
// (degree <= kFlLightMax) run one per group, G = 64 / LC per wavefront (the
// light list is sorted by degree, so a wavefront's columns need about the
// same number of batches), in batches of U slots whose row indices are loaded
// one batch ahead; heavy columns are segments, as in the head-major kernel.
// Large graphs only (the same threshold as the forward's): a group streams
// all of a light column's entries in sequence, up to 16 dependent batches,
// which bounds a small graph's launch (c2: 30.9 us against 23.1 us for the
// head-major kernel, whose wavefront splits a column of more than L entries
// over its groups).
// 4 slots per batch: at 62.4M edges 2.85 ms for the backward against 3.06 ms
// with 8 (138 VGPRs, one wavefront per SIMD fewer).
#ifndef CIGN_FL_COLS_CM_U
#define CIGN_FL_COLS_CM_U 4
#endif
constexpr int kColsCmHeads = 4;

inline bool cols_cm_ok(int H, int C) { return H == kColsCmHeads && (C == 16 || C == 32 || C == 64); }

// Four consecutive elements of T (16 bytes of fp32, 8 of bf16), kept raw
// while loads are in flight and unpacked on use.
template <typename T>
struct Four;
template <>
struct Four<float> {
  using Raw = float4;
  static __device__ __forceinline__ Raw load(const float* p) { return *reinterpret_cast<const float4*>(p); }
  static __device__ __forceinline__ void unpack(const Raw& q, float (&v)[4]) {
    v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
  }
};
template <>
struct Four<bf16> {
  using Raw = uint2;
  static __device__ __forceinline__ Raw load(const bf16* p) { return *reinterpret_cast<const uint2*>(p); }
  static __device__ __forceinline__ void unpack(const Raw& q, float (&v)[4]) {
    v[0] = __uint_as_float(q.x << 16);
    v[1] = __uint_as_float(q.x & 0xffff0000u);
    v[2] = __uint_as_float(q.y << 16);
    v[3] = __uint_as_float(q.y & 0xffff0000u);
  }
};
template <>
struct Four<bf16x> {
  using Raw = uint2;
  static __device__ __forceinline__ Raw load(const bf16x* p) { return *reinterpret_cast<const uint2*>(p); }
  static __device__ __forceinline__ void unpack(const Raw& q, float (&v)[4]) { Four<bf16>::unpack(q, v); }
};
template <typename T>
__device__ __forceinline__ void store4(T* p, const float (&v)[4]);
template <>
__device__ __forceinline__ void store4<float>(float* p, const float (&v)[4]) {
  Chunk<float, 4>::store(p, v);
}
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, const float (&v)[4]) {
  const uint32_t w0 = from_f32<bf16>(v[0]).bits | (static_cast<uint32_t>(from_f32<bf16>(v[1]).bits) << 16);
  const uint32_t w1 = from_f32<bf16>(v[2]).bits | (static_cast<uint32_t>(from_f32<bf16>(v[3]).bits) << 16);
  *reinterpret_cast<uint2*>(p) = make_uint2(w0, w1);
}

// Sums over a column's entries held by one lane: ug[h] = sum s kw g_pre
// chunk, ua[h] = sum s kw l' g_pre chunk for every head h; t = sum s l' wsum
// for the lane's quad head.
template <int HH>
struct CmAcc {
  float ug[HH][4], ua[HH][4];
  float t;
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int h = 0; h < HH; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) ug[h][q] = ua[h][q] = 0.0f;
    t = 0.0f;
  }
};

// One batch of U slots of a group: slot k's destination row index (and CSR
// edge id, with dropout) is held by lane src0 + k; slots k >= cnt are unused
// (their lanes hold index 0, a valid row and edge, read and ignored). c: the
// lane's channel chunk; hl: its quad lane (the head whose weights it
// computes); ac: attn_col of the column for head min(hl, HH - 1).
#ifndef CIGN_FL_COLS_CM_SHARE
#define CIGN_FL_COLS_CM_SHARE 1
#endif
// Whether only the first quad of a column loads the rows' records and
// computes the weights, the other quads receiving them by DPP row shifts
// (LC >= 8; otherwise every quad loads them): the repeated record loads were
// a quarter of the gathered bytes (62.4M edges: columns kernel 2.198 ms
// against 2.215 ms).
template <int LC>
constexpr bool cm_share() {
  return LC >= 8 && CIGN_FL_COLS_CM_SHARE;
}
// v of the column's first quad in every quad of the column: row_shr by 4, 8,
// 12 lanes into DPP banks 1, 2, 3 (a bank is a quad of a 16-lane row; an
// 8-lane column is banks 0-1 or 2-3 of its row), the other banks keeping
// their value.
template <int LC>
__device__ __forceinline__ float from_quad0(float v) {
  int x = __float_as_int(v);
  if constexpr (LC == 8) {
    x = __builtin_amdgcn_update_dpp(x, x, 0x114, 0xF, 0xA, false);
  } else if constexpr (LC == 16) {
    x = __builtin_amdgcn_update_dpp(x, x, 0x114, 0xF, 0x2, false);
    x = __builtin_amdgcn_update_dpp(x, x, 0x118, 0xF, 0x4, false);
    x = __builtin_amdgcn_update_dpp(x, x, 0x11C, 0xF, 0x8, false);
  }
  return __int_as_float(x);
}

template <typename T, int LC, int HH, bool DROP, int U>
__device__ __forceinline__ void cm_batch(const GatBwdArgs<T>& a, int c, int hl, int ii, int ee, int src0, int cnt,
                                         float ac, CmAcc<HH>& st) {
  constexpr bool kShare = cm_share<LC>();
  const int hc = hl < HH ? hl : HH - 1;
  const bool q0 = !kShare || c < 4;
  float gk[U][4];
  float4 rs[U];
  int mk[DROP ? U : 1];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const uint32_t i = shfl(ii, src0 + k);
    load_f32<4>(a.grad_pre + rec_off(i, a.gp_stride) + 4 * c, gk[k]);
    rs[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if constexpr (DROP) mk[k] = 0;
    if (q0) {
      rs[k] = a.rowstat[rec_off(i, a.rs_stride) + hc];
      if constexpr (DROP) mk[k] = a.mask[static_cast<int64_t>(shfl(ee, src0 + k)) * HH + hc];
    }
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const float raw = rs[k].x + ac;
    const float lp = raw < 0.0f ? a.slope : 1.0f;
    const float sm = col_weight(rs[k], raw, a.slope, k < cnt && hl < HH && q0);
    float w = sm;
    if constexpr (DROP) w = mk[k] != 0 ? sm * (1.0f / (1.0f - a.p)) : 0.0f;
    float wl = w * lp;
    st.t = fmaf(sm * lp, rs[k].w, st.t);
    if constexpr (kShare) {
      w = from_quad0<LC>(w);
      wl = from_quad0<LC>(wl);
    }
    static_for<HH>([&](auto HC) {
      constexpr int h = decltype(HC)::value;
      const float wh = quad_bcast<4, h>(w);
      const float wlh = quad_bcast<4, h>(wl);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        st.ug[h][q] = fmaf(wh, gk[k][q], st.ug[h][q]);
        st.ua[h][q] = fmaf(wlh, gk[k][q], st.ua[h][q]);
      }
    });
  }
}

// d[h] = <ua[h], x[j, h] chunk c> summed over the LC lanes of the group.
template <typename T, int LC, int HH>
__device__ __forceinline__ void cm_dots(const CmAcc<HH>& st, const typename Four<T>::Raw (&xr)[HH], float (&d)[HH]) {
#pragma unroll
  for (int h = 0; h < HH; ++h) {
    float xj[4];
    Four<T>::unpack(xr[h], xj);
    d[h] = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) d[h] = fmaf(st.ua[h][q], xj[q], d[h]);
  }
  for_offsets<1, LC>([&](auto OC) {
#pragma unroll
    for (int h = 0; h < HH; ++h) d[h] += xor_shfl<decltype(OC)::value>(d[h]);
  });
}

template <typename T, int LC, int HH, bool DROP, int U>
__global__ __launch_bounds__(kBlock) void gat_bwd_cols_cm_kernel(GatBwdArgs<T> a, Sched s, int light_blocks) {
  static_assert(LC >= 4 && LC <= 16 && U <= LC && HH <= 4, "channel-major geometry");
  constexpr int G = kWave / LC;
  const int C = a.C;
  const int F = HH * C;
  const int wave = wave_id();
  const int lane = lane_id();
  const int g = lane / LC;
  const int c = lane & (LC - 1);
  const int hl = lane & 3;
  const int hc = hl < HH ? hl : HH - 1;
  __shared__ float red[kWavesPerBlock][LC][HH * 4];
  __shared__ float gred[kWavesPerBlock][HH];
  __shared__ int flag;
  // the grad_bias workgroups first, as in gat_bwd_cols_fl_kernel
  int b = blockIdx.x;
  if (b < a.n_l2) {
    bias_from_grad_pre(a, b, a.col_counters + s.n_hrow, &flag);
    return;
  }
  b -= a.n_l2;
  CmAcc<HH> st;
  st.clear();
  typename Four<T>::Raw xr[HH];

  if (b >= s.n_seg) {
    // Light columns: group g of the wavefront owns light column li. Groups
    // exchange nothing (every shuffle and DPP read below stays within a
    // group), so each runs its own number of batches.
    const int li = ((b - s.n_seg) * kWavesPerBlock + wave) * G + g;
    if (li >= s.n_light) return;
    const int4 r = s.light[li];
    const int j = r.x;
    const int deg = r.z - r.y;
    const int nb = (deg + U - 1) / U;
    const float ac = a.attn_col[static_cast<int64_t>(j) * HH + hc];
    int ii = c < U && c < deg ? a.rowind[r.y + c] : 0;
    int ee = DROP && c < U && c < deg ? a.perm[r.y + c] : 0;
#pragma unroll
    for (int h = 0; h < HH; ++h) xr[h] = Four<T>::load(a.x + static_cast<int64_t>(j) * F + h * C + 4 * c);
    for (int bb = 0; bb < nb; ++bb) {
      const int k0 = bb * U;
      const int kn = k0 + U + c;
      const int in = c < U && kn < deg ? a.rowind[r.y + kn] : 0;
      const int en = DROP && c < U && kn < deg ? a.perm[r.y + kn] : 0;
      cm_batch<T, LC, HH, DROP, U>(a, c, hl, ii, ee, g * LC, deg - k0, ac, st);
      ii = in;
      ee = en;
    }
    float d[HH];
    cm_dots<T, LC, HH>(st, xr, d);
    float gac = 0.0f;
    static_for<HH>([&](auto HC) {
      constexpr int h = decltype(HC)::value;
      const float th = quad_bcast<4, h>(st.t);
      if (c == h) gac = d[h] * a.inv_h - th;
    });
#pragma unroll
    for (int h = 0; h < HH; ++h) {
      float o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = st.ug[h][q] * a.inv_h;
      store4<GatOut<T>>(a.grad_feat + static_cast<int64_t>(j) * F + h * C + 4 * c, o);
    }
    if (c < HH) a.grad_attn_col[static_cast<int64_t>(j) * HH + c] = gac;
    return;
  }

  // Heavy column segment: group gid = wave * G + g takes slots [gid U, gid U
  // + U) of every round of 4 G U entries; the groups' sums are added by
  // butterflies within the wavefront, then wave by wave through LDS.
  constexpr int E = kWavesPerBlock * G * U;
  const int4 sg = s.seg[b];
  const int j = sg.x;
  const int2 hr = s.hrow[sg.w];
  const int gid = wave * G + g;
  const float ac = a.attn_col[static_cast<int64_t>(j) * HH + hc];
#pragma unroll
  for (int h = 0; h < HH; ++h) xr[h] = Four<T>::load(a.x + static_cast<int64_t>(j) * F + h * C + 4 * c);
  int tb = sg.y;
  int t0 = tb + gid * U + c;
  int ii = c < U && t0 < sg.z ? a.rowind[t0] : 0;
  int ee = DROP && c < U && t0 < sg.z ? a.perm[t0] : 0;
  for (; tb < sg.z; tb += E) {
    const int tn = tb + E + gid * U + c;
    const int in = c < U && tn < sg.z ? a.rowind[tn] : 0;
    const int en = DROP && c < U && tn < sg.z ? a.perm[tn] : 0;
    cm_batch<T, LC, HH, DROP, U>(a, c, hl, ii, ee, g * LC, sg.z - (tb + gid * U), ac, st);
    ii = in;
    ee = en;
  }
  float d[HH];
  cm_dots<T, LC, HH>(st, xr, d);
  for_offsets<LC, kWave>([&](auto OC) {
    constexpr int o = decltype(OC)::value;
#pragma unroll
    for (int h = 0; h < HH; ++h) {
#pragma unroll
      for (int q = 0; q < 4; ++q) st.ug[h][q] += xor_shfl<o>(st.ug[h][q]);
      d[h] += xor_shfl<o>(d[h]);
    }
    st.t += xor_shfl<o>(st.t);
  });
  float gac = 0.0f;
  static_for<HH>([&](auto HC) {
    constexpr int h = decltype(HC)::value;
    const float th = quad_bcast<4, h>(st.t);
    if (c == h) gac = d[h] * a.inv_h - th;
  });
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < HH; ++h)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[wave][c][h * 4 + q] = st.ug[h][q];
    if (c < HH) gred[wave][c] = gac;
  }
  __syncthreads();
  const bool single = hr.y == 1;
  const int stride = F + HH;
  float* mine = a.part_col + static_cast<int64_t>(b) * stride;
  if (threadIdx.x < LC * HH * 4) {
    const int cc = threadIdx.x / (HH * 4), h = (threadIdx.x / 4) % HH, q = threadIdx.x % 4;
    const float v = red[0][cc][h * 4 + q] + red[1][cc][h * 4 + q] + red[2][cc][h * 4 + q] + red[3][cc][h * 4 + q];
    const int k = h * C + 4 * cc + q;
    if (single) a.grad_feat[static_cast<int64_t>(j) * F + k] = from_f32<GatOut<T>>(v * a.inv_h);
    else st_agent(mine + k, v);
  }
  if (threadIdx.x < HH) {
    const int h = threadIdx.x;
    const float v = gred[0][h] + gred[1][h] + gred[2][h] + gred[3][h];
    if (single) a.grad_attn_col[static_cast<int64_t>(j) * HH + h] = v;
    else st_agent(mine + F + h, v);
  }
  if (single) return;
  if (!arrive_last(a.col_counters + sg.w, hr.y, &flag)) return;
  for (int k = threadIdx.x; k < stride; k += kBlock) {
    float v = 0.0f;
    for (int z = 0; z < hr.y; ++z) v += ld_agent(a.part_col + static_cast<int64_t>(hr.x + z) * stride + k);
    if (k < F) a.grad_feat[static_cast<int64_t>(j) * F + k] = from_f32<GatOut<T>>(v * a.inv_h);
    else a.grad_attn_col[static_cast<int64_t>(j) * HH + (k - F)] = v;
  }
}

// Launches the channel-major columns kernel for LC = C / 4.
template <typename T>
int launch_cols_cm(hipStream_t st, const GatBwdArgs<T>& a, const Sched& cs) {
  auto go = [&](auto LCC) {
    constexpr int LC = decltype(LCC)::value;
    constexpr int G = kWave / LC;
    constexpr int U = LC < CIGN_FL_COLS_CM_U ? LC : CIGN_FL_COLS_CM_U;
    const int light_blocks = (cs.n_light + kWavesPerBlock * G - 1) / (kWavesPerBlock * G);
    const int cb = cs.n_seg + light_blocks + a.n_l2;
    if (cb == 0) return static_cast<int>(kOk);
    if (a.p > 0.0f)
      hipLaunchKernelGGL((gat_bwd_cols_cm_kernel<T, LC, kColsCmHeads, true, U>), dim3(cb), dim3(kBlock), 0, st, a,
                         cs, light_blocks);
    else
      hipLaunchKernelGGL((gat_bwd_cols_cm_kernel<T, LC, kColsCmHeads, false, U>), dim3(cb), dim3(kBlock), 0, st, a,
                         cs, light_blocks);
    return check_launch("cign_gat_bwd (cols, channel-major)");
  };
  if (a.C == 16) return go(std::integral_constant<int, 4>());
  if (a.C == 32) return go(std::integral_constant<int, 8>());
  return go(std::integral_constant<int, 16>());
}

template <typename T, int L, int V>
struct BwdFlLauncher {
  static int row_blocks(const Sched& rs, const int32_t* rhdr);

  static int run(hipStream_t st, const GatBwdArgs<T>& a, const Sched& rs, const int32_t* rhdr, const Sched& cs,
                 const int32_t* chdr, int lgcq);
};

// Out of class, so that the extern template declarations of the
// translation units that only call a launcher also suppress its kernels.
template <typename T, int L, int V>
int BwdFlLauncher<T, L, V>::row_blocks(const Sched& rs, const int32_t* rhdr) {
  constexpr int G = kWave / L;
  const int r_mid = G > 1 ? sched_count_gt(rhdr, L) : rs.n_light;
  return rs.n_seg + (r_mid + kWavesPerBlock - 1) / kWavesPerBlock +
         (rs.n_light - r_mid + kWavesPerBlock * G - 1) / (kWavesPerBlock * G);
}

template <typename T, int L, int V>
int BwdFlLauncher<T, L, V>::run(hipStream_t st, const GatBwdArgs<T>& a, const Sched& rs, const int32_t* rhdr, const Sched& cs,
                                const int32_t* chdr, int lgcq) {
  constexpr int G = kWave / L;
  const int r_mid = G > 1 ? sched_count_gt(rhdr, L) : rs.n_light;
  const int r_mid_blocks = (r_mid + kWavesPerBlock - 1) / kWavesPerBlock;
  const int rb = row_blocks(rs, rhdr);
  if (a.agg) {
    const int ab = (a.n + kWavesPerBlock * G - 1) / (kWavesPerBlock * G);
    if (ab > 0) {
      hipLaunchKernelGGL((gat_bwd_rows_agg_kernel<T, L, V>), dim3(ab), dim3(kBlock), 0, st, a, lgcq);
      const int rc = check_launch("cign_gat_bwd (rows from aggregates, feature layout)");
      if (rc) return rc;
    }
  } else if (rb > 0) {
    if (a.p > 0.0f)
      hipLaunchKernelGGL((gat_bwd_rows_fl_kernel<T, L, V, true>), dim3(rb), dim3(kBlock), 0, st, a, rs, r_mid,
                         r_mid_blocks, lgcq);
    else
      hipLaunchKernelGGL((gat_bwd_rows_fl_kernel<T, L, V, false>), dim3(rb), dim3(kBlock), 0, st, a, rs, r_mid,
                         r_mid_blocks, lgcq);
    const int rc = check_launch("cign_gat_bwd (rows, feature layout)");
    if (rc) return rc;
  }
  if constexpr (V == 1 && !std::is_same_v<T, bf16h>) {  // (bf16h runs on small graphs only)
    if (cols_cm_ok(a.H, a.C) && a.graph_nnz >= big_graph_edges()) return launch_cols_cm<T>(st, a, cs);
  }
  const int c_mid = G > 1 ? sched_count_gt(chdr, L) : cs.n_light;
  const int c_mid_blocks = (c_mid + kWavesPerBlock - 1) / kWavesPerBlock;
  const int cb = cs.n_seg + c_mid_blocks + (cs.n_light - c_mid + kWavesPerBlock * G - 1) / (kWavesPerBlock * G) +
                 a.n_l2;
  if (cb > 0) {
    // R lanes per head share the per-entry work of narrow columns (wide
    // columns have their pairwise batches).
    auto launch = [&](auto RC) {
      constexpr int R = decltype(RC)::value;
      if (a.p > 0.0f)
        hipLaunchKernelGGL((gat_bwd_cols_fl_kernel<T, L, V, true, R>), dim3(cb), dim3(kBlock), 0, st, a, cs, c_mid,
                           c_mid_blocks, lgcq);
      else
        hipLaunchKernelGGL((gat_bwd_cols_fl_kernel<T, L, V, false, R>), dim3(cb), dim3(kBlock), 0, st, a, cs, c_mid,
                           c_mid_blocks, lgcq);
    };
    // Below kFwdBigGraph edges the columns pass is a few dependent memory
    // rounds and the exchange costs more than it saves (c2: 25.1 us with it,
    // 23.7 us without), so every lane keeps its own weights there.
    const bool share = a.graph_nnz >= big_graph_edges();
    if constexpr (V == 1 && L >= 4) {
      if (!share) launch(std::integral_constant<int, 1>());
      else if (lgcq >= 2) launch(std::integral_constant<int, 4>());
      else if (lgcq == 1) launch(std::integral_constant<int, 2>());
      else launch(std::integral_constant<int, 1>());
    } else if constexpr (V == 1 && L == 2) {
      if (share && lgcq >= 1) launch(std::integral_constant<int, 2>());
      else launch(std::integral_constant<int, 1>());
    } else {
      launch(std::integral_constant<int, 1>());
    }
  }
  return check_launch("cign_gat_bwd (cols, feature layout)");
}

// Narrow rows: one chunk per lane, groups of 1..64 lanes.
#define CIGN_GAT_FL_LIST_NARROW(X, T) \
  X(T, 1, 1) X(T, 2, 1) X(T, 4, 1) X(T, 8, 1) X(T, 16, 1) X(T, 32, 1) X(T, 64, 1)
// Wide rows: a wavefront per row, V chunks per lane.
#define CIGN_GAT_FL_LIST_WIDE(X, T) X(T, 64, 2) X(T, 64, 3) X(T, 64, 4) X(T, 64, 6) X(T, 64, 8)

#define CIGN_GAT_FL_INST_ONE(T, L, V)                      \
  template struct ::cign::gatk::BwdFlLauncher<T, L, V>;    \
  template struct ::cign::gatk::FwdFlLauncher<T, L, V>;
#define CIGN_GAT_FL_DECL_ONE(T, L, V)                             \
  extern template struct ::cign::gatk::BwdFlLauncher<T, L, V>;    \
  extern template struct ::cign::gatk::FwdFlLauncher<T, L, V>;

#define CIGN_GAT_FL_INSTANTIATE(T) CIGN_GAT_FL_LIST_NARROW(CIGN_GAT_FL_INST_ONE, T)
#define CIGN_GAT_FLW_INSTANTIATE(T) CIGN_GAT_FL_LIST_WIDE(CIGN_GAT_FL_INST_ONE, T)
#define CIGN_GAT_FL_DECLARE(T) \
  CIGN_GAT_FL_LIST_NARROW(CIGN_GAT_FL_DECL_ONE, T) CIGN_GAT_FL_LIST_WIDE(CIGN_GAT_FL_DECL_ONE, T)
#define CIGN_GAT_FL_DECLARE_NARROW(T) CIGN_GAT_FL_LIST_NARROW(CIGN_GAT_FL_DECL_ONE, T)

}  // namespace gatk
}  // namespace cign
