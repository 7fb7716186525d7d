// Collapsed multi-head GAT (concat=False) kernels for gfx950: edge score, per
// destination edge softmax, edge dropout, weighted aggregation and the fused
// head-mean + bias + SiLU epilogue, forward and backward.
//
// Semantics follow the reference A3-v6 core (collapsed_gat_ext/
// collapsed_gat_cuda.cu:34-430; host glue :434-545): for destination row i,
// edge e = (i <- j) and head h,
//   raw_eh = attn_row[i,h] + attn_col[j,h],  sc = LeakyReLU(raw),
//   s_eh   = exp(sc - max_h) / sum_h (softmax over the in-edges of i),
//   w_eh   = s_eh * keep_eh / (1 - p)   (keep_eh = splitmix64 bit, p > 0),
//   pre_ic = (1/H) sum_h sum_e w_eh x[j,h,c] + bias_c,  out = SiLU(pre).
// edge_max / edge_sum [N,H] are saved for the backward; the mask [E,H] is in
// CSR edge order (written only when p > 0, like the reference).
//
// Design (own, MI355X-first). A lane owns one (edge, head) pair: the head
// count is padded to HP = 2^k so lane = el * HP + h and every reduction over
// the edges of a row is an xor-butterfly over lane bits >= log2(HP). Channels
// are handled in blocks of CP <= 32 consecutive values per lane (16-byte loads
// when the row layout allows). A wavefront takes at most 16 edges of a row
// (N = 16 / EPW tiles of EPW = 64 / HP edges per lane, N selected at run time
// from the row's degree), issuing every load of the row before consuming any
// (indices clamped to a valid edge and head, results masked): a row costs one
// memory round per level of indirection, with a small register footprint.
//
// The backward is two kernels (the reference uses five):
//   gat_bwd_rows (CSR, one pass): g_pre = g_y * SiLU'(pre); per edge
//     ge' = keep/(1-p) * <g_pre, x[j,h,:]>/H (stored), s, l' = LeakyReLU';
//     per row and head wsum = sum s ge', A = sum s ge' l', B = sum s l', so
//     grad_attn_row = sum_e s (ge' - wsum) l' = A - wsum * B and wsum is saved;
//   gat_bwd_cols (CSC): g_raw = s (ge' - wsum[i]) l' per edge, grad_attn_col =
//     sum g_raw (no atomics), grad_feat = sum_e w g_pre[i] / H, plus the
//     deterministic two-level grad_bias reduction in dedicated workgroups.
// Rows/columns with more than 16 edges use 64-edge segments of the schedule
// (schedule.h, built with light_max = 16, seg_edges = 64), one workgroup
// each, multi-segment rows merged by the last workgroup to finish.
#pragma once

#include <type_traits>

#include "common.h"
#include "schedule.h"

namespace cign {
namespace gatk {

constexpr int kTile = 64;
constexpr int kSegEdges = kWavesPerBlock * kTile;
constexpr int kMaxC = 256;  // channel limit (the reference's advertised range)
constexpr int kMaxH = 32;
constexpr float kNegBig = -1.0e38f;

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int ilog2c(int v) { return v <= 1 ? 0 : 1 + ilog2c(v / 2); }

// Softmax statistics merge: (m1, s1) <- (m1, s1) (+) (m2, s2).
__device__ __forceinline__ void ms_merge(float& m1, float& s1, float m2, float s2) {
  const float M = fmaxf(m1, m2);
  s1 = s1 * softmax_exp(m1 - M) + s2 * softmax_exp(m2 - M);
  m1 = M;
}

// Reduction of CP per-lane values over the lanes that share lane % HP
// (offsets HP .. 32), as a reduce-scatter: while more than one value is left
// each butterfly step keeps half of them. Afterwards lane l holds R values
// for channels chan_base(l) + r; lanes with writer(l) are one per
// (head, channel group).
template <int CP, int HP>
struct GroupReduce {
  static constexpr int LGH = ilog2c(HP);
  static constexpr int LGE = 6 - LGH;
  static constexpr int LGC = ilog2c(CP);
  static constexpr int K = LGC < LGE ? LGC : LGE;
  static constexpr int R = CP >> K;

  static __device__ __forceinline__ void run(float (&v)[CP], int lane) {
#pragma unroll
    for (int s = 0; s < LGE; ++s) {
      const int o = 32 >> s;
      if (s < K) {
        const int half = CP >> (s + 1);
        const bool up = (lane & o) != 0;
#pragma unroll
        for (int k = 0; k < half; ++k) {
          const float send = up ? v[k] : v[k + half];
          const float keep = up ? v[k + half] : v[k];
          v[k] = keep + shfl_xor(send, o);
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) v[r] += shfl_xor(v[r], o);
      }
    }
  }
  static __device__ __forceinline__ int chan_base(int lane) { return (lane >> (6 - K)) * R; }
  static __device__ __forceinline__ bool writer(int lane) {
    return ((lane >> LGH) & ((1 << (LGE - K)) - 1)) == 0;
  }
};

// Loads CP consecutive values starting at p (only the first nvalid are real);
// vec => p is 16-byte aligned and nvalid is a multiple of the vector width.
template <typename T, int CP>
__device__ __forceinline__ void load_run(const T* p, int nvalid, bool vec, float (&out)[CP]) {
  constexpr int VW = 16 / sizeof(T);
  if (CP >= VW && vec) {
#pragma unroll
    for (int q = 0; q < CP / VW; ++q) {
      float tmp[VW];
      if (q * VW < nvalid) {
        Chunk<T, VW>::load(p + q * VW, tmp);
      } else {
#pragma unroll
        for (int w = 0; w < VW; ++w) tmp[w] = 0.0f;
      }
#pragma unroll
      for (int w = 0; w < VW; ++w) out[q * VW + w] = tmp[w];
    }
  } else {
#pragma unroll
    for (int c = 0; c < CP; ++c) out[c] = c < nvalid ? to_f32(p[c]) : 0.0f;
  }
}

// Lane geometry of the (edge, head) layout.
template <int HP>
struct Lanes {
  static constexpr int LGH = ilog2c(HP);
  static constexpr int EPW = kWave / HP;
  int lane, h, el, hc;  // hc: head clamped to a valid head for loads
  bool hv;
  __device__ __forceinline__ explicit Lanes(int H) {
    lane = lane_id();
    h = lane & (HP - 1);
    el = lane >> LGH;
    hv = h < H;
    hc = hv ? h : H - 1;
  }
};

template <typename T>
struct GatFwdArgs {
  int n, H, C;
  // Edges of the whole graph: selects the large-graph kernel variants, so a
  // launch over one row shard computes each row as the whole-graph launch.
  int64_t graph_nnz;
  // Dropout hash index offset: H x the CSR id, in the whole graph, of the
  // launch's first edge (0 for a whole-graph launch). The mask is stored at
  // the launch's own edge ids.
  int64_t mask_base;
  float slope, p;
  uint64_t seed;
  bool vec;  // 16-byte loads of x rows are legal
  const float* attn_row;
  const float* attn_col;
  const int32_t* col;
  const T* x;
  const float* bias;
  GatOut<T>* out;
  float* pre;
  float* emax;
  float* esum;
  uint8_t* mask;
  float* partial;  // [n_seg, 2*H*C + 3H]
  int32_t* counters;
  // Optional (feature layout): per-row aggregates for the backward, null to
  // skip. agg [n, H*C] = sum_e s kw x[j_e], then [n, H*C] = sum_e s kw l'
  // x[j_e], then [n, H] = sum_e s l'.
  float* agg;
};

// Calls f(std::integral_constant<int, n>) for a wave-uniform n in [1, NMAX],
// so a row's tile count selects a fully unrolled, branch-free body.
template <int K, int NMAX, typename F>
__device__ __forceinline__ void dispatch_n(int n, F& f) {
  if constexpr (K <= NMAX) {
    if (n == K) {
      f(std::integral_constant<int, K>{});
      return;
    }
    dispatch_n<K + 1, NMAX>(n, f);
  }
}

// Schedule geometry of the GAT kernels: a wavefront handles at most
// kGatLight = 16 edges of a row (NTL = 16 / EPW tiles per lane, 1 for H <= 4),
// rows with more edges go to 64-edge segments (one 16-edge tile per wave).
constexpr int kGatLight = 16;
constexpr int kGatSeg = kWavesPerBlock * kGatLight;
template <int HP>
constexpr int kNTL = Lanes<HP>::EPW >= kGatLight ? 1 : kGatLight / Lanes<HP>::EPW;

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// The lane's N tiles of a wave's edges [eb, ee): indices, scores and (when it
// fits in registers) the first channel block of x, all loads issued before
// any result is consumed (indices clamped to a valid edge / head).
template <typename T, int HP, int CP, int N>
struct FwdWave {
  static constexpr bool kPrefetch = N * CP <= 32;
  int t[N], j[N];
  float sc[N];
  bool v[N];
  float x0[kPrefetch ? N : 1][CP];

  __device__ __forceinline__ void load(const GatFwdArgs<T>& a, const Lanes<HP>& L, int eb, int ee, float adst) {
    if (ee <= eb) {
      // No edges (wave-uniform): nothing is read; eb may equal nnz here.
#pragma unroll
      for (int k = 0; k < N; ++k) {
        t[k] = eb;
        v[k] = false;
        j[k] = 0;
        sc[k] = kNegBig;
        if constexpr (kPrefetch)
#pragma unroll
          for (int c = 0; c < CP; ++c) x0[k][c] = 0.0f;
      }
      return;
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
      t[k] = eb + L.el + k * Lanes<HP>::EPW;
      v[k] = L.hv && t[k] < ee;
      j[k] = a.col[t[k] < ee ? t[k] : eb];
    }
    if constexpr (kPrefetch) {
      const int nvalid = min(CP, a.C);
#pragma unroll
      for (int k = 0; k < N; ++k)
        load_run<T, CP>(a.x + (static_cast<int64_t>(j[k]) * a.H + L.hc) * a.C, nvalid, a.vec, x0[k]);
    }
#pragma unroll
    for (int k = 0; k < N; ++k) sc[k] = leaky(adst + a.attn_col[static_cast<int64_t>(j[k]) * a.H + L.hc], a.slope);
  }

  // Lane-local softmax statistics.
  __device__ __forceinline__ void stats(float& m, float& s) const {
    m = kNegBig;
#pragma unroll
    for (int k = 0; k < N; ++k) m = v[k] ? fmaxf(m, sc[k]) : m;
    s = 0.0f;
#pragma unroll
    for (int k = 0; k < N; ++k) s += v[k] ? softmax_exp(sc[k] - m) : 0.0f;
  }

  // Weight of one (edge, head): normalised softmax, or exp(sc - M) for a
  // segment partial, times keep / (1 - p); records the mask on block 0.
  __device__ __forceinline__ float weight(const GatFwdArgs<T>& a, int k, int h, float M, float S, bool normalise,
                                         bool write_mask) const {
    if (!v[k]) return 0.0f;
    bool keep = true;
    if (a.p > 0.0f) {
      const int64_t idx = static_cast<int64_t>(t[k]) * a.H + h;
      keep = gat_keep(a.seed, static_cast<uint64_t>(idx + a.mask_base), a.p);
      if (write_mask) a.mask[idx] = keep ? 1 : 0;
    }
    if (!keep || (normalise && !(S > 0.0f))) return 0.0f;
    float w = softmax_exp(sc[k] - M);
    if (normalise) w = w / S;
    if (a.p > 0.0f) w = w * (1.0f / (1.0f - a.p));
    return w;
  }

  // acc[c] = sum over the lane's edges of w * x[j, h, cb*CP + c].
  __device__ __forceinline__ void accumulate(const GatFwdArgs<T>& a, const Lanes<HP>& L, int cb, float M, float S,
                                             bool normalise, float (&acc)[CP]) const {
#pragma unroll
    for (int c = 0; c < CP; ++c) acc[c] = 0.0f;
    float xv[N][CP];
    if (kPrefetch && cb == 0) {
#pragma unroll
      for (int k = 0; k < N; ++k)
#pragma unroll
        for (int c = 0; c < CP; ++c) xv[k][c] = x0[kPrefetch ? k : 0][c];
    } else {
      const int nvalid = min(CP, a.C - cb * CP);
#pragma unroll
      for (int k = 0; k < N; ++k)
        load_run<T, CP>(a.x + (static_cast<int64_t>(j[k]) * a.H + L.hc) * a.C + cb * CP, nvalid, a.vec, xv[k]);
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
      const float w = weight(a, k, L.h, M, S, normalise, cb == 0);
#pragma unroll
      for (int c = 0; c < CP; ++c) acc[c] = fmaf(w, xv[k][c], acc[c]);
    }
  }
};

template <int HP>
__device__ __forceinline__ void ms_reduce_heads(float& m, float& s) {
  for (int o = HP; o < kWave; o <<= 1) {
    const float m2 = shfl_xor(m, o);
    const float s2 = shfl_xor(s, o);
    ms_merge(m, s, m2, s2);
  }
}

template <typename T>
__device__ __forceinline__ void fwd_emit(const GatFwdArgs<T>& a, int row, int c, float total) {
  const float pv = total / static_cast<float>(a.H) + a.bias[c];
  const int64_t idx = static_cast<int64_t>(row) * a.C + c;
  a.pre[idx] = pv;
  a.out[idx] = from_f32<T>(silu(pv));
}

template <typename T, int HP, int CP>
__global__ __launch_bounds__(kBlock) void gat_fwd_kernel(GatFwdArgs<T> a, Sched s) {
  using GR1 = GroupReduce<CP, 1>;
  using GRH = GroupReduce<CP, HP>;
  constexpr int EPW = Lanes<HP>::EPW;
  constexpr int NTL = kNTL<HP>;
  const Lanes<HP> L(a.H);
  const int wave = wave_id();
  const int ncb = (a.C + CP - 1) / CP;
  const int b = blockIdx.x;

  if (b >= s.n_seg) {
    const int li = (b - s.n_seg) * kWavesPerBlock + wave;
    if (li >= s.n_light) return;
    const int4 r = s.light[li];
    const float adst = a.attn_row[static_cast<int64_t>(r.x) * a.H + L.hc];
    const int nt = max(1, (r.z - r.y + EPW - 1) / EPW);
    auto body = [&](auto NC) {
      constexpr int N = decltype(NC)::value;
      FwdWave<T, HP, CP, N> w;
      w.load(a, L, r.y, r.z, adst);
      float m, sum;
      w.stats(m, sum);
      ms_reduce_heads<HP>(m, sum);
      if (L.el == 0 && L.hv) {
        a.emax[static_cast<int64_t>(r.x) * a.H + L.h] = m;
        a.esum[static_cast<int64_t>(r.x) * a.H + L.h] = sum;
      }
      for (int cb = 0; cb < ncb; ++cb) {
        float acc[CP];
        w.accumulate(a, L, cb, m, sum, true, acc);
        GR1::run(acc, L.lane);
        if (GR1::writer(L.lane)) {
          const int c0 = cb * CP + GR1::chan_base(L.lane);
#pragma unroll
          for (int q = 0; q < GR1::R; ++q)
            if (c0 + q < a.C) fwd_emit(a, r.x, c0 + q, acc[q]);
        }
      }
    };
    dispatch_n<1, NTL>(nt, body);
    return;
  }

  // Heavy-row segment: 4 waves, one kGatLight-edge tile each.
  __shared__ float sm_m[kWavesPerBlock][HP], sm_s[kWavesPerBlock][HP];
  __shared__ float red[kWavesPerBlock][HP * CP];
  __shared__ float fin_m[HP], fin_s[HP];
  __shared__ int flag;
  const int4 sg = s.seg[b];
  const int row = sg.x;
  const int2 hr = s.hrow[sg.w];
  const bool single = hr.y == 1;
  const int eb = min(sg.y + wave * kGatLight, sg.z);
  const int ee = min(sg.z, eb + kGatLight);
  const float adst = a.attn_row[static_cast<int64_t>(row) * a.H + L.hc];
  FwdWave<T, HP, CP, NTL> w;
  w.load(a, L, eb, ee, adst);
  float m, sum;
  w.stats(m, sum);
  ms_reduce_heads<HP>(m, sum);
  if (L.el == 0) {
    sm_m[wave][L.h] = m;
    sm_s[wave][L.h] = sum;
  }
  __syncthreads();
  float M = sm_m[0][L.h], S = sm_s[0][L.h];
#pragma unroll
  for (int q = 1; q < kWavesPerBlock; ++q) ms_merge(M, S, sm_m[q][L.h], sm_s[q][L.h]);

  const int HC = a.H * a.C;
  float* mine = a.partial + static_cast<int64_t>(b) * (HC + 2 * a.H);
  for (int cb = 0; cb < ncb; ++cb) {
    float acc[CP];
    w.accumulate(a, L, cb, M, S, single, acc);
    if (single) {
      GR1::run(acc, L.lane);
      if (GR1::writer(L.lane)) {
        const int c0 = GR1::chan_base(L.lane);
#pragma unroll
        for (int q = 0; q < GR1::R; ++q) red[wave][c0 + q] = acc[q];
      }
      __syncthreads();
      for (int c = threadIdx.x; c < CP; c += kBlock) {
        const int cc = cb * CP + c;
        if (cc < a.C) fwd_emit(a, row, cc, red[0][c] + red[1][c] + red[2][c] + red[3][c]);
      }
      __syncthreads();
    } else {
      GRH::run(acc, L.lane);
      if (GRH::writer(L.lane)) {
        const int c0 = GRH::chan_base(L.lane);
#pragma unroll
        for (int q = 0; q < GRH::R; ++q) red[wave][L.h * CP + c0 + q] = acc[q];
      }
      __syncthreads();
      for (int q = threadIdx.x; q < HP * CP; q += kBlock) {
        const int hh = q / CP, c = q % CP, cc = cb * CP + c;
        if (hh < a.H && cc < a.C) st_agent(mine + hh * a.C + cc, red[0][q] + red[1][q] + red[2][q] + red[3][q]);
      }
      __syncthreads();
    }
  }
  if (single) {
    if (wave == 0 && L.el == 0 && L.hv) {
      a.emax[static_cast<int64_t>(row) * a.H + L.h] = M;
      a.esum[static_cast<int64_t>(row) * a.H + L.h] = S;
    }
    return;
  }
  if (wave == 0 && L.el == 0 && L.hv) {
    st_agent(mine + HC + L.h, M);
    st_agent(mine + HC + a.H + L.h, S);
  }
  if (!arrive_last(a.counters + sg.w, hr.y, &flag)) return;
  // Last segment of this row: merge the per-segment (m, s, acc) in order.
  const int stride = HC + 2 * a.H;
  if (threadIdx.x < a.H) {
    const int hh = threadIdx.x;
    float MM = kNegBig, SS = 0.0f;
    for (int q = 0; q < hr.y; ++q) {
      const float* pq = a.partial + static_cast<int64_t>(hr.x + q) * stride;
      ms_merge(MM, SS, ld_agent(pq + HC + hh), ld_agent(pq + HC + a.H + hh));
    }
    fin_m[hh] = MM;
    fin_s[hh] = SS;
    a.emax[static_cast<int64_t>(row) * a.H + hh] = MM;
    a.esum[static_cast<int64_t>(row) * a.H + hh] = SS;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < a.C; c += kBlock) {
    float total = 0.0f;
    for (int hh = 0; hh < a.H; ++hh) {
      float acch = 0.0f;
      for (int q = 0; q < hr.y; ++q) {
        const float* pq = a.partial + static_cast<int64_t>(hr.x + q) * stride;
        acch += ld_agent(pq + hh * a.C + c) * softmax_exp(ld_agent(pq + HC + hh) - fin_m[hh]);
      }
      if (fin_s[hh] > 0.0f) total += acch / fin_s[hh];
    }
    fwd_emit(a, row, c, total);
  }
}


// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
template <typename T>
struct GatBwdArgs {
  int n, nnz, H, C;
  int64_t graph_nnz;  // edges of the whole graph (variant selection, as GatFwdArgs)
  // grad_bias sums grad_pre rows [bias_lo, bias_lo + bias_n) (0, n for a
  // whole-graph launch; a shard's own rows otherwise)
  int bias_lo, bias_n;
  float slope, p, inv_h;
  bool vec_x;   // 16-byte loads of x rows are legal
  bool vec_gp;  // 16-byte loads of grad_pre rows are legal
  const int32_t* col;
  const int32_t* rowind;
  const int32_t* perm;
  const float* emax;
  const float* esum;
  const uint8_t* mask;
  const T* x;
  const float* attn_row;
  const float* attn_col;
  const float* pre;
  const GatOut<T>* grad_y;
  const float* agg;  // per-row aggregates written by the forward, or null
  // workspace
  float* grad_pre;   // [n, gp_stride]: g_pre in the row's first C floats
  int gp_stride;     // floats per grad_pre row: C (pair layout) or C + 4H
  float* gscore;     // [nnz, H]: ge' = keep/(1-p) * <g_pre, x>/H
  float* wsum;       // [n, H]: sum_e s ge'
  // Feature layout: {attn_row, edge_max, 1/edge_sum, wsum} per head, stored
  // after the row's g_pre (rowstat = grad_pre + C, rs_stride = gp_stride / 4
  // float4s per row), so a column's entry gathers one contiguous record.
  float4* rowstat;
  int rs_stride;
  float* bias_part;  // [rows_blocks, C]
  float* bias_l2;    // [n_l2, C]
  float* part_row;   // [n_seg_rows, 3H]
  float* part_col;   // [n_seg_cols, H*C + H]
  int32_t* row_counters;
  int32_t* col_counters;  // [n_hrow_cols + 1]; last slot = bias counter
  int rows_blocks;
  int n_l2;
  // outputs
  GatOut<T>* grad_feat;
  float* grad_attn_row;
  float* grad_attn_col;
  float* grad_bias;
};

// g_pre of one row into LDS (and, when `publish`, into the grad_pre
// workspace); LDS entries [C, padded) are zeroed so whole channel blocks can
// be read.
template <typename T>
__device__ __forceinline__ void bwd_grad_pre(const GatBwdArgs<T>& a, int row, int first, int step, int padded,
                                             float* gp, bool publish) {
  for (int c = first; c < padded; c += step) {
    if (c >= a.C) {
      gp[c] = 0.0f;
      continue;
    }
    const int64_t idx = static_cast<int64_t>(row) * a.C + c;
    const float g = to_f32(a.grad_y[idx]) * silu_grad(a.pre[idx]);
    gp[c] = g;
    if (publish) a.grad_pre[static_cast<int64_t>(row) * a.gp_stride + c] = g;
  }
}

// One pass over the lane's N tiles of [eb, ee): stores ge' and accumulates
// (wsum, A, B) for the lane's head.
template <typename T, int HP, int CP, int N>
__device__ __forceinline__ void bwd_row_wave(const GatBwdArgs<T>& a, const Lanes<HP>& L, int eb, int ee, float adst,
                                             float M, float S, const float* gp, float& wsum, float& A, float& B) {
  wsum = A = B = 0.0f;
  if (ee <= eb) return;  // no edges (wave-uniform); eb may equal nnz here
  const int ncb = (a.C + CP - 1) / CP;
  int t[N], j[N];
  bool v[N];
#pragma unroll
  for (int k = 0; k < N; ++k) {
    t[k] = eb + L.el + k * Lanes<HP>::EPW;
    v[k] = L.hv && t[k] < ee;
    j[k] = a.col[t[k] < ee ? t[k] : eb];
  }
  float raw[N], dot[N];
  bool keep[N];
#pragma unroll
  for (int k = 0; k < N; ++k) {
    raw[k] = adst + a.attn_col[static_cast<int64_t>(j[k]) * a.H + L.hc];
    keep[k] = a.p > 0.0f ? a.mask[static_cast<int64_t>(v[k] ? t[k] : eb) * a.H + L.hc] != 0 : true;
    dot[k] = 0.0f;
  }
  for (int cb = 0; cb < ncb; ++cb) {
    const int nvalid = min(CP, a.C - cb * CP);
    float xv[N][CP];
#pragma unroll
    for (int k = 0; k < N; ++k)
      load_run<T, CP>(a.x + (static_cast<int64_t>(j[k]) * a.H + L.hc) * a.C + cb * CP, nvalid, a.vec_x, xv[k]);
#pragma unroll
    for (int c = 0; c < CP; ++c) {
      const float g = gp[cb * CP + c];
#pragma unroll
      for (int k = 0; k < N; ++k) dot[k] = fmaf(g, xv[k][c], dot[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < N; ++k) {
    float ge = dot[k] * a.inv_h;
    if (a.p > 0.0f) ge = (keep[k] ? ge : 0.0f) * (1.0f / (1.0f - a.p));
    const float soft = S > 0.0f ? softmax_exp(leaky(raw[k], a.slope) - M) / S : 0.0f;
    const float lp = raw[k] < 0.0f ? a.slope : 1.0f;
    if (v[k]) {
      a.gscore[static_cast<int64_t>(t[k]) * a.H + L.h] = ge;
      const float sg = soft * ge;
      wsum += sg;
      A += sg * lp;
      B += soft * lp;
    }
  }
}

template <typename T, int HP, int CP>
__global__ __launch_bounds__(kBlock) void gat_bwd_rows_kernel(GatBwdArgs<T> a, Sched s) {
  constexpr int EPW = Lanes<HP>::EPW;
  constexpr int NTL = kNTL<HP>;
  const Lanes<HP> L(a.H);
  const int wave = wave_id();
  const int b = blockIdx.x;
  const int padded = ((a.C + CP - 1) / CP) * CP;
  __shared__ float gp[kWavesPerBlock][kMaxC];
  __shared__ float red[kWavesPerBlock][3][HP];
  __shared__ int flag;

  if (b >= s.n_seg) {
    const int li = (b - s.n_seg) * kWavesPerBlock + wave;
    const bool has = li < s.n_light;
    const int4 r = has ? s.light[li] : make_int4(0, 0, 0, 0);
    if (has) {
      const int64_t rh = static_cast<int64_t>(r.x) * a.H + L.hc;
      const float adst = a.attn_row[rh];
      const float M = a.emax[rh];
      const float S = a.esum[rh];
      bwd_grad_pre(a, r.x, L.lane, kWave, padded, gp[wave], true);
      wave_sync();
      float wsum = 0.0f, A = 0.0f, B = 0.0f;
      const int nt = max(1, (r.z - r.y + EPW - 1) / EPW);
      auto body = [&](auto NC) {
        bwd_row_wave<T, HP, CP, decltype(NC)::value>(a, L, r.y, r.z, adst, M, S, gp[wave], wsum, A, B);
      };
      dispatch_n<1, NTL>(nt, body);
      {
        float t[1][3] = {{wsum, A, B}};
        sum_across_n(t, HP);
        wsum = t[0][0];
        A = t[0][1];
        B = t[0][2];
      }
      if (L.el == 0 && L.hv) {
        a.wsum[rh] = wsum;
        a.grad_attn_row[rh] = A - wsum * B;
      }
    } else {
      for (int c = L.lane; c < padded; c += kWave) gp[wave][c] = 0.0f;
    }
    __syncthreads();
    // Per-block bias partial: sum of this block's rows of g_pre.
    for (int c = threadIdx.x; c < a.C; c += kBlock)
      a.bias_part[static_cast<int64_t>(b) * a.C + c] = gp[0][c] + gp[1][c] + gp[2][c] + gp[3][c];
    return;
  }

  // Heavy-row segment.
  const int4 sg = s.seg[b];
  const int row = sg.x;
  const int2 hr = s.hrow[sg.w];
  const bool first_seg = (b == hr.x);
  bwd_grad_pre(a, row, threadIdx.x, kBlock, padded, gp[0], first_seg);
  __syncthreads();
  for (int c = threadIdx.x; c < a.C; c += kBlock)
    a.bias_part[static_cast<int64_t>(b) * a.C + c] = first_seg ? gp[0][c] : 0.0f;
  const int eb = min(sg.y + wave * kGatLight, sg.z);
  const int ee = min(sg.z, eb + kGatLight);
  const int64_t rh = static_cast<int64_t>(row) * a.H + L.hc;
  float wsum, A, B;
  bwd_row_wave<T, HP, CP, NTL>(a, L, eb, ee, a.attn_row[rh], a.emax[rh], a.esum[rh], gp[0], wsum, A, B);
  {
    float t[1][3] = {{wsum, A, B}};
    sum_across_n(t, HP);
    wsum = t[0][0];
    A = t[0][1];
    B = t[0][2];
  }
  if (L.el == 0) {
    red[wave][0][L.h] = wsum;
    red[wave][1][L.h] = A;
    red[wave][2][L.h] = B;
  }
  __syncthreads();
  if (threadIdx.x < 3 * HP) {
    const int k = threadIdx.x / HP, hh = threadIdx.x % HP;
    red[0][k][hh] = red[0][k][hh] + red[1][k][hh] + red[2][k][hh] + red[3][k][hh];
  }
  __syncthreads();
  if (hr.y == 1) {
    if (threadIdx.x < a.H) {
      const float w = red[0][0][threadIdx.x];
      a.wsum[static_cast<int64_t>(row) * a.H + threadIdx.x] = w;
      a.grad_attn_row[static_cast<int64_t>(row) * a.H + threadIdx.x] = red[0][1][threadIdx.x] - w * red[0][2][threadIdx.x];
    }
    return;
  }
  float* mine = a.part_row + static_cast<int64_t>(b) * 3 * a.H;
  if (threadIdx.x < 3 * a.H) st_agent(mine + threadIdx.x, red[0][threadIdx.x / a.H][threadIdx.x % a.H]);
  if (!arrive_last(a.row_counters + sg.w, hr.y, &flag)) return;
  if (threadIdx.x < a.H) {
    float w = 0.0f, AA = 0.0f, BB = 0.0f;
    for (int q = 0; q < hr.y; ++q) {
      const float* pq = a.part_row + static_cast<int64_t>(hr.x + q) * 3 * a.H;
      w += ld_agent(pq + threadIdx.x);
      AA += ld_agent(pq + a.H + threadIdx.x);
      BB += ld_agent(pq + 2 * a.H + threadIdx.x);
    }
    a.wsum[static_cast<int64_t>(row) * a.H + threadIdx.x] = w;
    a.grad_attn_row[static_cast<int64_t>(row) * a.H + threadIdx.x] = AA - w * BB;
  }
}

// The lane's N tiles of a CSC range [cb0, ce): per-edge weights w, source
// rows i, and the lane's sum of g_raw = s (ge' - wsum[i]) LeakyReLU'.
template <typename T, int HP, int N>
__device__ __forceinline__ float bwd_col_wave(const GatBwdArgs<T>& a, const Lanes<HP>& L, int cb0, int ce,
                                              float asrc, int (&i)[N], float (&w)[N]) {
  if (ce <= cb0) {
    // No edges (wave-uniform): nothing is read; cb0 may equal nnz here.
#pragma unroll
    for (int k = 0; k < N; ++k) {
      i[k] = 0;
      w[k] = 0.0f;
    }
    return 0.0f;
  }
  int e[N];
  bool v[N];
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int t = cb0 + L.el + k * Lanes<HP>::EPW;
    v[k] = L.hv && t < ce;
    const int tc = t < ce ? t : cb0;
    i[k] = a.rowind[tc];
    e[k] = a.perm[tc];
  }
  float gsum = 0.0f;
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int64_t ih = static_cast<int64_t>(i[k]) * a.H + L.hc;
    const int64_t eh = static_cast<int64_t>(e[k]) * a.H + L.hc;
    const float raw = a.attn_row[ih] + asrc;
    const float S = a.esum[ih];
    const float M = a.emax[ih];
    const float ws = a.wsum[ih];
    const float ge = a.gscore[eh];
    const bool keep = a.p > 0.0f ? a.mask[eh] != 0 : true;
    const float soft = S > 0.0f ? softmax_exp(leaky(raw, a.slope) - M) / S : 0.0f;
    float ww = 0.0f;
    if (v[k] && keep) {
      ww = soft;
      if (a.p > 0.0f) ww = ww * (1.0f / (1.0f - a.p));
    }
    w[k] = ww;
    float g = soft * (ge - ws);
    if (raw < 0.0f) g *= a.slope;
    gsum += v[k] ? g : 0.0f;
  }
  return gsum;
}

template <typename T, int CP, int N>
__device__ __forceinline__ void bwd_col_gather(const GatBwdArgs<T>& a, int cb, const int (&i)[N], const float (&w)[N],
                                               float (&acc)[CP]) {
  const int nvalid = min(CP, a.C - cb * CP);
  float gv[N][CP];
#pragma unroll
  for (int k = 0; k < N; ++k)
    load_run<float, CP>(a.grad_pre + static_cast<int64_t>(i[k]) * a.gp_stride + cb * CP, nvalid, a.vec_gp, gv[k]);
#pragma unroll
  for (int c = 0; c < CP; ++c) acc[c] = 0.0f;
#pragma unroll
  for (int k = 0; k < N; ++k)
#pragma unroll
    for (int c = 0; c < CP; ++c) acc[c] = fmaf(w[k], gv[k][c], acc[c]);
}

template <typename T>
__device__ __forceinline__ void store_gx(const GatBwdArgs<T>& a, int j, int h, int c, float v) {
  a.grad_feat[(static_cast<int64_t>(j) * a.H + h) * a.C + c] = from_f32<T>(v * a.inv_h);
}

// grad_bias = sum over kernel-1 blocks of their partials: level 1 in each
// bias workgroup (64 partials), level 2 in the last one to finish. Partial
// rows are summed by parallel thread groups, then combined through LDS.
template <typename T>
__device__ __forceinline__ void bias_reduce(const GatBwdArgs<T>& a, int q, int* counter, int* flag) {
  __shared__ float red[kBlock];
  const int C = a.C;
  const int rows_per = kBlock / C;  // C <= kMaxC = kBlock
  const int tid = threadIdx.x;
  const int c = tid % C;
  const int r0 = tid / C;
  auto reduce = [&](const float* src, int lo, int hi, float* dst) {
    float t = 0.0f;
    if (r0 < rows_per)
      for (int r = lo + r0; r < hi; r += rows_per) t += ld_agent(src + static_cast<int64_t>(r) * C + c);
    red[tid] = r0 < rows_per ? t : 0.0f;
    __syncthreads();
    if (tid < C) {
      float u = 0.0f;
      for (int k = 0; k < rows_per; ++k) u += red[k * C + tid];
      st_agent(dst + tid, u);
    }
    __syncthreads();
  };
  const int lo = q * 64, hi = min(a.rows_blocks, lo + 64);
  reduce(a.bias_part, lo, hi, a.bias_l2 + static_cast<int64_t>(q) * C);
  if (!arrive_last(counter, a.n_l2, flag)) return;
  reduce(a.bias_l2, 0, a.n_l2, a.grad_bias);
}

// grad_bias = sum_n grad_pre[n, :] over rows [bias_lo, bias_lo + bias_n) in
// two deterministic levels: workgroup q of a.n_l2 sums rows [q*R, q*R + R) of
// that range (R = ceil(bias_n / n_l2)) into bias_l2[q];
// the last one to finish sums the n_l2 partials in order. Threads own a
// (row, 4-channel chunk) pair and read float4 (C % 4 == 0, rows 16-byte
// aligned; grad_pre rows gp_stride floats apart), 256 / (C/4) rows per step.
template <typename T>
__device__ __forceinline__ void bias_from_grad_pre(const GatBwdArgs<T>& a, int q, int* counter, int* flag) {
  __shared__ float4 red[kBlock];
  const int C = a.C;
  const int c4n = C / 4;
  const int rpi = kBlock / c4n;
  const int tid = threadIdx.x;
  const int c4 = tid % c4n;
  const int r0 = tid / c4n;
  // agent: src was written in this launch (the second level reads the
  // first level's partials through ld_agent)
  auto reduce = [&](const float* src, int stride, int lo, int hi, float* dst, bool agent) {
    float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
    for (int r = lo + r0; r < hi; r += rpi) {
      const float* p = src + static_cast<int64_t>(r) * stride + c4 * 4;
      const float4 v = agent ? make_float4(ld_agent(p), ld_agent(p + 1), ld_agent(p + 2), ld_agent(p + 3))
                             : *reinterpret_cast<const float4*>(p);
      t.x += v.x;
      t.y += v.y;
      t.z += v.z;
      t.w += v.w;
    }
    red[tid] = t;
    __syncthreads();
    // the rpi row slots in a pairwise tree (fixed order; a serial sum by the
    // c4n chunk threads took 64 dependent LDS reads at C = 16, and the bias
    // workgroups were the c2 columns kernel's last 7 us)
    for (int h = 1; h < rpi; h <<= 1) {
      if (r0 < rpi && (r0 & (2 * h - 1)) == 0 && r0 + h < rpi) {
        const float4 v = red[tid + h * c4n];
        float4 u = red[tid];
        u.x += v.x;
        u.y += v.y;
        u.z += v.z;
        u.w += v.w;
        red[tid] = u;
      }
      __syncthreads();
    }
    if (tid < c4n) {
      const float4 u = red[tid];
      st_agent(dst + tid * 4, u.x);
      st_agent(dst + tid * 4 + 1, u.y);
      st_agent(dst + tid * 4 + 2, u.z);
      st_agent(dst + tid * 4 + 3, u.w);
    }
    __syncthreads();
  };
  const int R = (a.bias_n + a.n_l2 - 1) / a.n_l2;
  const int lo = min(a.bias_n, q * R), hi = min(a.bias_n, lo + R);
  reduce(a.grad_pre + static_cast<int64_t>(a.bias_lo) * a.gp_stride, a.gp_stride, lo, hi,
         a.bias_l2 + static_cast<int64_t>(q) * C, false);
  if (!arrive_last(counter, a.n_l2, flag)) return;
  reduce(a.bias_l2, C, 0, a.n_l2, a.grad_bias, true);
}

template <typename T, int HP, int CP>
__global__ __launch_bounds__(kBlock) void gat_bwd_cols_kernel(GatBwdArgs<T> a, Sched s) {
  using GR = GroupReduce<CP, HP>;
  constexpr int EPW = Lanes<HP>::EPW;
  constexpr int NTL = kNTL<HP>;
  const Lanes<HP> L(a.H);
  const int wave = wave_id();
  const int ncb = (a.C + CP - 1) / CP;
  __shared__ float red[kWavesPerBlock][HP * CP];
  __shared__ float gred[kWavesPerBlock][HP];
  __shared__ int flag;

  // the grad_bias workgroups first (their sums overlap the columns)
  if (static_cast<int>(blockIdx.x) < a.n_l2) {
    bias_reduce(a, blockIdx.x, a.col_counters + s.n_hrow, &flag);
    return;
  }
  const int b = blockIdx.x - a.n_l2;

  if (b >= s.n_seg) {
    const int li = (b - s.n_seg) * kWavesPerBlock + wave;
    if (li >= s.n_light) return;
    const int4 r = s.light[li];
    const int j = r.x;
    const int64_t jh = static_cast<int64_t>(j) * a.H + L.hc;
    const float asrc = a.attn_col[jh];
    float gsrc = 0.0f;
    const int nt = max(1, (r.z - r.y + EPW - 1) / EPW);
    auto body = [&](auto NC) {
      constexpr int N = decltype(NC)::value;
      int i[N];
      float w[N];
      gsrc = bwd_col_wave<T, HP, N>(a, L, r.y, r.z, asrc, i, w);
      for (int cb = 0; cb < ncb; ++cb) {
        float acc[CP];
        bwd_col_gather<T, CP, N>(a, cb, i, w, acc);
        GR::run(acc, L.lane);
        if (GR::writer(L.lane) && L.hv) {
          const int c0 = cb * CP + GR::chan_base(L.lane);
#pragma unroll
          for (int q = 0; q < GR::R; ++q)
            if (c0 + q < a.C) store_gx(a, j, L.h, c0 + q, acc[q]);
        }
      }
    };
    dispatch_n<1, NTL>(nt, body);
    gsrc = sum_across(gsrc, HP);
    if (L.el == 0 && L.hv) a.grad_attn_col[jh] = gsrc;
    return;
  }

  // Heavy column segment.
  const int4 sg = s.seg[b];
  const int j = sg.x;
  const int2 hr = s.hrow[sg.w];
  const bool single = hr.y == 1;
  const int t0 = min(sg.y + wave * kGatLight, sg.z);
  const int te = min(sg.z, t0 + kGatLight);
  const float asrc = a.attn_col[static_cast<int64_t>(j) * a.H + L.hc];
  const int HC = a.H * a.C;
  float* mine = a.part_col + static_cast<int64_t>(b) * (HC + a.H);
  int i[NTL];
  float w[NTL];
  float gsrc = bwd_col_wave<T, HP, NTL>(a, L, t0, te, asrc, i, w);
  for (int cb = 0; cb < ncb; ++cb) {
    float acc[CP];
    bwd_col_gather<T, CP, NTL>(a, cb, i, w, acc);
    GR::run(acc, L.lane);
    if (GR::writer(L.lane)) {
      const int c0 = GR::chan_base(L.lane);
#pragma unroll
      for (int q = 0; q < GR::R; ++q) red[wave][L.h * CP + c0 + q] = acc[q];
    }
    __syncthreads();
    for (int q = threadIdx.x; q < HP * CP; q += kBlock) {
      const int hh = q / CP, c = q % CP, cc = cb * CP + c;
      if (hh < a.H && cc < a.C) {
        const float v = red[0][q] + red[1][q] + red[2][q] + red[3][q];
        if (single) store_gx(a, j, hh, cc, v);
        else st_agent(mine + hh * a.C + cc, v);
      }
    }
    __syncthreads();
  }
  gsrc = sum_across(gsrc, HP);
  if (L.el == 0) gred[wave][L.h] = gsrc;
  __syncthreads();
  if (threadIdx.x < a.H) {
    const int hh = threadIdx.x;
    const float v = gred[0][hh] + gred[1][hh] + gred[2][hh] + gred[3][hh];
    if (single) a.grad_attn_col[static_cast<int64_t>(j) * a.H + hh] = v;
    else st_agent(mine + HC + hh, v);
  }
  if (single) return;
  if (!arrive_last(a.col_counters + sg.w, hr.y, &flag)) return;
  const int stride = HC + a.H;
  for (int q = threadIdx.x; q < HC + a.H; q += kBlock) {
    float t = 0.0f;
    for (int z = 0; z < hr.y; ++z) t += ld_agent(a.part_col + static_cast<int64_t>(hr.x + z) * stride + q);
    if (q < HC) store_gx(a, j, q / a.C, q % a.C, t);
    else a.grad_attn_col[static_cast<int64_t>(j) * a.H + (q - HC)] = t;
  }
}


// ---------------------------------------------------------------------------
// Launchers (explicitly instantiated in gat_inst_*.hip).
// ---------------------------------------------------------------------------
template <typename T, int HP, int CP>
struct FwdLauncher {
  static int run(hipStream_t st, const GatFwdArgs<T>& a, const Sched& s);
};

// Out of class, so that the extern template declarations of the
// translation units that only call a launcher also suppress its kernels.
template <typename T, int HP, int CP>
int FwdLauncher<T, HP, CP>::run(hipStream_t st, const GatFwdArgs<T>& a, const Sched& s) {
  const int blocks = sched_blocks(s);
  if (blocks > 0)
    hipLaunchKernelGGL((gat_fwd_kernel<T, HP, CP>), dim3(blocks), dim3(kBlock), 0, st, a, s);
  return check_launch("cign_gat_fwd");
}

template <typename T, int HP, int CP>
struct BwdLauncher {
  static int run(hipStream_t st, const GatBwdArgs<T>& a, const Sched& rs, const Sched& cs);
};

// Out of class, so that the extern template declarations of the
// translation units that only call a launcher also suppress its kernels.
template <typename T, int HP, int CP>
int BwdLauncher<T, HP, CP>::run(hipStream_t st, const GatBwdArgs<T>& a, const Sched& rs, const Sched& cs) {
  const int rb = sched_blocks(rs);
  if (rb > 0) {
    hipLaunchKernelGGL((gat_bwd_rows_kernel<T, HP, CP>), dim3(rb), dim3(kBlock), 0, st, a, rs);
    const int rc = check_launch("cign_gat_bwd (rows)");
    if (rc) return rc;
  }
  const int cb = sched_blocks(cs) + a.n_l2;
  if (cb > 0) hipLaunchKernelGGL((gat_bwd_cols_kernel<T, HP, CP>), dim3(cb), dim3(kBlock), 0, st, a, cs);
  return check_launch("cign_gat_bwd (cols)");
}

#define CIGN_GAT_INSTANTIATE(T, HP)                        \
  template struct ::cign::gatk::FwdLauncher<T, HP, 8>;     \
  template struct ::cign::gatk::FwdLauncher<T, HP, 16>;    \
  template struct ::cign::gatk::FwdLauncher<T, HP, 32>;    \
  template struct ::cign::gatk::BwdLauncher<T, HP, 8>;     \
  template struct ::cign::gatk::BwdLauncher<T, HP, 16>;    \
  template struct ::cign::gatk::BwdLauncher<T, HP, 32>;

#define CIGN_GAT_DECLARE(T, HP)                                   \
  extern template struct ::cign::gatk::FwdLauncher<T, HP, 8>;     \
  extern template struct ::cign::gatk::FwdLauncher<T, HP, 16>;    \
  extern template struct ::cign::gatk::FwdLauncher<T, HP, 32>;    \
  extern template struct ::cign::gatk::BwdLauncher<T, HP, 8>;     \
  extern template struct ::cign::gatk::BwdLauncher<T, HP, 16>;    \
  extern template struct ::cign::gatk::BwdLauncher<T, HP, 32>;

}  // namespace gatk
}  // namespace cign
