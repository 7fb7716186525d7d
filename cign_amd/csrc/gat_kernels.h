// Collapsed multi-head GAT (concat=False) for gfx950: edge score, per
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
// edge_max / edge_sum [N,H] are saved for the backward, and the mask [E,H]
// is in CSR edge order (written only when p > 0, like the reference).
//
// Design (own, MI355X-first): a lane owns one (edge, head) pair; the head
// count is padded to HP = 2^k so lane = el * HP + h and every reduction over
// edges is an xor-butterfly over lane bits >= log2(HP). Channels are handled
// in blocks of CP <= 32 consecutive values per lane (16-byte loads when the
// row layout allows). The backward is two kernels instead of five:
//   gat_bwd_rows (CSR): g_pre = g_y * SiLU'(pre), per-edge g_w = <g_pre, x>/H,
//     softmax + LeakyReLU backward, grad_attn_row; g_raw kept for kernel 2.
//   gat_bwd_cols (CSC): grad_feat, grad_attn_col (no atomics), plus the
//     deterministic two-level grad_bias reduction in dedicated workgroups.
// Heavy rows/columns use the segmented schedule of schedule.h.
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
  s1 = s1 * expf(m1 - M) + s2 * expf(m2 - M);
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

template <typename T>
struct GatFwdArgs {
  int n, H, C;
  float slope, p, inv_keep;
  uint64_t seed;
  bool vec;  // 16-byte loads of x rows are legal
  const float* attn_row;
  const float* attn_col;
  const int32_t* rowptr;
  const int32_t* col;
  const T* x;
  const float* bias;
  T* out;
  float* pre;
  float* emax;
  float* esum;
  uint8_t* mask;
  float* partial;  // [n_seg, H*C + 2H]
  int32_t* counters;
};

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// One 64-edge tile for one wave: scores into registers, local (m, s) per head.
template <typename T, int HP>
__device__ __forceinline__ void fwd_scores(const GatFwdArgs<T>& a, int row, int eb, int ee, float adst, int h,
                                           int el, bool hv, int (&jR)[HP], float (&scR)[HP], float& m,
                                           float& s) {
  constexpr int EPW = kWave / HP;
  m = kNegBig;
  s = 0.0f;
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    const int t = eb + el + k * EPW;
    jR[k] = 0;
    scR[k] = kNegBig;
    if (hv && t < ee) {
      const int j = a.col[t];
      jR[k] = j;
      scR[k] = leaky(adst + a.attn_col[static_cast<int64_t>(j) * a.H + h], a.slope);
      m = fmaxf(m, scR[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    const int t = eb + el + k * EPW;
    if (hv && t < ee) s += expf(scR[k] - m);
  }
}

template <int HP>
__device__ __forceinline__ void ms_reduce_heads(float& m, float& s) {
  for (int o = HP; o < kWave; o <<= 1) {
    const float m2 = shfl_xor(m, o);
    const float s2 = shfl_xor(s, o);
    ms_merge(m, s, m2, s2);
  }
}

// Edge weights of one tile given the row's (M, S) per head; applies and (on
// the first channel block) records the dropout mask.
template <typename T, int HP>
__device__ __forceinline__ void fwd_weights(const GatFwdArgs<T>& a, int eb, int ee, int h, int el, bool hv,
                                            const float (&scR)[HP], float M, float S, bool normalise,
                                            bool write_mask, float (&wR)[HP]) {
  constexpr int EPW = kWave / HP;
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    const int t = eb + el + k * EPW;
    float w = 0.0f;
    if (hv && t < ee) {
      bool keep = true;
      if (a.p > 0.0f) {
        const int64_t idx = static_cast<int64_t>(t) * a.H + h;
        keep = gat_keep(a.seed, static_cast<uint64_t>(idx), a.p);
        if (write_mask) a.mask[idx] = keep ? 1 : 0;
      }
      if (keep && (!normalise || S > 0.0f)) {
        w = expf(scR[k] - M);
        if (normalise) w = w / S;
        if (a.p > 0.0f) w = w / (1.0f - a.p);
      }
    }
    wR[k] = w;
  }
}

template <typename T, int HP, int CP>
__device__ __forceinline__ void fwd_gather(const GatFwdArgs<T>& a, int cb, int h, bool hv, const int (&jR)[HP],
                                           const float (&wR)[HP], float (&acc)[CP]) {
#pragma unroll
  for (int c = 0; c < CP; ++c) acc[c] = 0.0f;
  if (!hv) return;
  const int nvalid = min(CP, a.C - cb * CP);
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    if (wR[k] != 0.0f) {
      float xv[CP];
      const T* p = a.x + (static_cast<int64_t>(jR[k]) * a.H + h) * a.C + cb * CP;
      load_run<T, CP>(p, nvalid, a.vec, xv);
#pragma unroll
      for (int c = 0; c < CP; ++c) acc[c] = fmaf(wR[k], xv[c], acc[c]);
    }
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
  constexpr int LGH = ilog2c(HP);
  const int lane = lane_id();
  const int wave = wave_id();
  const int h = lane & (HP - 1);
  const int el = lane >> LGH;
  const bool hv = h < a.H;
  const int ncb = (a.C + CP - 1) / CP;
  const int b = blockIdx.x;

  int jR[HP];
  float scR[HP], wR[HP], acc[CP];

  if (b >= s.n_seg) {
    const int li = (b - s.n_seg) * kWavesPerBlock + wave;
    if (li >= s.n_light) return;
    const int row = s.light[li];
    const int eb = a.rowptr[row], ee = a.rowptr[row + 1];
    const float adst = hv ? a.attn_row[static_cast<int64_t>(row) * a.H + h] : 0.0f;
    float m, sum;
    fwd_scores<T, HP>(a, row, eb, ee, adst, h, el, hv, jR, scR, m, sum);
    ms_reduce_heads<HP>(m, sum);
    if (el == 0 && hv) {
      a.emax[static_cast<int64_t>(row) * a.H + h] = m;
      a.esum[static_cast<int64_t>(row) * a.H + h] = sum;
    }
    for (int cb = 0; cb < ncb; ++cb) {
      fwd_weights<T, HP>(a, eb, ee, h, el, hv, scR, m, sum, true, cb == 0, wR);
      fwd_gather<T, HP, CP>(a, cb, h, hv, jR, wR, acc);
      GroupReduce<CP, 1>::run(acc, lane);
      if (GroupReduce<CP, 1>::writer(lane)) {
        const int c0 = cb * CP + GroupReduce<CP, 1>::chan_base(lane);
#pragma unroll
        for (int r = 0; r < GroupReduce<CP, 1>::R; ++r)
          if (c0 + r < a.C) fwd_emit(a, row, c0 + r, acc[r]);
      }
    }
    return;
  }

  // Heavy-row segment: 4 waves, one 64-edge tile each.
  __shared__ float sm_m[kWavesPerBlock][HP], sm_s[kWavesPerBlock][HP];
  __shared__ float red[kWavesPerBlock][HP * CP];
  __shared__ float fin_m[HP], fin_s[HP];
  __shared__ int flag;
  const int4 sg = s.seg[b];
  const int row = sg.x;
  const int2 hr = s.hrow[sg.w];
  const bool single = hr.y == 1;
  const int eb = sg.y + wave * kTile;
  const int ee = min(sg.z, eb + kTile);
  const float adst = hv ? a.attn_row[static_cast<int64_t>(row) * a.H + h] : 0.0f;
  float m, sum;
  fwd_scores<T, HP>(a, row, eb, ee, adst, h, el, hv, jR, scR, m, sum);
  ms_reduce_heads<HP>(m, sum);
  if (el == 0) {
    sm_m[wave][h] = m;
    sm_s[wave][h] = sum;
  }
  __syncthreads();
  float M = sm_m[0][h], S = sm_s[0][h];
#pragma unroll
  for (int w = 1; w < kWavesPerBlock; ++w) ms_merge(M, S, sm_m[w][h], sm_s[w][h]);

  const int HC = a.H * a.C;
  float* mine = a.partial + static_cast<int64_t>(b) * (HC + 2 * a.H);
  for (int cb = 0; cb < ncb; ++cb) {
    fwd_weights<T, HP>(a, eb, ee, h, el, hv, scR, M, S, single, cb == 0, wR);
    fwd_gather<T, HP, CP>(a, cb, h, hv, jR, wR, acc);
    if (single) {
      GroupReduce<CP, 1>::run(acc, lane);
      if (GroupReduce<CP, 1>::writer(lane)) {
        const int c0 = GroupReduce<CP, 1>::chan_base(lane);
#pragma unroll
        for (int r = 0; r < GroupReduce<CP, 1>::R; ++r) red[wave][c0 + r] = acc[r];
      }
      __syncthreads();
      for (int c = threadIdx.x; c < CP; c += kBlock) {
        const int cc = cb * CP + c;
        if (cc < a.C) fwd_emit(a, row, cc, red[0][c] + red[1][c] + red[2][c] + red[3][c]);
      }
      __syncthreads();
    } else {
      GroupReduce<CP, HP>::run(acc, lane);
      if (GroupReduce<CP, HP>::writer(lane)) {
        const int c0 = GroupReduce<CP, HP>::chan_base(lane);
#pragma unroll
        for (int r = 0; r < GroupReduce<CP, HP>::R; ++r) red[wave][h * CP + c0 + r] = acc[r];
      }
      __syncthreads();
      for (int q = threadIdx.x; q < HP * CP; q += kBlock) {
        const int hh = q / CP, c = q % CP, cc = cb * CP + c;
        if (hh < a.H && cc < a.C) mine[hh * a.C + cc] = red[0][q] + red[1][q] + red[2][q] + red[3][q];
      }
      __syncthreads();
    }
  }
  if (single) {
    if (wave == 0 && el == 0 && hv) {
      a.emax[static_cast<int64_t>(row) * a.H + h] = M;
      a.esum[static_cast<int64_t>(row) * a.H + h] = S;
    }
    return;
  }
  if (wave == 0 && el == 0 && hv) {
    mine[HC + h] = M;
    mine[HC + a.H + h] = S;
  }
  if (!arrive_last(a.counters + sg.w, hr.y, &flag)) return;
  // Last segment of this row: merge the per-segment (m, s, acc) in order.
  const int stride = HC + 2 * a.H;
  if (threadIdx.x < a.H) {
    const int hh = threadIdx.x;
    float MM = kNegBig, SS = 0.0f;
    for (int q = 0; q < hr.y; ++q) {
      const float* pq = a.partial + static_cast<int64_t>(hr.x + q) * stride;
      ms_merge(MM, SS, pq[HC + hh], pq[HC + a.H + hh]);
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
        acch += pq[hh * a.C + c] * expf(pq[HC + hh] - fin_m[hh]);
      }
      if (fin_s[hh] > 0.0f) total += acch / fin_s[hh];
    }
    fwd_emit(a, row, c, total);
  }
}

// ---------------------------------------------------------------------------
// Backward, kernel 1: CSR rows.
// ---------------------------------------------------------------------------
template <typename T>
struct GatBwdArgs {
  int n, nnz, H, C;
  float slope, p, inv_h;
  bool vec_x;   // 16-byte loads of x rows are legal
  bool vec_gp;  // 16-byte loads of grad_pre rows are legal
  bool vec_gx;  // 16-byte stores of grad_feat rows are legal
  const int32_t* rowptr;
  const int32_t* col;
  const int32_t* colptr;
  const int32_t* rowind;
  const int32_t* perm;
  const float* emax;
  const float* esum;
  const uint8_t* mask;
  const T* x;
  const float* attn_row;
  const float* attn_col;
  const float* pre;
  const T* grad_y;
  // workspace
  float* grad_pre;   // [n, C]
  float* gscore;     // [nnz, H]: g_w/(1-p)-masked, then g_raw
  float* bias_part;  // [rows_blocks, C]
  float* bias_l2;    // [n_l2, C]
  float* part_row;   // [n_seg_rows, H]
  float* part_col;   // [n_seg_cols, H*C + H]
  int32_t* row_counters;
  int32_t* col_counters;  // [n_hrow_cols + 1]; last slot = bias counter
  int rows_blocks;
  int n_l2;
  // outputs
  T* grad_feat;
  float* grad_attn_row;
  float* grad_attn_col;
  float* grad_bias;
};

// Per-edge first pass of one tile: ge = <g_pre, x[j,h,:]>/H with the dropout
// mask and 1/(1-p) applied (the reference's grad_edge handling,
// collapsed_gat_cuda.cu:394-396), soft = s_eh, raw; returns sum_e s*ge.
template <typename T, int HP, int CP>
__device__ __forceinline__ float bwd_edge_pass(const GatBwdArgs<T>& a, int row, int eb, int ee, int h, int el,
                                               bool hv, float adst, float M, float S, const float* gp,
                                               float (&geR)[HP], float (&sR)[HP], float (&rawR)[HP]) {
  constexpr int EPW = kWave / HP;
  const int ncb = (a.C + CP - 1) / CP;
  float wpart = 0.0f;
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    const int t = eb + el + k * EPW;
    geR[k] = 0.0f;
    sR[k] = 0.0f;
    rawR[k] = 0.0f;
    if (hv && t < ee) {
      const int j = a.col[t];
      const T* xr = a.x + (static_cast<int64_t>(j) * a.H + h) * a.C;
      float dot = 0.0f;
      for (int cb = 0; cb < ncb; ++cb) {
        const int nvalid = min(CP, a.C - cb * CP);
        float xv[CP];
        load_run<T, CP>(xr + cb * CP, nvalid, a.vec_x, xv);
#pragma unroll
        for (int c = 0; c < CP; ++c) dot = fmaf(gp[cb * CP + c], xv[c], dot);
      }
      float ge = dot * a.inv_h;
      const float raw = adst + a.attn_col[static_cast<int64_t>(j) * a.H + h];
      const float sc = leaky(raw, a.slope);
      const float soft = S > 0.0f ? expf(sc - M) / S : 0.0f;
      if (a.p > 0.0f) {
        const bool keep = a.mask[static_cast<int64_t>(t) * a.H + h] != 0;
        ge = keep ? ge : 0.0f;
        ge = ge / (1.0f - a.p);
      }
      geR[k] = ge;
      sR[k] = soft;
      rawR[k] = raw;
      wpart += soft * ge;
    }
  }
  return wpart;
}

template <typename T, int HP>
__device__ __forceinline__ float bwd_edge_finish(const GatBwdArgs<T>& a, int eb, int ee, int h, int el, bool hv,
                                                 float wsum, const float (&geR)[HP], const float (&sR)[HP],
                                                 const float (&rawR)[HP]) {
  constexpr int EPW = kWave / HP;
  float gdst = 0.0f;
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    const int t = eb + el + k * EPW;
    if (hv && t < ee) {
      float g = sR[k] * (geR[k] - wsum);
      if (rawR[k] < 0.0f) g *= a.slope;
      a.gscore[static_cast<int64_t>(t) * a.H + h] = g;
      gdst += g;
    }
  }
  return gdst;
}

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
    if (publish) a.grad_pre[idx] = g;
  }
}

template <typename T, int HP, int CP>
__global__ __launch_bounds__(kBlock) void gat_bwd_rows_kernel(GatBwdArgs<T> a, Sched s) {
  constexpr int LGH = ilog2c(HP);
  const int lane = lane_id();
  const int wave = wave_id();
  const int h = lane & (HP - 1);
  const int el = lane >> LGH;
  const bool hv = h < a.H;
  const int b = blockIdx.x;
  const int padded = ((a.C + CP - 1) / CP) * CP;
  __shared__ float gp[kWavesPerBlock][kMaxC];
  __shared__ float wred[kWavesPerBlock][HP];
  __shared__ float fin[kMaxH];
  __shared__ int flag;

  float geR[HP], sR[HP], rawR[HP];

  if (b >= s.n_seg) {
    const int li = (b - s.n_seg) * kWavesPerBlock + wave;
    const bool has = li < s.n_light;
    const int row = has ? s.light[li] : 0;
    if (has) {
      bwd_grad_pre(a, row, lane, kWave, padded, gp[wave], true);
      wave_sync();
      const int eb = a.rowptr[row], ee = a.rowptr[row + 1];
      const int64_t rh = static_cast<int64_t>(row) * a.H + h;
      const float adst = hv ? a.attn_row[rh] : 0.0f;
      const float M = hv ? a.emax[rh] : 0.0f;
      const float S = hv ? a.esum[rh] : 0.0f;
      float wsum = bwd_edge_pass<T, HP, CP>(a, row, eb, ee, h, el, hv, adst, M, S, gp[wave], geR, sR, rawR);
      wsum = sum_across(wsum, HP);
      float gdst = bwd_edge_finish<T, HP>(a, eb, ee, h, el, hv, wsum, geR, sR, rawR);
      gdst = sum_across(gdst, HP);
      if (el == 0 && hv) a.grad_attn_row[rh] = gdst;
    } else {
      for (int c = lane; c < padded; c += kWave) gp[wave][c] = 0.0f;
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
  const int eb = sg.y + wave * kTile;
  const int ee = min(sg.z, eb + kTile);
  const int64_t rh = static_cast<int64_t>(row) * a.H + h;
  const float adst = hv ? a.attn_row[rh] : 0.0f;
  const float M = hv ? a.emax[rh] : 0.0f;
  const float S = hv ? a.esum[rh] : 0.0f;
  float wpart = bwd_edge_pass<T, HP, CP>(a, row, eb, ee, h, el, hv, adst, M, S, gp[0], geR, sR, rawR);
  wpart = sum_across(wpart, HP);
  if (el == 0) wred[wave][h] = wpart;
  __syncthreads();
  const float wblk = wred[0][h] + wred[1][h] + wred[2][h] + wred[3][h];
  __syncthreads();
  if (hr.y == 1) {
    float gdst = bwd_edge_finish<T, HP>(a, eb, ee, h, el, hv, wblk, geR, sR, rawR);
    gdst = sum_across(gdst, HP);
    if (el == 0) wred[wave][h] = gdst;
    __syncthreads();
    if (wave == 0 && el == 0 && hv) a.grad_attn_row[rh] = wred[0][h] + wred[1][h] + wred[2][h] + wred[3][h];
    return;
  }
  // Multi-segment row: publish g_w and the partial weighted sum, the last
  // segment finishes every edge of the row.
  {
    constexpr int EPW = kWave / HP;
#pragma unroll
    for (int k = 0; k < HP; ++k) {
      const int t = eb + el + k * EPW;
      if (hv && t < ee) a.gscore[static_cast<int64_t>(t) * a.H + h] = geR[k];
    }
  }
  if (wave == 0 && el == 0 && hv) a.part_row[static_cast<int64_t>(b) * a.H + h] = wblk;
  if (!arrive_last(a.row_counters + sg.w, hr.y, &flag)) return;
  if (threadIdx.x < a.H) {
    float t = 0.0f;
    for (int q = 0; q < hr.y; ++q) t += a.part_row[static_cast<int64_t>(hr.x + q) * a.H + threadIdx.x];
    fin[threadIdx.x] = t;
  }
  __syncthreads();
  const int rb = a.rowptr[row], re = a.rowptr[row + 1];
  // Thread -> (edge, head) with head = tid % HP fixed per thread.
  const int th = threadIdx.x & (HP - 1);
  const bool thv = th < a.H;
  const float tadst = thv ? a.attn_row[static_cast<int64_t>(row) * a.H + th] : 0.0f;
  const float tM = thv ? a.emax[static_cast<int64_t>(row) * a.H + th] : 0.0f;
  const float tS = thv ? a.esum[static_cast<int64_t>(row) * a.H + th] : 0.0f;
  const float tw = thv ? fin[th] : 0.0f;
  float gdst = 0.0f;
  if (thv) {
    for (int t = rb + (threadIdx.x >> LGH); t < re; t += kBlock / HP) {
      const int64_t eh = static_cast<int64_t>(t) * a.H + th;
      const int j = a.col[t];
      const float raw = tadst + a.attn_col[static_cast<int64_t>(j) * a.H + th];
      const float sc = leaky(raw, a.slope);
      const float soft = tS > 0.0f ? expf(sc - tM) / tS : 0.0f;
      float g = soft * (a.gscore[eh] - tw);
      if (raw < 0.0f) g *= a.slope;
      a.gscore[eh] = g;
      gdst += g;
    }
  }
  gdst = sum_across(gdst, HP);
  if (el == 0) wred[wave][h] = gdst;
  __syncthreads();
  if (threadIdx.x < a.H)
    a.grad_attn_row[static_cast<int64_t>(row) * a.H + threadIdx.x] =
        wred[0][threadIdx.x] + wred[1][threadIdx.x] + wred[2][threadIdx.x] + wred[3][threadIdx.x];
}

// ---------------------------------------------------------------------------
// Backward, kernel 2: CSC columns (source nodes) + grad_bias.
// ---------------------------------------------------------------------------
template <typename T, int HP>
__device__ __forceinline__ float bwd_col_weights(const GatBwdArgs<T>& a, int cb0, int ce, int h, int el, bool hv,
                                                 float asrc, int (&iR)[HP], float (&wR)[HP]) {
  constexpr int EPW = kWave / HP;
  float gsrc = 0.0f;
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    const int t = cb0 + el + k * EPW;
    iR[k] = 0;
    wR[k] = 0.0f;
    if (hv && t < ce) {
      const int i = a.rowind[t];
      const int e = a.perm[t];
      const int64_t ih = static_cast<int64_t>(i) * a.H + h;
      const int64_t eh = static_cast<int64_t>(e) * a.H + h;
      iR[k] = i;
      const float raw = a.attn_row[ih] + asrc;
      const float S = a.esum[ih];
      float w = 0.0f;
      bool keep = true;
      if (a.p > 0.0f) keep = a.mask[eh] != 0;
      if (keep && S > 0.0f) {
        w = expf(leaky(raw, a.slope) - a.emax[ih]) / S;
        if (a.p > 0.0f) w = w / (1.0f - a.p);
      }
      wR[k] = w;
      gsrc += a.gscore[eh];
    }
  }
  return gsrc;
}

template <typename T, int HP, int CP>
__device__ __forceinline__ void bwd_col_gather(const GatBwdArgs<T>& a, int cb, const int (&iR)[HP],
                                               const float (&wR)[HP], float (&acc)[CP]) {
  const int nvalid = min(CP, a.C - cb * CP);
#pragma unroll
  for (int c = 0; c < CP; ++c) acc[c] = 0.0f;
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    if (wR[k] != 0.0f) {
      float gv[CP];
      load_run<float, CP>(a.grad_pre + static_cast<int64_t>(iR[k]) * a.C + cb * CP, nvalid, a.vec_gp, gv);
#pragma unroll
      for (int c = 0; c < CP; ++c) acc[c] = fmaf(wR[k], gv[c], acc[c]);
    }
  }
}

template <typename T>
__device__ __forceinline__ void store_gx(const GatBwdArgs<T>& a, int j, int h, int c, float v) {
  a.grad_feat[(static_cast<int64_t>(j) * a.H + h) * a.C + c] = from_f32<T>(v * a.inv_h);
}

template <typename T, int HP, int CP>
__global__ __launch_bounds__(kBlock) void gat_bwd_cols_kernel(GatBwdArgs<T> a, Sched s) {
  constexpr int LGH = ilog2c(HP);
  using GR = GroupReduce<CP, HP>;
  const int lane = lane_id();
  const int wave = wave_id();
  const int h = lane & (HP - 1);
  const int el = lane >> LGH;
  const bool hv = h < a.H;
  const int ncb = (a.C + CP - 1) / CP;
  const int b = blockIdx.x;
  const int nsched = sched_blocks(s);
  __shared__ float red[kWavesPerBlock][HP * CP];
  __shared__ float gred[kWavesPerBlock][HP];
  __shared__ int flag;

  if (b >= nsched) {
    // grad_bias: level 1 sums 64 per-block partials of kernel 1, level 2
    // (last arriving workgroup) sums the level-1 results in order.
    const int q = b - nsched;
    const int lo = q * 64, hi = min(a.rows_blocks, lo + 64);
    for (int c = threadIdx.x; c < a.C; c += kBlock) {
      float t = 0.0f;
      for (int r = lo; r < hi; ++r) t += a.bias_part[static_cast<int64_t>(r) * a.C + c];
      a.bias_l2[static_cast<int64_t>(q) * a.C + c] = t;
    }
    if (!arrive_last(a.col_counters + s.n_hrow, a.n_l2, &flag)) return;
    for (int c = threadIdx.x; c < a.C; c += kBlock) {
      float t = 0.0f;
      for (int r = 0; r < a.n_l2; ++r) t += a.bias_l2[static_cast<int64_t>(r) * a.C + c];
      a.grad_bias[c] = t;
    }
    return;
  }

  int iR[HP];
  float wR[HP], acc[CP];

  if (b >= s.n_seg) {
    const int li = (b - s.n_seg) * kWavesPerBlock + wave;
    if (li >= s.n_light) return;
    const int j = s.light[li];
    const int cb0 = a.colptr[j], ce = a.colptr[j + 1];
    const int64_t jh = static_cast<int64_t>(j) * a.H + h;
    const float asrc = hv ? a.attn_col[jh] : 0.0f;
    float gsrc = bwd_col_weights<T, HP>(a, cb0, ce, h, el, hv, asrc, iR, wR);
    gsrc = sum_across(gsrc, HP);
    if (el == 0 && hv) a.grad_attn_col[jh] = gsrc;
    for (int cb = 0; cb < ncb; ++cb) {
      bwd_col_gather<T, HP, CP>(a, cb, iR, wR, acc);
      GR::run(acc, lane);
      if (GR::writer(lane) && hv) {
        const int c0 = cb * CP + GR::chan_base(lane);
#pragma unroll
        for (int r = 0; r < GR::R; ++r)
          if (c0 + r < a.C) store_gx(a, j, h, c0 + r, acc[r]);
      }
    }
    return;
  }

  // Heavy column segment.
  const int4 sg = s.seg[b];
  const int j = sg.x;
  const int2 hr = s.hrow[sg.w];
  const bool single = hr.y == 1;
  const int t0 = sg.y + wave * kTile;
  const int te = min(sg.z, t0 + kTile);
  const int64_t jh = static_cast<int64_t>(j) * a.H + h;
  const float asrc = hv ? a.attn_col[jh] : 0.0f;
  float gsrc = bwd_col_weights<T, HP>(a, t0, te, h, el, hv, asrc, iR, wR);
  gsrc = sum_across(gsrc, HP);
  if (el == 0) gred[wave][h] = gsrc;
  const int HC = a.H * a.C;
  float* mine = a.part_col + static_cast<int64_t>(b) * (HC + a.H);
  for (int cb = 0; cb < ncb; ++cb) {
    bwd_col_gather<T, HP, CP>(a, cb, iR, wR, acc);
    GR::run(acc, lane);
    if (GR::writer(lane)) {
      const int c0 = GR::chan_base(lane);
#pragma unroll
      for (int r = 0; r < GR::R; ++r) red[wave][h * CP + c0 + r] = acc[r];
    }
    __syncthreads();
    for (int q = threadIdx.x; q < HP * CP; q += kBlock) {
      const int hh = q / CP, c = q % CP, cc = cb * CP + c;
      if (hh < a.H && cc < a.C) {
        const float v = red[0][q] + red[1][q] + red[2][q] + red[3][q];
        if (single) store_gx(a, j, hh, cc, v);
        else mine[hh * a.C + cc] = v;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x < a.H) {
    const int hh = threadIdx.x;
    const float v = gred[0][hh] + gred[1][hh] + gred[2][hh] + gred[3][hh];
    if (single) a.grad_attn_col[static_cast<int64_t>(j) * a.H + hh] = v;
    else mine[HC + hh] = v;
  }
  if (single) return;
  if (!arrive_last(a.col_counters + sg.w, hr.y, &flag)) return;
  const int stride = HC + a.H;
  for (int q = threadIdx.x; q < HC + a.H; q += kBlock) {
    float t = 0.0f;
    for (int z = 0; z < hr.y; ++z) t += a.part_col[static_cast<int64_t>(hr.x + z) * stride + q];
    if (q < HC) store_gx(a, j, q / a.C, q % a.C, t);
    else a.grad_attn_col[static_cast<int64_t>(j) * a.H + (q - HC)] = t;
  }
}


template <typename T, int HP, int CP>
struct FwdLauncher {
  static int run(hipStream_t st, const GatFwdArgs<T>& a, const Sched& s) {
    const int blocks = sched_blocks(s);
    if (blocks > 0)
      hipLaunchKernelGGL((gat_fwd_kernel<T, HP, CP>), dim3(blocks), dim3(kBlock), 0, st, a, s);
    return check_launch("cign_gat_fwd");
  }
};

template <typename T, int HP, int CP>
struct BwdLauncher {
  static int run(hipStream_t st, const GatBwdArgs<T>& a, const Sched& rs, const Sched& cs) {
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
};


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
