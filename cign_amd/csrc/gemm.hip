// Dense projections of the CIGN block on gfx950 matrix cores (MFMA), with the
// elementwise work that follows them fused into the epilogue, and their C-ABI.
//
//   y = x W^T (+ b)                        nn.Linear / _local_amp_linear
//                                          (generic_engine/model_cign.py:86-103)
//   GAT lin + attention logits             x_proj = x W^T, alpha_src[n,h] =
//                                          <x_proj[n,h,:], att_src[h,:]>, alpha_dst
//                                          likewise (model_cign.py:546-553 then
//                                          fused_gat_sideops_cuda.cu:25-60)
//   proj + dropout-gamma-residual          g = x W^T + b, out = h + gamma * drop(g)
//                                          (model_cign.py:927-933, fused_block_ops
//                                          gamma residual, keep = 53-bit splitmix64)
//   backward                               grad_x = grad_y W (the forward kernel
//                                          against W^T), grad_W = grad_y^T x
//                                          (split-M MFMA partials), grad_b =
//                                          sum_n grad_y (chunked column sums)
//
// Math: fp32 (v_mfma_f32_16x16x4_f32, exact fp32 products) or bf16
// (v_mfma_f32_16x16x32_bf16, the autocast path of _local_amp_linear: operands
// rounded to bf16, fp32 accumulation, output rounded to bf16 and returned as
// fp32). The skinny shapes of the block (outputs <= 1536, K <= 1536, M =
// nodes) are HBM-bound in bf16 and MFMA-bound in fp32.
//
// Forward tiling: a 256-thread workgroup computes a 128 x BN tile (BN = 64 or
// 128), each wavefront 32 rows x BN columns (2 x BN/16 accumulator tiles of
// 16x16). x rows belong to one wavefront, so its MFMA fragments go straight
// from global memory to registers, two K steps (of 32) ahead; the W tile
// (BN x 32 per step) is shared by the four wavefronts through a
// double-buffered LDS tile in the MFMA operand type (converted once, at the
// LDS store), rows padded so 16 consecutive rows' 16-byte reads fall on
// distinct banks. W is the MFMA's first operand and x the second, so the
// accumulator layout gives each lane four consecutive output columns of one
// row: the epilogue stores 16 bytes per lane. MFMA fragment layouts (16x16xK,
// lane l): the first operand supplies row l%16 and k-slice l/16, the second
// column l%16 and the same k-slice, D holds rows 4*(l/16)+i, i < 4, of
// column l%16.
#include <algorithm>
#include <type_traits>

#include "rowops.h"

namespace cign {
namespace gemm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum Epi : int { kEpiStore = 0, kEpiLogits = 1, kEpiGamma = 2 };
enum Math : int { kMathF32 = 0, kMathBF16 = 1 };

constexpr int kThreads = 256;
constexpr int kBM = 128;
constexpr int kBK = 32;  // K per step: one bf16 MFMA K (32), two fp32 halves of 16
constexpr int kRowsPerWave = 32;

struct GemmArgs {
  int64_t M;
  int N, K;
  const void* x;      // [M, K] fp32 or bf16
  bool vec;           // rows of x and w start 16-byte aligned (vector loads)
  bool vec4;          // y (and h, out, mask) rows take 16-byte (4-column) stores
  const float* w;     // [N, K] fp32
  const float* bias;  // [N] or null
  float* y;           // [M, N]
  bool round_bf16;    // y holds bf16-rounded values (autocast output)
  // logits epilogue: heads of C columns, alpha_* [M, N / C]
  int C;
  const float* att_src;
  const float* att_dst;
  float* alpha_src;
  float* alpha_dst;
  // gamma-residual epilogue: out = h + gamma * keep(seed, m*N + n) / (1-p) * y
  const float* h;
  const float* gamma;
  float p;
  uint64_t seed;
  float* out;
  uint8_t* mask;
};

// Round to nearest even (gfx950 converts with v_cvt_pk_bf16_f32).
__device__ __forceinline__ float round_bf16(float v) { return static_cast<float>(static_cast<__bf16>(v)); }

// Operand type in LDS and the row padding of the LDS tiles.
template <int MATH>
struct Op;

template <>
struct Op<kMathF32> {
  using T = float;
  static constexpr int PAD = 4;  // row stride 36 floats (144 B)
};

template <>
struct Op<kMathBF16> {
  using T = __bf16;
  static constexpr int PAD = 8;  // row stride 40 bf16 (80 B)
};

template <int MATH>
constexpr int lds_stride() { return kBK + Op<MATH>::PAD; }

// Loads CNT consecutive values (4 fp32 or 8 bf16) at element k of row p, as
// fp32; zero past the row or K.
template <typename TS>
constexpr int CNT_OF = std::is_same_v<TS, float> ? 4 : 8;

template <typename TS, int CNT>
__device__ __forceinline__ void gload(const TS* p, bool valid, int k, int K, bool vec, float (&v)[CNT]) {
  if constexpr (std::is_same_v<TS, float>) {
    static_assert(CNT == 4, "fp32 chunks are 4 values");
    if (vec && valid && k + 4 <= K) {
      const float4 u = *reinterpret_cast<const float4*>(p + k);
      v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = (valid && k + q < K) ? p[k + q] : 0.0f;
    }
  } else {
    static_assert(CNT == 8, "bf16 chunks are 8 values");
    if (vec && valid && k + 8 <= K) {
      const uint4 u = *reinterpret_cast<const uint4*>(p + k);
      const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w4[i] << 16);
        v[2 * i + 1] = __uint_as_float(w4[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = (valid && k + q < K) ? to_f32(p[k + q]) : 0.0f;
    }
  }
}

// CNT values at element k of row p with one unconditional 16-byte load: the
// caller has checked (wave-uniformly) that the whole K step is in bounds and
// rows are aligned. Keeping these loads free of per-chunk branches lets a K
// step issue all of its loads back to back; a guarded load in its own basic
// block is followed by a wait for the previous one.
template <typename TS, int CNT>
__device__ __forceinline__ void gload_fast(const TS* p, int k, float (&v)[CNT]) {
  if constexpr (std::is_same_v<TS, float>) {
    static_assert(CNT == 4, "fp32 chunks are 4 values");
    const float4 u = *reinterpret_cast<const float4*>(p + k);
    v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
  } else {
    static_assert(CNT == 8, "bf16 chunks are 8 values");
    const uint4 u = *reinterpret_cast<const uint4*>(p + k);
    const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w4[i] << 16);
      v[2 * i + 1] = __uint_as_float(w4[i] & 0xffff0000u);
    }
  }
}

// One vector LDS store of N values converted to the operand type (16 bytes
// for fp32 x 4 and bf16 x 8, 8 bytes for bf16 x 4).
template <typename T, int N>
__device__ __forceinline__ void st_lds(T* d, const float (&v)[N]) {
  if constexpr (std::is_same_v<T, float>) {
    static_assert(N == 4, "fp32 LDS chunks are 4 values");
    *reinterpret_cast<float4*>(d) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (N == 4) {
    *reinterpret_cast<bf16x4*>(d) = bf16x4{static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1]),
                                           static_cast<__bf16>(v[2]), static_cast<__bf16>(v[3])};
  } else {
    static_assert(N == 8, "bf16 LDS chunks are 4 or 8 values");
    bf16x8 t;
#pragma unroll
    for (int q = 0; q < 8; ++q) t[q] = static_cast<__bf16>(v[q]);
    *reinterpret_cast<bf16x8*>(d) = t;
  }
}

// x fragments of one K step (32) for one 16-row tile, loaded straight from
// global memory into registers (a wavefront owns its rows, so x needs no LDS
// staging): lane l holds row l%16 and, for bf16 math, k = 8*(l/16) .. +7;
// for fp32 math, k = 4*(l/16) .. +3 and 16 + 4*(l/16) .. +3.
// `fast`: the K step lies inside K and rows are aligned (wave-uniform); rows
// past M then read row M-1, whose products land in output rows that are
// never stored.
template <typename TX, int MATH>
__device__ __forceinline__ void load_x(const GemmArgs& g, const TX* x, int64_t m, int k0, int ks, bool fast,
                                       float (&v)[8]) {
  const bool valid = m < g.M;
  float lo[CNT_OF<TX>], hi[CNT_OF<TX>];
  if (fast) {
    const TX* p = x + (valid ? m : g.M - 1) * g.K;
    if constexpr (!std::is_same_v<TX, float>) {
      gload_fast<TX, 8>(p, k0 + 8 * ks, lo);
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = lo[q];
    } else {
      const int ka = MATH == kMathBF16 ? k0 + 8 * ks : k0 + 4 * ks;
      const int kb = MATH == kMathBF16 ? ka + 4 : ka + 16;
      gload_fast<float, 4>(p, ka, lo);
      gload_fast<float, 4>(p, kb, hi);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = lo[q];
        v[4 + q] = hi[q];
      }
    }
    return;
  }
  const TX* p = x + (valid ? m : 0) * g.K;
  if constexpr (!std::is_same_v<TX, float>) {
    gload<TX, 8>(p, valid, k0 + 8 * ks, g.K, g.vec, lo);
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = lo[q];
  } else {
    const int ka = MATH == kMathBF16 ? k0 + 8 * ks : k0 + 4 * ks;
    const int kb = MATH == kMathBF16 ? ka + 4 : ka + 16;
    gload<float, 4>(p, valid, ka, g.K, g.vec, lo);
    gload<float, 4>(p, valid, kb, g.K, g.vec, hi);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = lo[q];
      v[4 + q] = hi[q];
    }
  }
}

// The K step starting at k0 can take the unconditional loads.
__device__ __forceinline__ bool fast_step(const GemmArgs& g, int k0) { return g.vec && k0 + kBK <= g.K; }

// One K step's x fragments of a wavefront: its two 16-row tiles.
struct XStep {
  float v[2][8];
};

template <typename TX, int MATH>
__device__ __forceinline__ void load_xstep(const GemmArgs& g, const TX* x, int64_t row0, int k0, int lane, XStep& a) {
  const bool fast = fast_step(g, k0);
#pragma unroll
  for (int r = 0; r < 2; ++r) load_x<TX, MATH>(g, x, row0 + 16 * r + (lane & 15), k0, lane >> 4, fast, a.v[r]);
}

// W tile of one K step (BN rows x 32) held in registers between the global
// load and the LDS store; all 256 threads share it.
template <int MATH, int BN>
struct WStage {
  static constexpr int CHUNKS = BN * kBK / 4 / kThreads;  // 16-byte fp32 chunks per thread
  float b[CHUNKS][4];

  __device__ __forceinline__ void load(const GemmArgs& g, int n0, int k0) {
    constexpr int CPR = kBK / 4;
    if (fast_step(g, k0)) {
      // Rows past N read row N-1; their output columns are never stored.
#pragma unroll
      for (int i = 0; i < CHUNKS; ++i) {
        const int id = threadIdx.x + i * kThreads;
        const int r = id / CPR, c = id % CPR;
        const int n = n0 + r;
        gload_fast<float, 4>(g.w + static_cast<int64_t>(n < g.N ? n : g.N - 1) * g.K, k0 + c * 4, b[i]);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id / CPR, c = id % CPR;
      const int n = n0 + r;
      gload<float, 4>(g.w + static_cast<int64_t>(n < g.N ? n : 0) * g.K, n < g.N, k0 + c * 4, g.K, g.vec, b[i]);
    }
  }
  __device__ __forceinline__ void store(typename Op<MATH>::T* Bs) const {
    constexpr int S = lds_stride<MATH>();
    constexpr int CPR = kBK / 4;
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id / CPR, c = id % CPR;
      st_lds<typename Op<MATH>::T, 4>(Bs + r * S + c * 4, b[i]);
    }
  }
};

// MFMAs of one K step. The W tile is the MFMA's first operand and x the
// second, so D = W x^T: lane l holds output rows (of y) 16r + l%16 and, per
// 16-column tile f, the four consecutive columns 16f + 4*(l/16) + q.
template <int MATH, int TN>
__device__ __forceinline__ void mma_step(const XStep& a, const typename Op<MATH>::T* Bs, int lane,
                                         f32x4 (&acc)[2][TN]) {
  constexpr int S = lds_stride<MATH>();
  const int rl = lane & 15, ks = lane >> 4;
  if constexpr (MATH == kMathBF16) {
    bf16x8 xa[2];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int q = 0; q < 8; ++q) xa[r][q] = static_cast<__bf16>(a.v[r][q]);
#pragma unroll
    for (int f = 0; f < TN; ++f) {
      const bf16x8 wb = *reinterpret_cast<const bf16x8*>(Bs + (16 * f + rl) * S + ks * 8);
#pragma unroll
      for (int r = 0; r < 2; ++r) acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb, xa[r], acc[r][f], 0, 0, 0);
    }
  } else {
    // Two 16-k halves; within a half, lane group ks supplies k = 4*ks .. +3
    // to four 16x16x4 MFMAs (the k order inside a sum is immaterial).
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int f = 0; f < TN; ++f) {
        const float4 wb = *reinterpret_cast<const float4*>(Bs + (16 * f + rl) * S + 16 * h + ks * 4);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const float* xv = a.v[r] + 4 * h;
          acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.x, xv[0], acc[r][f], 0, 0, 0);
          acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.y, xv[1], acc[r][f], 0, 0, 0);
          acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.z, xv[2], acc[r][f], 0, 0, 0);
          acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.w, xv[3], acc[r][f], 0, 0, 0);
        }
      }
  }
}

// Block index -> (row tile, column tile). Workgroups are dealt to the 8 XCDs
// round robin; consecutive blocks of one XCD take the column tiles of one row
// tile, so that row tile's x rows are fetched into one L2.
__device__ __forceinline__ void tile_of(int nrt, int nct, int& rt, int& ct) {
  const int b = blockIdx.x;
  const int total = nrt * nct;
  constexpr int kXcd = 8;
  const int full = total - total % kXcd;
  int v = b;
  if (b < full) v = (b % kXcd) * (full / kXcd) + b / kXcd;
  rt = v / nct;
  ct = v % nct;
}

// Epilogue of the swapped-operand layout: lane holds output row m = row0 +
// 16r + lane%16 and columns n = n0 + 16f + 4*(lane/16) + q, q < 4.
template <int EPI, int TN>
__device__ __forceinline__ void epilogue_swapped(const GemmArgs& g, f32x4 (&acc)[2][TN], int64_t row0, int n0,
                                                 int lane) {
  const int cg = (lane >> 4) * 4;
#pragma unroll
  for (int f = 0; f < TN; ++f) {
    const int nb = n0 + 16 * f + cg;
    const bool full4 = g.vec4 && nb + 4 <= g.N;
    float bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // Autocast casts the bias to bf16 with the other operands.
      const float b = (g.bias && nb + q < g.N) ? g.bias[nb + q] : 0.0f;
      bv[q] = g.round_bf16 ? round_bf16(b) : b;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int64_t m = row0 + 16 * r + (lane & 15);
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = acc[r][f][q] + bv[q];
        if (g.round_bf16) v[q] = round_bf16(v[q]);
        acc[r][f][q] = v[q];
      }
      if (m >= g.M) continue;
      const int64_t o = m * g.N + nb;
      if (full4) {
        *reinterpret_cast<float4*>(g.y + o) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nb + q < g.N) g.y[o + q] = v[q];
      }
      if constexpr (EPI == kEpiGamma) {
        float hv[4], ov[4];
        uint8_t mk[4];
        if (full4) {
          const float4 t = *reinterpret_cast<const float4*>(g.h + o);
          hv[0] = t.x; hv[1] = t.y; hv[2] = t.z; hv[3] = t.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) hv[q] = nb + q < g.N ? g.h[o + q] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bool keep = block_keep(g.seed, static_cast<uint64_t>(o + q), g.p);
          const float dv = keep ? (g.p > 0.0f ? v[q] / (1.0f - g.p) : v[q]) : 0.0f;
          ov[q] = hv[q] + (nb + q < g.N ? g.gamma[nb + q] : 0.0f) * dv;
          mk[q] = keep ? 1 : 0;
        }
        if (full4) {
          *reinterpret_cast<float4*>(g.out + o) = make_float4(ov[0], ov[1], ov[2], ov[3]);
          *reinterpret_cast<uchar4*>(g.mask + o) = make_uchar4(mk[0], mk[1], mk[2], mk[3]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (nb + q < g.N) {
              g.out[o + q] = ov[q];
              g.mask[o + q] = mk[q];
            }
        }
      }
    }
  }
  if constexpr (EPI == kEpiLogits) {
    // Heads of C columns lie whole inside the tile (host: BN % C == 0,
    // C % 16 == 0): sum y * att over a head's tiles and the lane's four
    // columns, then over the four lane groups.
    const int H = g.N / g.C;
    const int fph = g.C / 16;
    for (int h0 = 0; h0 < TN; h0 += fph) {
      const int head = (n0 + 16 * h0) / g.C;
      float ss[2] = {0.0f, 0.0f}, sd[2] = {0.0f, 0.0f};
#pragma unroll
      for (int f = 0; f < TN; ++f) {
        if (f < h0 || f >= h0 + fph) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + 16 * f + cg + q;
          const int c = n - head * g.C;
          const float as = n < g.N ? g.att_src[static_cast<int64_t>(head) * g.C + c] : 0.0f;
          const float ad = n < g.N ? g.att_dst[static_cast<int64_t>(head) * g.C + c] : 0.0f;
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            ss[r] = fmaf(acc[r][f][q], as, ss[r]);
            sd[r] = fmaf(acc[r][f][q], ad, sd[r]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int o = 16; o < kWave; o <<= 1) {
          ss[r] += shfl_xor(ss[r], o);
          sd[r] += shfl_xor(sd[r], o);
        }
      if (lane < 16 && head < H) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int64_t m = row0 + 16 * r + lane;
          if (m < g.M) {
            g.alpha_src[m * H + head] = ss[r];
            g.alpha_dst[m * H + head] = sd[r];
          }
        }
      }
    }
  }
}

// y = x W^T (+ bias) with the epilogue EPI, one 128 x BN tile per workgroup.
// The K loop keeps the x fragments of the next two K steps in flight (a
// two-slot register ring per wavefront) and double-buffers the shared W tile
// in LDS.
template <typename TX, int MATH, int BN, int EPI>
__global__ __launch_bounds__(kThreads) void gemm_nt_kernel(GemmArgs g, int nrt, int nct) {
  using T = typename Op<MATH>::T;
  constexpr int S = lds_stride<MATH>();
  constexpr int TN = BN / 16;
  __shared__ __align__(16) T Bs[2][BN * S];
  const int lane = lane_id();
  const int wave = wave_id();
  int rt, ct;
  tile_of(nrt, nct, rt, ct);
  const int64_t row0 = static_cast<int64_t>(rt) * kBM + wave * kRowsPerWave;
  const int n0 = ct * BN;
  const TX* x = static_cast<const TX*>(g.x);

  f32x4 acc[2][TN];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int f = 0; f < TN; ++f) acc[r][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int nk = (g.K + kBK - 1) / kBK;
  XStep a0, a1;
  WStage<MATH, BN> wst;
  load_xstep<TX, MATH>(g, x, row0, 0, lane, a0);
  if (nk > 1) load_xstep<TX, MATH>(g, x, row0, kBK, lane, a1);
  wst.load(g, n0, 0);
  wst.store(Bs[0]);
  __syncthreads();
  int buf = 0;
  for (int s = 0; s < nk; s += 2) {
    if (s + 1 < nk) wst.load(g, n0, (s + 1) * kBK);
    mma_step<MATH, TN>(a0, Bs[buf], lane, acc);
    if (s + 2 < nk) load_xstep<TX, MATH>(g, x, row0, (s + 2) * kBK, lane, a0);
    if (s + 1 < nk) wst.store(Bs[buf ^ 1]);
    __syncthreads();
    buf ^= 1;
    if (s + 1 >= nk) break;  // uniform
    if (s + 2 < nk) wst.load(g, n0, (s + 2) * kBK);
    mma_step<MATH, TN>(a1, Bs[buf], lane, acc);
    if (s + 3 < nk) load_xstep<TX, MATH>(g, x, row0, (s + 3) * kBK, lane, a1);
    if (s + 2 < nk) wst.store(Bs[buf ^ 1]);
    __syncthreads();
    buf ^= 1;
  }

  epilogue_swapped<EPI, TN>(g, acc, row0, n0, lane);
}

// ---------------------------------------------------------------------------
// bf16 math: both operands staged through LDS
// ---------------------------------------------------------------------------
// With bf16 MFMAs (four times the fp32 rate) the K loop is bound by operand
// delivery; staging x and W tiles in LDS as bf16 (converted once) and keeping
// three workgroups per CU measured faster than register-resident x
// fragments, which need the raw fp32 rows in flight. The tile loads of one K
// step are held in registers between the global load and the LDS store. A: 128 x 32 of x; B: BN x 32 of w (fp32).
template <typename TX, int MATH, int BN>
struct LdsStage {
  static constexpr int XC = std::is_same_v<TX, float> ? 4 : 8;  // values per x chunk (16 bytes)
  static constexpr int A_CHUNKS = kBM * kBK / XC / kThreads;   // per thread
  static constexpr int B_CHUNKS = BN * kBK / 4 / kThreads;
  float a[A_CHUNKS][XC];
  float b[B_CHUNKS][4];

  __device__ __forceinline__ void load(const GemmArgs& g, const TX* x, int64_t m0, int n0, int k0) {
    constexpr int ACPR = kBK / XC;  // chunks per A row
    if (fast_step(g, k0)) {
      // Rows past M (N) read row M-1 (N-1); their outputs are never stored.
#pragma unroll
      for (int i = 0; i < A_CHUNKS; ++i) {
        const int id = threadIdx.x + i * kThreads;
        const int r = id / ACPR, c = id % ACPR;
        const int64_t m = m0 + r;
        gload_fast<TX, XC>(x + (m < g.M ? m : g.M - 1) * g.K, k0 + c * XC, a[i]);
      }
      constexpr int BCPR = kBK / 4;
#pragma unroll
      for (int i = 0; i < B_CHUNKS; ++i) {
        const int id = threadIdx.x + i * kThreads;
        const int r = id / BCPR, c = id % BCPR;
        const int n = n0 + r;
        gload_fast<float, 4>(g.w + static_cast<int64_t>(n < g.N ? n : g.N - 1) * g.K, k0 + c * 4, b[i]);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id / ACPR, c = id % ACPR;
      const int64_t m = m0 + r;
      gload<TX, XC>(x + m * g.K, m < g.M, k0 + c * XC, g.K, g.vec, a[i]);
    }
    constexpr int BCPR = kBK / 4;
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id / BCPR, c = id % BCPR;
      const int n = n0 + r;
      gload<float, 4>(g.w + static_cast<int64_t>(n) * g.K, n < g.N, k0 + c * 4, g.K, g.vec, b[i]);
    }
  }

  __device__ __forceinline__ void store(typename Op<MATH>::T* As, typename Op<MATH>::T* Bs) const {
    using T = typename Op<MATH>::T;
    constexpr int S = lds_stride<MATH>();
    constexpr int ACPR = kBK / XC;
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id / ACPR, c = id % ACPR;
      st_lds<T, XC>(As + r * S + c * XC, a[i]);
    }
    constexpr int BCPR = kBK / 4;
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id / BCPR, c = id % BCPR;
      st_lds<T, 4>(Bs + r * S + c * 4, b[i]);
    }
  }
};

// MFMAs of one K step on the LDS tiles: the wave's 2 row tiles x TN column
// tiles, W as the first operand (the swapped-operand accumulator layout of
// epilogue_swapped).
template <int MATH, int TN>
__device__ __forceinline__ void mma_step_lds(const typename Op<MATH>::T* As, const typename Op<MATH>::T* Bs, int wave,
                                         int lane, f32x4 (&acc)[2][TN]) {
  constexpr int S = lds_stride<MATH>();
  const int rl = lane & 15, ks = lane >> 4;
  if constexpr (MATH == kMathBF16) {
#pragma unroll
    for (int hk = 0; hk < kBK; hk += 32) {
      bf16x8 a[2];
#pragma unroll
      for (int r = 0; r < 2; ++r)
        a[r] = *reinterpret_cast<const bf16x8*>(As + (wave * kRowsPerWave + 16 * r + rl) * S + hk + ks * 8);
#pragma unroll
      for (int f = 0; f < TN; ++f) {
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(Bs + (16 * f + rl) * S + hk + ks * 8);
#pragma unroll
        for (int r = 0; r < 2; ++r) acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, a[r], acc[r][f], 0, 0, 0);
      }
    }
  } else {
    // Two 16-k halves; within a half, lane group ks supplies k = 4*ks .. +3
    // to four 16x16x4 MFMAs (the k order inside a sum is immaterial).
#pragma unroll
    for (int hk = 0; hk < kBK; hk += 16) {
      float4 a[2];
#pragma unroll
      for (int r = 0; r < 2; ++r)
        a[r] = *reinterpret_cast<const float4*>(As + (wave * kRowsPerWave + 16 * r + rl) * S + hk + ks * 4);
#pragma unroll
      for (int f = 0; f < TN; ++f) {
        const float4 b = *reinterpret_cast<const float4*>(Bs + (16 * f + rl) * S + hk + ks * 4);
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(b.x, a[r].x, acc[r][f], 0, 0, 0);
          acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(b.y, a[r].y, acc[r][f], 0, 0, 0);
          acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(b.z, a[r].z, acc[r][f], 0, 0, 0);
          acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(b.w, a[r].w, acc[r][f], 0, 0, 0);
        }
      }
    }
  }
}


template <typename TX, int MATH, int BN, int EPI>
__global__ __launch_bounds__(kThreads) void gemm_nt_lds_kernel(GemmArgs g, int nrt, int nct) {
  using T = typename Op<MATH>::T;
  constexpr int S = lds_stride<MATH>();
  constexpr int TN = BN / 16;
  __shared__ __align__(16) T As[2][kBM * S];
  __shared__ __align__(16) T Bs[2][BN * S];
  const int lane = lane_id();
  const int wave = wave_id();
  int rt, ct;
  tile_of(nrt, nct, rt, ct);
  const int64_t m0 = static_cast<int64_t>(rt) * kBM;
  const int n0 = ct * BN;
  const TX* x = static_cast<const TX*>(g.x);

  f32x4 acc[2][TN];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int f = 0; f < TN; ++f) acc[r][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  LdsStage<TX, MATH, BN> regs;
  regs.load(g, x, m0, n0, 0);
  regs.store(As[0], Bs[0]);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < g.K; k0 += kBK) {
    const bool more = k0 + kBK < g.K;
    if (more) regs.load(g, x, m0, n0, k0 + kBK);
    mma_step_lds<MATH, TN>(As[buf], Bs[buf], wave, lane, acc);
    if (more) regs.store(As[buf ^ 1], Bs[buf ^ 1]);
    __syncthreads();
    buf ^= 1;
  }

  epilogue_swapped<EPI, TN>(g, acc, m0 + wave * kRowsPerWave, n0, lane);
}

// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// Backward helpers
// ---------------------------------------------------------------------------
// part[c][n] = sum of grad_y rows of chunk c (a workgroup: 64 columns x 4 row
// slices, four accumulators per thread, slices combined in order).
__global__ __launch_bounds__(kThreads) void bias_grad_kernel(const float* gy, int64_t M, int N, int64_t chunk,
                                                             float* part) {
  __shared__ float red[kThreads];
  const int t = threadIdx.x;
  const int n = blockIdx.x * 64 + (t & 63);
  const int s = t >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * chunk;
  const int64_t r1 = r0 + chunk < M ? r0 + chunk : M;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  if (n < N) {
    int64_t r = r0 + s;
    for (; r + 12 < r1; r += 16) {
      a0 += gy[r * N + n];
      a1 += gy[(r + 4) * N + n];
      a2 += gy[(r + 8) * N + n];
      a3 += gy[(r + 12) * N + n];
    }
    for (; r < r1; r += 4) a0 += gy[r * N + n];
  }
  red[t] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (s == 0 && n < N)
    part[static_cast<int64_t>(blockIdx.y) * N + n] = red[t] + red[t + 64] + red[t + 128] + red[t + 192];
}

// wt [K, N] = w [N, K]^T through a 32 x 32 LDS tile (row stride 33 floats,
// so the column reads of the transposed store fall on distinct banks). Grid
// (ceil(K/32), ceil(N/32)), 256 threads, four rows each; reads and writes are
// 128-byte row segments.
__global__ void __launch_bounds__(256) transpose_w_kernel(const float* __restrict__ w, int N, int K,
                                                         float* __restrict__ wt) {
  __shared__ float tile[32][33];
  const int k0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
  const int c = threadIdx.x & 31, r0 = threadIdx.x >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + 8 * i;
    if (n0 + r < N && k0 + c < K) tile[r][c] = w[static_cast<int64_t>(n0 + r) * K + k0 + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + 8 * i;
    if (k0 + r < K && n0 + c < N) wt[static_cast<int64_t>(k0 + r) * N + n0 + c] = tile[c][r];
  }
}

// ---- grad_W = grad_y^T x of the larger projections: a reduction over the
// M node rows with a small output, which the library GEMMs run at a fraction
// of their speed. A workgroup owns a 128 x 128 tile of grad_W and a chunk of
// rows; per 32-row step it loads the grad_y and x row slices (fp32, 16-byte
// loads), converts them to the MFMA operand type and stores them transposed
// in LDS ([n][m] and [k][m], double buffered), so each MFMA operand fragment
// (8 consecutive m of one n or k) is one 16-byte LDS read. The four
// wavefronts each compute 64 x 64 outputs. Each chunk writes its partial
// tile; colsum_kernel adds the chunks in order (deterministic, no atomics).
constexpr int kWgT = 128;  // grad_W tile (n and k)
constexpr int kWgM = 32;   // rows per step

// LDS layout of a transposed operand tile: 128 rows (n or k) of 32 m values
// in the MFMA operand type, no padding; the 16-byte chunk c of row j is
// stored at chunk position c ^ ((j / 4) % chunks), which spreads the
// transposed stores of one wavefront over the banks while every operand
// fragment stays one aligned 16-byte read.
template <int MATH>
struct WgLayout {
  using T = typename Op<MATH>::T;
  static constexpr int CE = 16 / sizeof(T);  // elements per 16-byte chunk
  static constexpr int NC = kWgM / CE;       // chunks per row
  __device__ __forceinline__ static int pos(int j, int m) {
    return j * kWgM + (((m / CE) ^ ((j / 4) % NC)) * CE) + m % CE;
  }
  __device__ __forceinline__ static int frag(int j, int chunk) { return j * kWgM + ((chunk ^ ((j / 4) % NC)) * CE); }
};

template <int MATH>
struct WgStage {
  // 128 columns x 32 rows of one operand: 1024 float4, four per thread.
  // Thread id takes row id / 8 and column quads id % 8 + 8i, so a
  // wavefront's load covers 8 rows x 128 contiguous bytes.
  float v[4][4];
  __device__ __forceinline__ void load(const float* src, int64_t ld, int64_t m0, int64_t m1, int c0, int cmax,
                                       bool vec) {
    const int r = threadIdx.x / 8;
    const int64_t m = m0 + r;
    const bool ok = m < m1;
    if (vec && m0 + 32 <= m1 && c0 + 128 <= cmax) {
      // Whole step in bounds (wave-uniform): unconditional loads, issued
      // back to back.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = ((threadIdx.x % 8) + 8 * i) * 4;
        const float4 t = *reinterpret_cast<const float4*>(src + m * ld + c0 + c);
        v[i][0] = t.x; v[i][1] = t.y; v[i][2] = t.z; v[i][3] = t.w;
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = ((threadIdx.x % 8) + 8 * i) * 4;
      const float* p = src + (ok ? m : 0) * ld + c0 + c;
      if (vec && ok && c0 + c + 4 <= cmax) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        v[i][0] = t.x; v[i][1] = t.y; v[i][2] = t.z; v[i][3] = t.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[i][q] = (ok && c0 + c + q < cmax) ? p[q] : 0.0f;
      }
    }
  }
  __device__ __forceinline__ void store(typename Op<MATH>::T* Ts) const {
    using T = typename Op<MATH>::T;
    const int r = threadIdx.x / 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = ((threadIdx.x % 8) + 8 * i) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) Ts[WgLayout<MATH>::pos(c + q, r)] = static_cast<T>(v[i][q]);
    }
  }
};

template <int MATH>
__global__ __launch_bounds__(kThreads) void wgrad_kernel(const float* gy, const float* x, int64_t M, int N, int K,
                                                         int64_t chunk, int ntk, bool vec, float* part) {
  using T = typename Op<MATH>::T;
  using Lay = WgLayout<MATH>;
  __shared__ __align__(16) T Gs[2][kWgT * kWgM];
  __shared__ __align__(16) T Xs[2][kWgT * kWgM];
  const int lane = lane_id();
  const int wave = wave_id();
  const int n0 = (blockIdx.x / ntk) * kWgT, k0 = (blockIdx.x % ntk) * kWgT;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * chunk;
  const int64_t m1 = m0 + chunk < M ? m0 + chunk : M;
  const int wn = (wave >> 1) * 64, wk = (wave & 1) * 64;  // the wave's 64 x 64 quadrant
  const int rl = lane & 15, ks = lane >> 4;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  WgStage<MATH> sg, sx;
  sg.load(gy, N, m0, m1, n0, N, vec);
  sx.load(x, K, m0, m1, k0, K, vec);
  sg.store(Gs[0]);
  sx.store(Xs[0]);
  __syncthreads();
  int buf = 0;
  for (int64_t mb = m0; mb < m1; mb += kWgM) {
    const bool more = mb + kWgM < m1;
    if (more) {
      sg.load(gy, N, mb + kWgM, m1, n0, N, vec);
      sx.load(x, K, mb + kWgM, m1, k0, K, vec);
    }
    const T* G = Gs[buf];
    const T* X = Xs[buf];
    if constexpr (MATH == kMathBF16) {
      bf16x8 xb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xb[j] = *reinterpret_cast<const bf16x8*>(X + Lay::frag(wk + 16 * j + rl, ks));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bf16x8 gb = *reinterpret_cast<const bf16x8*>(G + Lay::frag(wn + 16 * i + rl, ks));
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(gb, xb[j], acc[i][j], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float4 xb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xb[j] = *reinterpret_cast<const float4*>(X + Lay::frag(wk + 16 * j + rl, 4 * h + ks));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 gb = *reinterpret_cast<const float4*>(G + Lay::frag(wn + 16 * i + rl, 4 * h + ks));
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(gb.x, xb[j].x, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(gb.y, xb[j].y, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(gb.z, xb[j].z, acc[i][j], 0, 0, 0);
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(gb.w, xb[j].w, acc[i][j], 0, 0, 0);
          }
        }
      }
    }
    if (more) {
      sg.store(Gs[buf ^ 1]);
      sx.store(Xs[buf ^ 1]);
    }
    __syncthreads();
    buf ^= 1;
  }
  // lane holds grad_W rows n = n0 + wn + 16i + 4*(lane/16) + q of column
  // k = k0 + wk + 16j + lane%16
  float* out = part + static_cast<int64_t>(blockIdx.y) * N * K;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = k0 + wk + 16 * j + rl;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn + 16 * i + 4 * ks + q;
        if (n < N && k < K) out[static_cast<int64_t>(n) * K + k] = acc[i][j][q];
      }
    }
}

// ---- Backward of a projection with few outputs (N <= kSmallN, e.g. the
// classifier): two streaming passes on the VALU, where the library GEMMs
// pick poor kernels for the degenerate shapes. Under autocast (RB) every
// operand is rounded to bf16 before its product, as the bf16 GEMM would.
constexpr int kSmallN = 16;

__device__ __forceinline__ float rb_if(bool rb, float v) { return rb ? round_bf16(v) : v; }

// grad_x[m, 4c .. 4c+3] = sum_n grad_y[m, n] W[n, 4c .. 4c+3]; a workgroup
// covers 4 rows x 64 column quads (16-byte stores when K % 4 == 0).
template <bool RB>
__global__ __launch_bounds__(kThreads) void small_n_grad_x_kernel(const float* gy, int64_t M, int N, int K,
                                                                  const float* w, float* gx) {
  const int k = (blockIdx.x * 64 + (threadIdx.x & 63)) * 4;
  const int64_t m = static_cast<int64_t>(blockIdx.y) * 4 + (threadIdx.x >> 6);
  if (m >= M || k >= K) return;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const bool full = (K & 3) == 0;
  for (int n = 0; n < N; ++n) {
    const float g = rb_if(RB, gy[m * N + n]);
    const float* wr = w + static_cast<int64_t>(n) * K + k;
    if (full) {
      const float4 t = *reinterpret_cast<const float4*>(wr);
      acc[0] = fmaf(g, rb_if(RB, t.x), acc[0]);
      acc[1] = fmaf(g, rb_if(RB, t.y), acc[1]);
      acc[2] = fmaf(g, rb_if(RB, t.z), acc[2]);
      acc[3] = fmaf(g, rb_if(RB, t.w), acc[3]);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (k + q < K) acc[q] = fmaf(g, rb_if(RB, wr[q]), acc[q]);
    }
  }
  float* o = gx + m * K + k;
  if (full) {
    *reinterpret_cast<float4*>(o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (k + q < K) o[q] = acc[q];
  }
}

// part[c][n][k] = sum over the rows of chunk c of grad_y[m, n] x[m, k]; a
// thread owns four consecutive k for all n.
template <bool RB>
__global__ __launch_bounds__(kThreads) void small_n_grad_w_kernel(const float* gy, const float* x, int64_t M, int N,
                                                                  int K, int64_t chunk, float* part) {
  const int K4 = (K + 3) / 4;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * chunk;
  const int64_t r1 = r0 + chunk < M ? r0 + chunk : M;
  for (int c4 = blockIdx.x * kThreads + threadIdx.x; c4 < K4; c4 += gridDim.x * kThreads) {
    const int k = c4 * 4;
    float acc[kSmallN][4];
#pragma unroll
    for (int n = 0; n < kSmallN; ++n)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[n][q] = 0.0f;
#pragma unroll 4
    for (int64_t m = r0; m < r1; ++m) {
      float xv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) xv[q] = k + q < K ? rb_if(RB, x[m * K + k + q]) : 0.0f;
#pragma unroll
      for (int n = 0; n < kSmallN; ++n) {
        const float g = n < N ? rb_if(RB, gy[m * N + n]) : 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[n][q] = fmaf(g, xv[q], acc[n][q]);
      }
    }
    float* out = part + static_cast<int64_t>(blockIdx.y) * N * K;
#pragma unroll
    for (int n = 0; n < kSmallN; ++n)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n < N && k + q < K) out[static_cast<int64_t>(n) * K + k + q] = acc[n][q];
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
inline bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Column tile: fp32 math 64 (two waves per SIMD with the register-resident x
// fragments); bf16 math 64 up to N = 256 (more workgroups for the skinny
// shapes), else 128. For the logits epilogue the tile must hold whole heads
// of 16..128 columns.
inline int pick_bn(int N, int C, int math) {
  int bn = (math == kMathF32 || N <= 256) ? 64 : 128;
  if (C > 0) {
    if (C % 16 != 0 || C > 128) return 0;
    if (bn % C != 0) bn = 128;
    if (bn % C != 0) return 0;
  }
  return bn;
}

template <typename TX, int MATH, int EPI>
int launch_nt(hipStream_t st, const GemmArgs& g, int bn) {
  const int nrt = static_cast<int>((g.M + kBM - 1) / kBM);
  const int nct = (g.N + bn - 1) / bn;
  const int64_t blocks = static_cast<int64_t>(nrt) * nct;
  if (blocks == 0) return kOk;
  if (blocks > 0x7fffffff) return set_error(kInvalid, "cign linear: too many tiles");
  if constexpr (MATH == kMathBF16) {
    if (bn == 64)
      hipLaunchKernelGGL((gemm_nt_lds_kernel<TX, MATH, 64, EPI>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                         0, st, g, nrt, nct);
    else
      hipLaunchKernelGGL((gemm_nt_lds_kernel<TX, MATH, 128, EPI>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kThreads), 0, st, g, nrt, nct);
  } else {
    if (bn == 64)
      hipLaunchKernelGGL((gemm_nt_kernel<TX, MATH, 64, EPI>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0,
                         st, g, nrt, nct);
    else
      hipLaunchKernelGGL((gemm_nt_kernel<TX, MATH, 128, EPI>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                         0, st, g, nrt, nct);
  }
  return check_launch("cign linear");
}

template <int EPI>
int dispatch_nt(hipStream_t st, const GemmArgs& g, int x_dtype, int math, int bn) {
  if (x_dtype == kBF16) {
    if (math != kMathBF16) return set_error(kInvalid, "cign linear: bfloat16 inputs need math=1 (bf16 MFMA)");
    return launch_nt<bf16, kMathBF16, EPI>(st, g, bn);
  }
  if (x_dtype != kF32) return set_error(kInvalid, "cign linear: unsupported x dtype %d", x_dtype);
  if (math == kMathF32) return launch_nt<float, kMathF32, EPI>(st, g, bn);
  if (math == kMathBF16) return launch_nt<float, kMathBF16, EPI>(st, g, bn);
  return set_error(kInvalid, "cign linear: math must be 0 (fp32) or 1 (bf16)");
}

inline int check_common(const char* who, int64_t M, int N, int K, const void* x, const float* w, const void* y) {
  if (M < 0 || N <= 0 || K <= 0) return set_error(kInvalid, "%s: bad sizes M=%lld N=%d K=%d", who,
                                                 static_cast<long long>(M), N, K);
  if (!w || (M > 0 && (!x || !y))) return set_error(kInvalid, "%s: null pointer", who);
  return kOk;
}

// 16-byte vector loads are legal when every row of x and w starts aligned.
inline bool rows_aligned(const void* x, int x_dtype, const float* w, int K) {
  const int xrow = K * (x_dtype == kBF16 ? 2 : 4);
  return aligned16(x) && aligned16(w) && xrow % 16 == 0 && (K * 4) % 16 == 0;
}

// Workspace layout of cign_linear_bwd.
struct BwdWs {
  int chunks, wg_chunks;
  int64_t chunk, wg_chunk, part_b, part_w, wt, total;
};

inline BwdWs bwd_ws(int64_t M, int N, int K, bool bias) {
  BwdWs L;
  // row chunks of the bias (and, for few outputs, grad_W) partials: 64 rows,
  // or 16 for few outputs (more workgroups for the per-chunk VALU sums)
  const int64_t rows_per = N <= kSmallN ? 16 : 64;
  int64_t chunks = std::max<int64_t>(1, std::min<int64_t>(N <= kSmallN ? 4096 : 1024, (M + rows_per - 1) / rows_per));
  L.chunk = std::max<int64_t>(1, (M + chunks - 1) / chunks);
  chunks = M > 0 ? (M + L.chunk - 1) / L.chunk : 1;
  L.chunks = static_cast<int>(chunks);
  auto al = [](int64_t v) { return (v + 255) & ~int64_t(255); };
  int64_t off = 0;
  L.part_b = off; off = al(off + (bias ? 4LL * chunks * N : 0));
  // grad_W partials per row chunk: the few-output VALU sums use the bias
  // chunks; the MFMA kernel takes chunks of >= 256 rows, about 512
  // workgroups over its 128 x 128 tiles
  const bool small = N <= kSmallN;
  const int64_t tiles = static_cast<int64_t>((N + kWgT - 1) / kWgT) * ((K + kWgT - 1) / kWgT);
  int64_t wgc = std::max<int64_t>(1, std::min<int64_t>((M + 255) / 256, 512 / tiles));
  L.wg_chunk = std::max<int64_t>(kWgM, ((M + wgc - 1) / wgc + kWgM - 1) / kWgM * kWgM);
  wgc = M > 0 ? (M + L.wg_chunk - 1) / L.wg_chunk : 1;
  L.wg_chunks = static_cast<int>(wgc);
  L.part_w = off; off = al(off + 4LL * (small ? chunks : wgc) * N * K);
  // grad_x = grad_y W runs on the forward NT kernel against W^T [K, N]
  L.wt = off; off = al(off + (small ? 0 : 4LL * N * K));
  L.total = off;
  return L;
}

}  // namespace gemm
}  // namespace cign

using namespace cign;
using namespace cign::gemm;

extern "C" {

int cign_linear_fwd(void* stream, int64_t M, int32_t N, int32_t K, int32_t x_dtype, int32_t math, const void* x,
                    const float* w, const float* bias, float* y) {
  int rc = check_common("cign_linear_fwd", M, N, K, x, w, y);
  if (rc) return rc;
  if (M == 0) return kOk;
  GemmArgs g{};
  g.M = M; g.N = N; g.K = K; g.x = x; g.w = w; g.bias = bias; g.y = y;
  g.vec = rows_aligned(x, x_dtype, w, K);
  g.vec4 = N % 4 == 0 && aligned16(y);
  g.round_bf16 = math == kMathBF16;
  return dispatch_nt<kEpiStore>(static_cast<hipStream_t>(stream), g, x_dtype, math, pick_bn(N, 0, math));
}

int cign_linear_logits_fwd(void* stream, int64_t M, int32_t heads, int32_t channels, int32_t K, int32_t x_dtype,
                           int32_t math, const void* x, const float* w, const float* att_src, const float* att_dst,
                           float* y, float* alpha_src, float* alpha_dst) {
  const int N = heads * channels;
  int rc = check_common("cign_linear_logits_fwd", M, N, K, x, w, y);
  if (rc) return rc;
  if (!att_src || !att_dst || (M > 0 && (!alpha_src || !alpha_dst)))
    return set_error(kInvalid, "cign_linear_logits_fwd: null pointer");
  const int bn = pick_bn(N, channels, math);
  if (bn == 0)
    return set_error(kInvalid, "cign_linear_logits_fwd: channels=%d must be 16, 32, 64 or 128 (use cign_linear_fwd + "
                     "cign_attn_logits_fwd)", channels);
  if (M == 0) return kOk;
  GemmArgs g{};
  g.M = M; g.N = N; g.K = K; g.x = x; g.w = w; g.y = y;
  g.vec = rows_aligned(x, x_dtype, w, K);
  g.vec4 = N % 4 == 0 && aligned16(y);
  g.round_bf16 = math == kMathBF16;
  g.C = channels; g.att_src = att_src; g.att_dst = att_dst; g.alpha_src = alpha_src; g.alpha_dst = alpha_dst;
  return dispatch_nt<kEpiLogits>(static_cast<hipStream_t>(stream), g, x_dtype, math, bn);
}

int cign_linear_gamma_fwd(void* stream, int64_t M, int32_t N, int32_t K, int32_t x_dtype, int32_t math,
                          const void* x, const float* w, const float* bias, const float* h, const float* gamma,
                          float dropout_p, uint64_t seed, float* g_out, float* y, uint8_t* mask) {
  int rc = check_common("cign_linear_gamma_fwd", M, N, K, x, w, g_out);
  if (rc) return rc;
  if (!gamma || (M > 0 && (!h || !y || !mask))) return set_error(kInvalid, "cign_linear_gamma_fwd: null pointer");
  if (!(dropout_p >= 0.0f && dropout_p < 1.0f))
    return set_error(kInvalid, "cign_linear_gamma_fwd: dropout_p must be in [0,1)");
  if (M == 0) return kOk;
  GemmArgs g{};
  g.M = M; g.N = N; g.K = K; g.x = x; g.w = w; g.bias = bias; g.y = g_out;
  g.vec = rows_aligned(x, x_dtype, w, K);
  g.vec4 = N % 4 == 0 && aligned16(g_out) && aligned16(h) && aligned16(y) &&
           reinterpret_cast<uintptr_t>(mask) % 4 == 0;
  g.round_bf16 = math == kMathBF16;
  g.h = h; g.gamma = gamma; g.p = dropout_p; g.seed = seed; g.out = y; g.mask = mask;
  return dispatch_nt<kEpiGamma>(static_cast<hipStream_t>(stream), g, x_dtype, math, pick_bn(N, 0, math));
}

int64_t cign_linear_bwd_workspace_bytes(int64_t M, int32_t N, int32_t K, int32_t with_bias) {
  return bwd_ws(M, N, K, with_bias != 0).total;
}

int cign_linear_bwd(void* stream, int64_t M, int32_t N, int32_t K, int32_t math, const float* grad_y, const float* x,
                    const float* w, float* grad_x, float* grad_w, float* grad_b, void* workspace,
                    int64_t workspace_bytes) {
  if (M < 0 || N <= 0 || K <= 0) return set_error(kInvalid, "cign_linear_bwd: bad sizes");
  if (!w || !grad_w || (M > 0 && (!grad_y || !x))) return set_error(kInvalid, "cign_linear_bwd: null pointer");
  if (math != kMathF32 && math != kMathBF16) return set_error(kInvalid, "cign_linear_bwd: math must be 0 or 1");
  if (M > 0x7fffffff) return set_error(kInvalid, "cign_linear_bwd: M too large");
  const BwdWs L = bwd_ws(M, N, K, grad_b != nullptr);
  if (workspace_bytes < L.total || (L.total > 0 && !workspace))
    return set_error(kInvalid, "cign_linear_bwd: workspace too small (%lld < %lld)",
                     static_cast<long long>(workspace_bytes), static_cast<long long>(L.total));
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int rc;
  if (M == 0) return rowops::zero_outputs(st, grad_w, N * K, grad_b, grad_b ? N : 0, "cign_linear_bwd");
  auto bias_grad = [&]() -> int {
    if (!grad_b) return kOk;
    float* part = reinterpret_cast<float*>(ws + L.part_b);
    hipLaunchKernelGGL(bias_grad_kernel, dim3((N + 63) / 64, L.chunks), dim3(kThreads), 0, st, grad_y, M, N, L.chunk,
                       part);
    const int r = check_launch("cign_linear_bwd (bias partials)");
    return r ? r : rowops::launch_colsum(st, part, L.chunks, N, 1, grad_b, nullptr, "cign_linear_bwd (bias)");
  };
  if (N <= kSmallN) {
    const bool rb = math == kMathBF16;
    const int K4 = (K + 3) / 4;
    if (grad_x) {
      const dim3 gxg((K4 + 63) / 64, static_cast<unsigned>((M + 3) / 4));
      if (rb)
        hipLaunchKernelGGL(small_n_grad_x_kernel<true>, gxg, dim3(kThreads), 0, st, grad_y, M, N, K, w, grad_x);
      else
        hipLaunchKernelGGL(small_n_grad_x_kernel<false>, gxg, dim3(kThreads), 0, st, grad_y, M, N, K, w, grad_x);
      if ((rc = check_launch("cign_linear_bwd (grad_x, few outputs)"))) return rc;
    }
    float* part = reinterpret_cast<float*>(ws + L.part_w);
    const dim3 grid((K4 + kThreads - 1) / kThreads, L.chunks);
    if (rb)
      hipLaunchKernelGGL(small_n_grad_w_kernel<true>, grid, dim3(kThreads), 0, st, grad_y, x, M, N, K, L.chunk, part);
    else
      hipLaunchKernelGGL(small_n_grad_w_kernel<false>, grid, dim3(kThreads), 0, st, grad_y, x, M, N, K, L.chunk, part);
    if ((rc = check_launch("cign_linear_bwd (grad_W partials, few outputs)"))) return rc;
    if ((rc = rowops::launch_colsum(st, part, L.chunks, N * K, 1, grad_w, nullptr, "cign_linear_bwd (grad_W)")))
      return rc;
    return bias_grad();
  }
  // grad_W [N,K] = grad_y^T x: split-M MFMA partials, then chunk sums.
  {
    const int ntk = (K + kWgT - 1) / kWgT;
    const dim3 grid(static_cast<unsigned>(((N + kWgT - 1) / kWgT) * ntk), static_cast<unsigned>(L.wg_chunks));
    const bool vec = N % 4 == 0 && K % 4 == 0 && aligned16(grad_y) && aligned16(x);
    float* part = reinterpret_cast<float*>(ws + L.part_w);
    if (math == kMathBF16)
      hipLaunchKernelGGL(wgrad_kernel<kMathBF16>, grid, dim3(kThreads), 0, st, grad_y, x, M, N, K, L.wg_chunk, ntk,
                         vec, part);
    else
      hipLaunchKernelGGL(wgrad_kernel<kMathF32>, grid, dim3(kThreads), 0, st, grad_y, x, M, N, K, L.wg_chunk, ntk,
                         vec, part);
    if ((rc = check_launch("cign_linear_bwd (grad_W partials)"))) return rc;
    if ((rc = rowops::launch_colsum(st, part, L.wg_chunks, N * K, 1, grad_w, nullptr, "cign_linear_bwd (grad_W)")))
      return rc;
  }
  if (!grad_x) return bias_grad();
  // grad_x [M,K] = grad_y [M,N] W [N,K] = grad_y (W^T)^T: the forward NT
  // kernel with W^T [K,N] as its weight. Under bf16 math it rounds both
  // operands to bf16 as autocast's backward GEMM reads them; the output stays
  // fp32 (not rounded).
  float* wt = reinterpret_cast<float*>(ws + L.wt);
  hipLaunchKernelGGL(transpose_w_kernel, dim3((K + 31) / 32, (N + 31) / 32), dim3(256), 0, st, w, N, K, wt);
  if ((rc = check_launch("cign_linear_bwd (W^T)"))) return rc;
  GemmArgs g{};
  g.M = M; g.N = K; g.K = N; g.x = grad_y; g.w = wt; g.y = grad_x;
  g.vec = rows_aligned(grad_y, kF32, wt, N);
  g.vec4 = K % 4 == 0 && aligned16(grad_x);
  g.round_bf16 = false;
  if ((rc = dispatch_nt<kEpiStore>(st, g, kF32, math, pick_bn(K, 0, math)))) return rc;
  return bias_grad();
}

}  // extern "C"
