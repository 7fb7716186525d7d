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
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "clifford.h"
#include "gate.h"
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
  bool y_bf16;        // y is bf16 storage (with round_bf16: the same values, exactly)
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
  if constexpr (std::is_same_v<T, float> && N == 2) {
    *reinterpret_cast<float2*>(d) = make_float2(v[0], v[1]);
  } else if constexpr (std::is_same_v<T, float>) {
    static_assert(N == 4, "fp32 LDS chunks are 2 or 4 values");
    *reinterpret_cast<float4*>(d) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (N == 2) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<bf16x2*>(d) = bf16x2{static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1])};
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

// The K step starting at k0 can take the unconditional loads. FULL: the host
// has checked that every step can (aligned rows, K a multiple of kBK), so the
// guarded loads are not compiled: a guarded path in the loop makes the
// compiler wait for every load in flight before the step's MFMAs.
template <bool FULL = false>
__device__ __forceinline__ bool fast_step(const GemmArgs& g, int k0) {
  return FULL || (g.vec && k0 + kBK <= g.K);
}

// One K step's x fragments of a wavefront: its two 16-row tiles.
struct XStep {
  float v[2][8];
};

template <typename TX, int MATH, bool FULL = false>
__device__ __forceinline__ void load_xstep(const GemmArgs& g, const TX* x, int64_t row0, int k0, int lane, XStep& a) {
  const bool fast = fast_step<FULL>(g, k0);
#pragma unroll
  for (int r = 0; r < 2; ++r) load_x<TX, MATH>(g, x, row0 + 16 * r + (lane & 15), k0, lane >> 4, fast, a.v[r]);
}

// W tile of one K step (BN rows x 32) held in registers between the global
// load and the LDS store; all 256 threads share it.
template <int MATH, int BN>
struct WStage {
  static constexpr int CHUNKS = BN * kBK / 4 / kThreads;  // 16-byte fp32 chunks per thread
  float b[CHUNKS][4];

  template <bool FULL = false>
  __device__ __forceinline__ void load(const GemmArgs& g, int n0, int k0) {
    constexpr int CPR = kBK / 4;
    if (fast_step<FULL>(g, k0)) {
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

#ifndef CIGN_GEMM_ASM_MFMA
#define CIGN_GEMM_ASM_MFMA 1
#endif
// MFMAs accumulating in place (vdst == srcC), for the K loops of the
// unguarded (FULL) kernels. With the builtins the compiler allocates each
// result apart from its accumulator and copies it back every iteration (two
// moves per MFMA in the bf16 loop, as many VALU cycles as the MFMAs take);
// here the accumulators stay put. Their operands come straight from global
// or LDS loads, whose waits the compiler inserts; the compiler does not see
// these as MFMAs, so mfma_settle puts the wait states an MFMA result needs
// between the accumulators' initialisation, the K loop and the epilogue.
// The guarded kernels, whose operands pass through selects, keep the
// builtins.
__device__ __forceinline__ void mfma_bf16_acc(f32x4& c, const bf16x8& a, const bf16x8& b) {
  asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_f32_acc(f32x4& c, float a, float b) {
  asm("v_mfma_f32_16x16x4_f32 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}

// Wait states between MFMAs writing the accumulators and any other
// instruction reading or writing them (at most 18 for any MFMA): every
// accumulator passes through an empty statement before and after the nops.
template <int R, int TN>
__device__ __forceinline__ void mfma_settle(f32x4 (&acc)[R][TN]) {
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int f = 0; f < TN; ++f) asm volatile("" : "+v"(acc[r][f]));
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4");
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int f = 0; f < TN; ++f) asm volatile("" : "+v"(acc[r][f]));
}

// One bf16 MFMA, or the four fp32 MFMAs of a 16-wide k chunk (k slices x, y,
// z, w), accumulating into c: in place when ASM (operands from LDS reads).
template <bool ASM>
__device__ __forceinline__ void mma_bf16(f32x4& c, const bf16x8& a, const bf16x8& b) {
  if constexpr (ASM) mfma_bf16_acc(c, a, b);
  else c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <bool ASM>
__device__ __forceinline__ void mma_f32x4(f32x4& c, const float4& a, const float4& b) {
  if constexpr (ASM) {
    mfma_f32_acc(c, a.x, b.x);
    mfma_f32_acc(c, a.y, b.y);
    mfma_f32_acc(c, a.z, b.z);
    mfma_f32_acc(c, a.w, b.w);
  } else {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, c, 0, 0, 0);
  }
}
// Kernels whose MFMA operands all come from LDS reads take the in-place
// form whether or not their global loads are guarded.
constexpr bool kLdsAsm = CIGN_GEMM_ASM_MFMA;

// MFMAs of one K step. The W tile is the MFMA's first operand and x the
// second, so D = W x^T: lane l holds output rows (of y) 16r + l%16 and, per
// 16-column tile f, the four consecutive columns 16f + 4*(l/16) + q.
template <int MATH, int TN, bool ASM = false>
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
          if constexpr (ASM) {
            mfma_f32_acc(acc[r][f], wb.x, xv[0]);
            mfma_f32_acc(acc[r][f], wb.y, xv[1]);
            mfma_f32_acc(acc[r][f], wb.z, xv[2]);
            mfma_f32_acc(acc[r][f], wb.w, xv[3]);
          } else {
            acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.x, xv[0], acc[r][f], 0, 0, 0);
            acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.y, xv[1], acc[r][f], 0, 0, 0);
            acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.z, xv[2], acc[r][f], 0, 0, 0);
            acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.w, xv[3], acc[r][f], 0, 0, 0);
          }
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
// 16r + lane%16 (r < RT) and columns n = n0 + 16f + 4*(lane/16) + q, q < 4.
// Every load here is unconditional, at an index clamped into the tensor
// (values for columns past N or rows past M are never stored): a load behind
// a per-lane branch ends in its own block, and the compiler then waits for
// every memory operation in flight (vmcnt(0)) once per value, 16 to 80 waits
// per workgroup before. Stores stay guarded.
template <int EPI, int TN, int RT = 2>
__device__ __forceinline__ void epilogue_swapped(const GemmArgs& g, f32x4 (&acc)[RT][TN], int64_t row0, int n0,
                                                 int lane) {
  const int cg = (lane >> 4) * 4;
  const int nmax = g.N - 1;
  float bv[TN][4];
  if (g.bias) {
#pragma unroll
    for (int f = 0; f < TN; ++f)
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[f][q] = g.bias[min(n0 + 16 * f + cg + q, nmax)];
  } else {
#pragma unroll
    for (int f = 0; f < TN; ++f)
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[f][q] = 0.0f;
  }
  float gmv[EPI == kEpiGamma ? TN : 1][4];
  if constexpr (EPI == kEpiGamma) {
#pragma unroll
    for (int f = 0; f < TN; ++f)
#pragma unroll
      for (int q = 0; q < 4; ++q) gmv[f][q] = g.gamma[min(n0 + 16 * f + cg + q, nmax)];
  }
#pragma unroll
  for (int f = 0; f < TN; ++f)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      // Autocast casts the bias to bf16 with the other operands.
      if (g.round_bf16) bv[f][q] = round_bf16(bv[f][q]);
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    const int64_t m = row0 + 16 * r + (lane & 15);
    // the residual rows of this r, loaded before any of its stores
    float hv[EPI == kEpiGamma ? TN : 1][4];
    if constexpr (EPI == kEpiGamma) {
      const int64_t mc = m < g.M ? m : g.M - 1;
#pragma unroll
      for (int f = 0; f < TN; ++f) {
        const int nb = n0 + 16 * f + cg;
        if (g.vec4) {
          const float4 t = *reinterpret_cast<const float4*>(g.h + mc * g.N + min(nb, g.N - 4));
          hv[f][0] = t.x; hv[f][1] = t.y; hv[f][2] = t.z; hv[f][3] = t.w;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) hv[f][q] = g.h[mc * g.N + min(nb + q, nmax)];
        }
      }
    }
#pragma unroll
    for (int f = 0; f < TN; ++f) {
      const int nb = n0 + 16 * f + cg;
      const bool full4 = g.vec4 && nb + 4 <= g.N;
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = acc[r][f][q] + bv[f][q];
        if (g.round_bf16) v[q] = round_bf16(v[q]);
        acc[r][f][q] = v[q];
      }
      if (m >= g.M) continue;
      const int64_t o = m * g.N + nb;
      if (g.y_bf16) {
        __bf16* yb = reinterpret_cast<__bf16*>(g.y);
        if (full4) {
          *reinterpret_cast<bf16x4*>(yb + o) = bf16x4{static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1]),
                                                      static_cast<__bf16>(v[2]), static_cast<__bf16>(v[3])};
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (nb + q < g.N) yb[o + q] = static_cast<__bf16>(v[q]);
        }
      } else if (full4) {
        *reinterpret_cast<float4*>(g.y + o) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nb + q < g.N) g.y[o + q] = v[q];
      }
      if constexpr (EPI == kEpiGamma) {
        float ov[4];
        uint8_t mk[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bool keep = block_keep(g.seed, static_cast<uint64_t>(o + q), g.p);
          const float dv = keep ? (g.p > 0.0f ? v[q] / (1.0f - g.p) : v[q]) : 0.0f;
          ov[q] = hv[f][q] + gmv[f][q] * dv;
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
      float ss[RT], sd[RT];
#pragma unroll
      for (int r = 0; r < RT; ++r) ss[r] = sd[r] = 0.0f;
#pragma unroll
      for (int f = 0; f < TN; ++f) {
        if (f < h0 || f >= h0 + fph) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + 16 * f + cg + q;
          // att_* are [H, C] = N values: the clamped index stays inside
          const int64_t ai = min(n, nmax);
          const float asv = g.att_src[ai], adv = g.att_dst[ai];
          const float as = n < g.N ? asv : 0.0f;
          const float ad = n < g.N ? adv : 0.0f;
#pragma unroll
          for (int r = 0; r < RT; ++r) {
            ss[r] = fmaf(acc[r][f][q], as, ss[r]);
            sd[r] = fmaf(acc[r][f][q], ad, sd[r]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int o = 16; o < kWave; o <<= 1) {
          ss[r] += shfl_xor(ss[r], o);
          sd[r] += shfl_xor(sd[r], o);
        }
      if (lane < 16 && head < H) {
#pragma unroll
        for (int r = 0; r < RT; ++r) {
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
template <typename TX, int MATH, int BN, int EPI, bool FULL>
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
  constexpr bool ASM = FULL && CIGN_GEMM_ASM_MFMA && MATH == kMathF32;
  if constexpr (ASM) mfma_settle(acc);
  XStep a0, a1;
  WStage<MATH, BN> wst;
  // With FULL every prefetch is issued, past the end as a repeat of the last
  // step (in bounds, unused), so no load sits behind a branch and each wait
  // covers only the loads it needs.
  const int last = (nk - 1) * kBK;
  load_xstep<TX, MATH, FULL>(g, x, row0, 0, lane, a0);
  if (FULL || nk > 1) load_xstep<TX, MATH, FULL>(g, x, row0, min(kBK, last), lane, a1);
  wst.template load<FULL>(g, n0, 0);
  wst.store(Bs[0]);
  __syncthreads();
  int buf = 0;
  for (int s = 0; s < nk; s += 2) {
    if (FULL || s + 1 < nk) wst.template load<FULL>(g, n0, min((s + 1) * kBK, last));
    // keep the W loads ahead of the MFMAs (the scheduler sinks them below,
    // exposing their latency at the LDS store)
    __builtin_amdgcn_sched_barrier(0);
    mma_step<MATH, TN, ASM>(a0, Bs[buf], lane, acc);
    if (FULL || s + 2 < nk) load_xstep<TX, MATH, FULL>(g, x, row0, min((s + 2) * kBK, last), lane, a0);
    if (FULL || s + 1 < nk) wst.store(Bs[buf ^ 1]);
    __syncthreads();
    buf ^= 1;
    if (s + 1 >= nk) break;  // uniform
    if (FULL || s + 2 < nk) wst.template load<FULL>(g, n0, min((s + 2) * kBK, last));
    __builtin_amdgcn_sched_barrier(0);
    mma_step<MATH, TN, ASM>(a1, Bs[buf], lane, acc);
    if (FULL || s + 3 < nk) load_xstep<TX, MATH, FULL>(g, x, row0, min((s + 3) * kBK, last), lane, a1);
    if (FULL || s + 2 < nk) wst.store(Bs[buf ^ 1]);
    __syncthreads();
    buf ^= 1;
  }

  if constexpr (ASM) mfma_settle(acc);
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

  template <bool FULL = false>
  __device__ __forceinline__ void load(const GemmArgs& g, const TX* x, int64_t m0, int n0, int k0) {
    constexpr int ACPR = kBK / XC;  // chunks per A row
    if (fast_step<FULL>(g, k0)) {
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
template <int MATH, int TN, bool ASM = false>
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
        for (int r = 0; r < 2; ++r) {
          if constexpr (ASM) mfma_bf16_acc(acc[r][f], b, a[r]);
          else acc[r][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, a[r], acc[r][f], 0, 0, 0);
        }
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


template <typename TX, int MATH, int BN, int EPI, bool FULL>
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

  constexpr bool ASM = FULL && CIGN_GEMM_ASM_MFMA && MATH == kMathBF16;
  if constexpr (ASM) mfma_settle(acc);
  LdsStage<TX, MATH, BN> regs;
  regs.template load<FULL>(g, x, m0, n0, 0);
  regs.store(As[0], Bs[0]);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < g.K; k0 += kBK) {
    // with FULL the last step loads itself again (in bounds, unused): no
    // load behind a branch
    const bool more = k0 + kBK < g.K;
    if (FULL || more) regs.template load<FULL>(g, x, m0, n0, more ? k0 + kBK : k0);
    __builtin_amdgcn_sched_barrier(0);  // the next step's loads ahead of the MFMAs,
    mma_step_lds<MATH, TN, ASM>(As[buf], Bs[buf], wave, lane, acc);
    __builtin_amdgcn_sched_barrier(0);  // and the MFMAs ahead of the wait for them
    if (FULL || more) regs.store(As[buf ^ 1], Bs[buf ^ 1]);
    __syncthreads();
    buf ^= 1;
  }

  if constexpr (ASM) mfma_settle(acc);
  epilogue_swapped<EPI, TN>(g, acc, m0 + wave * kRowsPerWave, n0, lane);
}

// ---------------------------------------------------------------------------
// bf16 math, K <= 256: x fragments resident in registers
// ---------------------------------------------------------------------------
// For M >> N with a short K (the GAT lin of the production block, 24.5K x 256
// -> 1536) the 128 x BN tiles above fetch each x row once per column tile (12
// times at N = 1536, 300 MB of L2 reads for a 25 MB input). Here a workgroup
// owns 128 rows and a run of column tiles: each wavefront converts its 32 x
// rows to bf16 MFMA fragments once, for all of K, and keeps them in registers
// (K/4 VGPRs) while the workgroup streams the W tiles of its columns through
// LDS (64 columns x 64 k per stage, converted at the LDS store, double
// buffered, one stage of loads in flight across tile boundaries). Every
// output takes the same MFMA sequence as in gemm_nt_lds_kernel (K steps of
// 32 in order from zero, W the first operand), so the results are identical.
constexpr int kXrBN = 64;          // columns per tile (each wavefront: its 32 rows x all 64)
constexpr int kXrKC = 64;          // k per W stage
constexpr int kXrLS = kXrKC + 16;  // LDS row stride in bf16: 160 B, 8 x odd floats
constexpr int kXrMaxK = 256;
constexpr int kXrPerCu = 3;        // workgroups per CU the grid is sized for
constexpr int kXrMaxTiles = 16;    // column tiles per workgroup (its bias slice in LDS)

// fp32-y epilogue of gemm_nt_xres_kernel: the wavefront's 32 x 64 output tile
// passes through LDS, 16 rows at a time, so that every global store writes
// whole lines (4 rows x 256 B an instruction, against 16 rows x 64 B for the
// swapped layout's own stores). Its stores go out at the end of the tile, so
// the next tile's first W wait also waits for them; bf16 y takes the deferred
// path below instead. E: this wavefront's 16 x kXrES floats; LDS operations
// of one wavefront run in order, so its staged rows need no barrier.
constexpr int kXrES = 72;  // staged row stride in floats: 288 B, 8 x odd

__device__ __forceinline__ void xres_epilogue(const GemmArgs& g, f32x4 (&acc)[2][kXrBN / 16], int64_t row0, int n0,
                                              int lane, const float* bias, float* E) {
  constexpr int TN = kXrBN / 16;
  const int cg = (lane >> 4) * 4;
  float bv[TN][4];
#pragma unroll
  for (int f = 0; f < TN; ++f) {
    const float4 t = *reinterpret_cast<const float4*>(bias + 16 * f + cg);
    bv[f][0] = t.x; bv[f][1] = t.y; bv[f][2] = t.z; bv[f][3] = t.w;
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
#pragma unroll
    for (int f = 0; f < TN; ++f) {
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = acc[r][f][q] + bv[f][q];
        if (g.round_bf16) v[q] = round_bf16(v[q]);
      }
      *reinterpret_cast<float4*>(E + (lane & 15) * kXrES + 16 * f + cg) = make_float4(v[0], v[1], v[2], v[3]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = lane + kWave * i;
      const int rr = id / 16, c = id % 16;
      const float4 a = *reinterpret_cast<const float4*>(E + rr * kXrES + 4 * c);
      const int64_t m = row0 + 16 * r + rr;
      const int n = n0 + 4 * c;
      if (m >= g.M) continue;
      if (g.vec4 && n + 4 <= g.N) {
        *reinterpret_cast<float4*>(g.y + m * g.N + n) = a;
      } else {
        const float v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < g.N) g.y[m * g.N + n + q] = v[q];
      }
    }
  }
}

// bf16 y: the wavefront's 32 x 64 tile is staged in LDS as bf16 (row stride
// kXrEB) and stored as four instructions of 8 rows x 128 B, issued during the
// next column tile's W stages, each right after that stage's W loads.
// Stores and loads share one in-order counter (vmcnt), so a load issued after
// a store cannot be waited for without waiting for the store: stores issued
// in a block at the end of a tile made the next tile's first W wait take
// their acknowledgements (24 of 57 us at N = 1536). Interleaved this way, the
// wait at the end of each stage covers only the stores of the stage before.
constexpr int kXrEB = 80;  // staged bf16 row stride: 160 B, 8 x odd floats

__device__ __forceinline__ void xres_stage_bf16(f32x4 (&acc)[2][kXrBN / 16], const float* bias, int lane,
                                                __bf16* E) {
  constexpr int TN = kXrBN / 16;
  const int cg = (lane >> 4) * 4;
#pragma unroll
  for (int f = 0; f < TN; ++f) {
    const float4 bv = *reinterpret_cast<const float4*>(bias + 16 * f + cg);
#pragma unroll
    for (int r = 0; r < 2; ++r)
      *reinterpret_cast<bf16x4*>(E + (16 * r + (lane & 15)) * kXrEB + 16 * f + cg) =
          bf16x4{static_cast<__bf16>(acc[r][f][0] + bv.x), static_cast<__bf16>(acc[r][f][1] + bv.y),
                 static_cast<__bf16>(acc[r][f][2] + bv.z), static_cast<__bf16>(acc[r][f][3] + bv.w)};
  }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Store instruction i (< 4) of a staged tile: rows 8i .. 8i+7 of the
// wavefront's 32, lane: row 8i + lane/8, columns n0 + 8 (lane%8) .. +7.
// mlim: rows at or past it are not stored (0 before the first tile).
// YB == 2 (N % 8 == 0, aligned, y under 2 GiB): one buffer store with no
// branch, rows past mlim and columns past N sent past the buffer's end (the
// hardware drops them), so the count of memory operations after each stage's loads is the
// same on every path and the stage's wait can leave the store in flight.
// YB == 1: guarded stores.
template <int YB>
__device__ __forceinline__ void xres_store_bf16(const GemmArgs& g, __amdgpu_buffer_rsrc_t yr, int64_t row0, int64_t mlim,
                                                int n0, int lane, const __bf16* E, int i) {
  const int rr = 8 * i + lane / 8, c = lane % 8;
  const bf16x8 t = *reinterpret_cast<const bf16x8*>(E + rr * kXrEB + 8 * c);
  const int64_t m = row0 + rr;
  const int n = n0 + 8 * c;
  if constexpr (YB == 2) {
    // (N % 8 == 0: a chunk lies wholly inside or wholly past the row)
    const uint32_t off = m < mlim && n < g.N ? static_cast<uint32_t>((m * g.N + n) * 2) : 0x80000000u;
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, t), yr, off, 0, 0);
  } else {
    if (m >= mlim) return;
    __bf16* yb = reinterpret_cast<__bf16*>(g.y) + m * g.N + n;
    if (g.vec4 && g.N % 8 == 0 && n + 8 <= g.N) {
      *reinterpret_cast<bf16x8*>(yb) = t;
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q)
        if (n + q < g.N) yb[q] = t[q];
    }
  }
}

// W stage registers between the global load and the LDS store: 256 threads
// x 4 chunks of 4 fp32 (16 threads a row). Stage j: column tile ct0 + j /
// STAGES, k0 = 64 (j % STAGES); rows past N read row N-1 (never stored).
struct XrWf32 {
  float v[4][4];
  __device__ __forceinline__ void load(const GemmArgs& g, int n0, int k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int n = n0 + id / 16;
      gload_fast<float, 4>(g.w + static_cast<int64_t>(n < g.N ? n : g.N - 1) * g.K, k0 + 4 * (id % 16), v[i]);
    }
  }
  __device__ __forceinline__ void store(__bf16* d) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = threadIdx.x + i * kThreads;
      st_lds<__bf16, 4>(d + (id / 16) * kXrLS + 4 * (id % 16), v[i]);
    }
  }
};

// (K = 192 keeps two waves a SIMD: three would spill)
template <typename TX, int KS, int YB>
__global__ __launch_bounds__(kThreads, KS == 6 ? 2 : kXrPerCu) void gemm_nt_xres_kernel(GemmArgs g, int nrt, int ncg, int tpg) {
  static_assert(KS % 2 == 0 && KS * kBK <= kXrMaxK, "K is a multiple of 64, at most 256");
  constexpr int STAGES = KS * kBK / kXrKC;  // W stages per column tile
  constexpr int TN = kXrBN / 16;
  using WReg = XrWf32;
  __shared__ __align__(16) __bf16 Ws[2][kXrBN * kXrLS];
  // per wavefront: 16 x kXrES floats (fp32 y) or 32 x kXrEB bf16 (bf16 y)
  constexpr int kEsFloats = 32 * kXrEB / 2 > 16 * kXrES ? 32 * kXrEB / 2 : 16 * kXrES;
  __shared__ __align__(16) float Es[kThreads / kWave][kEsFloats];
  // the bias of the group's columns (bf16-rounded under autocast, 0 without
  // one), so that the epilogues issue no global loads
  __shared__ __align__(16) float Bias[kXrMaxTiles * kXrBN];
  const int lane = lane_id();
  const int wave = wave_id();
  int rt, cg;
  tile_of(nrt, ncg, rt, cg);
  const int nct = (g.N + kXrBN - 1) / kXrBN;
  const int ct0 = cg * tpg;
  const int ct1 = min(ct0 + tpg, nct);
  const int nsteps = (ct1 - ct0) * STAGES;  // >= STAGES: the host gives every group a tile
  const int64_t row0 = static_cast<int64_t>(rt) * kBM + wave * kRowsPerWave;
  const TX* x = static_cast<const TX*>(g.x);
  // stages past the last reload the last (in bounds, never stored)
  auto wload = [&](WReg& w, int j) __attribute__((always_inline)) {
    j = min(j, nsteps - 1);
    w.load(g, (ct0 + j / STAGES) * kXrBN, (j % STAGES) * kXrKC);
  };

  for (int t = threadIdx.x; t < (ct1 - ct0) * kXrBN; t += kThreads) {
    const int n = ct0 * kXrBN + t;
    const float b = g.bias ? g.bias[n < g.N ? n : g.N - 1] : 0.0f;
    Bias[t] = g.round_bf16 ? round_bf16(b) : b;
  }
  WReg w0;  // stage 0, stored to LDS after the x loads
  wload(w0, 0);
  // x fragments (rows past M read row M-1; their outputs are never stored),
  // in two halves of K to bound the fp32 staging registers
  bf16x8 xf[2][KS];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float v[2][KS / 2][8];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int s = 0; s < KS / 2; ++s)
        load_x<TX, kMathBF16>(g, x, row0 + 16 * r + (lane & 15), (h * KS / 2 + s) * kBK, lane >> 4, true, v[r][s]);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int s = 0; s < KS / 2; ++s)
#pragma unroll
        for (int q = 0; q < 8; ++q) xf[r][h * KS / 2 + s][q] = static_cast<__bf16>(v[r][s][q]);
  }
  w0.store(Ws[0]);
  __syncthreads();

  f32x4 acc[2][TN];
  const int rl = lane & 15, ks = lane >> 4;
  __bf16* Eb = reinterpret_cast<__bf16*>(Es[wave]);
  // y as a buffer of M N bf16 (used when YB == 2; the host checks it is under 2 GiB)
  const __amdgpu_buffer_rsrc_t yr =
      __builtin_amdgcn_make_buffer_rsrc(g.y, 0, YB == 2 ? static_cast<int>(g.M * g.N * 2) : 0, 0x00020000);
  int64_t mlim = 0;  // row limit of the staged tile's stores (0: nothing staged)
  int pend_n0 = 0;   // its first column

  // Stage st of column tile ct: the loads of stage j + 1 go out, then a share
  // of the previous tile's stores, the MFMAs on stage j, and stage j + 1 goes
  // to LDS.
  auto stage = [&](int ct, int st) __attribute__((always_inline)) {
    const int j = (ct - ct0) * STAGES + st;
    WReg nw;
    wload(nw, j + 1);
    if constexpr (YB != 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i * STAGES / 4 == st) xres_store_bf16<YB>(g, yr, row0, mlim, pend_n0, lane, Eb, i);
    }
    __builtin_amdgcn_sched_barrier(0);  // the next stage's loads ahead of the MFMAs
    const __bf16* B = Ws[j & 1];
#pragma unroll
    for (int sub = 0; sub < kXrKC / kBK; ++sub) {
#pragma unroll
      for (int f = 0; f < TN; ++f) {
        const bf16x8 wb = *reinterpret_cast<const bf16x8*>(B + (16 * f + rl) * kXrLS + sub * kBK + ks * 8);
#pragma unroll
        for (int r = 0; r < 2; ++r) mfma_bf16_acc(acc[r][f], wb, xf[r][st * (kXrKC / kBK) + sub]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // and the MFMAs ahead of the wait for them
    nw.store(Ws[(j + 1) & 1]);
    __syncthreads();
  };

  for (int ct = ct0; ct < ct1; ++ct) {
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int f = 0; f < TN; ++f) acc[r][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    mfma_settle(acc);
#pragma unroll
    for (int st = 0; st < STAGES; ++st) stage(ct, st);
    mfma_settle(acc);
    if constexpr (YB != 0) {
      xres_stage_bf16(acc, Bias + (ct - ct0) * kXrBN, lane, Eb);
      mlim = g.M;
      pend_n0 = ct * kXrBN;
    } else {
      xres_epilogue(g, acc, row0, ct * kXrBN, lane, Bias + (ct - ct0) * kXrBN, Es[wave]);
    }
  }
  if constexpr (YB != 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) xres_store_bf16<YB>(g, yr, row0, mlim, pend_n0, lane, Eb, i);
  }
}

// CUs of the current device, cached per device.
inline int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  cache[dev].store(v, std::memory_order_relaxed);
  return v;
}

// CIGN_GEMM_XRES=0 (read at each call) keeps these shapes on
// gemm_nt_lds_kernel, for comparisons.
inline bool xres_enabled() {
  const char* e = std::getenv("CIGN_GEMM_XRES");
  return !(e && e[0] == '0');
}

// bf16 y the x-resident kernel can store with branch-free buffer stores
inline bool xres_buffer_y(const GemmArgs& g) { return g.vec4 && g.N % 8 == 0 && g.M * g.N * 2 < 0x80000000LL; }

template <typename TX>
int launch_xres(hipStream_t st, const GemmArgs& g) {
  const int nrt = static_cast<int>((g.M + kBM - 1) / kBM);
  const int nct = (g.N + kXrBN - 1) / kXrBN;
  // column groups so that the grid fills kXrPerCu workgroups per CU (each
  // group re-reads its rows of x once); every group gets at least one tile
  const int64_t slots = static_cast<int64_t>(kXrPerCu) * device_cus();
  int ncg = static_cast<int>(std::min<int64_t>(nct, std::max<int64_t>(1, (slots + nrt - 1) / nrt)));
  ncg = std::max(ncg, (nct + kXrMaxTiles - 1) / kXrMaxTiles);
  const int tpg = (nct + ncg - 1) / ncg;
  ncg = (nct + tpg - 1) / tpg;
  const int64_t blocks = static_cast<int64_t>(nrt) * ncg;
  if (blocks > 0x7fffffff) return set_error(kInvalid, "cign linear: too many tiles");
  const dim3 grid(static_cast<unsigned>(blocks));
  auto go = [&](auto YBC) {
    constexpr int YB = decltype(YBC)::value;
    switch (g.K / kBK) {
      case 2: hipLaunchKernelGGL((gemm_nt_xres_kernel<TX, 2, YB>), grid, dim3(kThreads), 0, st, g, nrt, ncg, tpg); break;
      case 4: hipLaunchKernelGGL((gemm_nt_xres_kernel<TX, 4, YB>), grid, dim3(kThreads), 0, st, g, nrt, ncg, tpg); break;
      case 6: hipLaunchKernelGGL((gemm_nt_xres_kernel<TX, 6, YB>), grid, dim3(kThreads), 0, st, g, nrt, ncg, tpg); break;
      default: hipLaunchKernelGGL((gemm_nt_xres_kernel<TX, 8, YB>), grid, dim3(kThreads), 0, st, g, nrt, ncg, tpg);
    }
  };
  if (!g.y_bf16) go(std::integral_constant<int, 0>());
  else if (xres_buffer_y(g)) go(std::integral_constant<int, 2>());
  else go(std::integral_constant<int, 1>());
  return check_launch("cign linear (x-resident)");
}

// ---------------------------------------------------------------------------

// ---------------------------------------------------------------------------
// Backward helpers
// ---------------------------------------------------------------------------
// part[c][n] = sum of grad_y rows of chunk c (a workgroup: 64 columns x 4 row
// slices, four accumulators per thread, slices combined in order). With rb
// (bf16 autocast) each grad_y value is rounded to bf16 first: the bf16
// Linear's backward sums its bf16 incoming gradient.
__global__ __launch_bounds__(kThreads) void bias_grad_kernel(const float* gy, int64_t M, int N, int64_t chunk,
                                                             float* part, bool rb) {
  __shared__ float red[kThreads];
  const int t = threadIdx.x;
  const int n = blockIdx.x * 64 + (t & 63);
  const int s = t >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * chunk;
  const int64_t r1 = r0 + chunk < M ? r0 + chunk : M;
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
  if (n < N) {
    int64_t r = r0 + s;
    auto v = [&](int64_t i) { const float t = gy[i * N + n]; return rb ? round_bf16(t) : t; };
    for (; r + 12 < r1; r += 16) {
      a0 += v(r);
      a1 += v(r + 4);
      a2 += v(r + 8);
      a3 += v(r + 12);
    }
    for (; r < r1; r += 4) a0 += v(r);
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
  // 128 columns x 32 rows of one operand: 1024 four-value chunks, four per
  // thread. Thread id takes row id / 8 and column quads id % 8 + 8i, so a
  // wavefront's load covers 8 rows x 128 contiguous values. The source is
  // fp32, or bf16 storage (TS = bf16h, four values per 8-byte load).
  float v[4][4];
  template <typename TS = float>
  __device__ __forceinline__ void load(const TS* src, int64_t ld, int64_t m0, int64_t m1, int c0, int cmax,
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
        Chunk<TS, 4>::load(src + m * ld + c0 + c, v[i]);
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = ((threadIdx.x % 8) + 8 * i) * 4;
      const TS* p = src + (ok ? m : 0) * ld + c0 + c;
      if (vec && ok && c0 + c + 4 <= cmax) {
        Chunk<TS, 4>::load(p, v[i]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[i][q] = (ok && c0 + c + q < cmax) ? to_f32(p[q]) : 0.0f;
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

// Workgroup -> (tile, row chunk) of the split-M weight-gradient kernels.
// Workgroup ids go round-robin over the 8 XCDs. With `xcd` (bf16 operands),
// a one-dimensional grid of `tiles` x (row chunks rounded up to 8) gives
// every tile of a row chunk to one XCD, so the chunk's rows of both operands
// reach that XCD's L2 once and its tiles share them: at the production block
// (M = 24.5K, 24 tiles) grad_W of proj took 155 against 169 us, the pack
// projection's backward 302 against 313 us. fp32 operands (twice the LDS,
// two workgroups per CU) ran slower that way (446 against 391 us, and 16
// chunks to avoid a second round still 433), so they keep chunk-major ids.
// False for the padding workgroups.
__device__ __forceinline__ bool wg_tile_chunk(int tiles, int chunks, bool xcd, int& tile, int& chunk) {
  if (xcd) {
    const int x = blockIdx.x % 8, j = blockIdx.x / 8;
    chunk = (j / tiles) * 8 + x;
    tile = j % tiles;
  } else {
    chunk = blockIdx.x / tiles;
    tile = blockIdx.x % tiles;
  }
  return chunk < chunks;
}
inline unsigned wg_grid(int tiles, int chunks, bool xcd) {
  return static_cast<unsigned>(tiles * (xcd ? (chunks + 7) / 8 * 8 : chunks));
}
// Row chunks of those kernels: about `target`; with `xcd` a multiple of 8
// (one per XCD each round) once there are at least 8.
inline int64_t wg_chunk_count(int64_t M, int64_t target, bool xcd) {
  const int64_t c = std::max<int64_t>(1, std::min<int64_t>((M + 255) / 256, target));
  return xcd && c >= 8 ? (c + 7) / 8 * 8 : c;
}

// gy: fp32, or bf16 storage (TG = bf16h: a gradient the caller has rounded to
// bf16, as bf16 math rounds it anyway).
template <int MATH, typename TG = float>
__global__ __launch_bounds__(kThreads) void wgrad_kernel(const TG* gy, const float* x, int64_t M, int N, int K,
                                                         int64_t chunk, int nchunks, int ntk, bool vec, float* part) {
  constexpr bool kXcd = MATH == kMathBF16;
  using T = typename Op<MATH>::T;
  using Lay = WgLayout<MATH>;
  __shared__ __align__(16) T Gs[2][kWgT * kWgM];
  __shared__ __align__(16) T Xs[2][kWgT * kWgM];
  const int lane = lane_id();
  const int wave = wave_id();
  int tile, cy;
  if (!wg_tile_chunk(((N + kWgT - 1) / kWgT) * ntk, nchunks, kXcd, tile, cy)) return;  // whole workgroup
  const int n0 = (tile / ntk) * kWgT, k0 = (tile % ntk) * kWgT;
  const int64_t m0 = static_cast<int64_t>(cy) * chunk;
  const int64_t m1 = m0 + chunk < M ? m0 + chunk : M;
  const int wn = (wave >> 1) * 64, wk = (wave & 1) * 64;  // the wave's 64 x 64 quadrant
  const int rl = lane & 15, ks = lane >> 4;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (kLdsAsm) mfma_settle(acc);

  WgStage<MATH> sg, sx;
  sg.template load<TG>(gy, N, m0, m1, n0, N, vec);
  sx.load(x, K, m0, m1, k0, K, vec);
  sg.store(Gs[0]);
  sx.store(Xs[0]);
  __syncthreads();
  int buf = 0;
  for (int64_t mb = m0; mb < m1; mb += kWgM) {
    const bool more = mb + kWgM < m1;
    if (more) {
      sg.template load<TG>(gy, N, mb + kWgM, m1, n0, N, vec);
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
        for (int j = 0; j < 4; ++j) mma_bf16<kLdsAsm>(acc[i][j], gb, xb[j]);
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
          for (int j = 0; j < 4; ++j) mma_f32x4<kLdsAsm>(acc[i][j], gb, xb[j]);
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
  if constexpr (kLdsAsm) mfma_settle(acc);
  // lane holds grad_W rows n = n0 + wn + 16i + 4*(lane/16) + q of column
  // k = k0 + wk + 16j + lane%16
  float* out = part + static_cast<int64_t>(cy) * N * K;
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

// ---- Narrow projections (kSmallN < N <= 64 outputs: the c2 GAT lin, 300 -> 64)
// The 128-row tiles above leave such a shape short of work: at the c2 lin
// (M = 24,492) 192 workgroups, under one wavefront per SIMD, each a chain of
// ten dependent K steps. Here a workgroup owns 32 rows and all (at most 64)
// columns; wavefront w owns column tile w (16 columns) over all of K. The
// 32 rows of x are one contiguous block of memory, staged through LDS in
// chunks of 128 k by fully coalesced 16-byte loads (a direct fragment load
// touches 16 rows per instruction and kept the texture units, not the
// MFMAs, busy); W fragments come straight from L2, clamped in K where the
// staged x is zero.
constexpr int kNarrowN = 64;
constexpr int kNarrowRows = 32;
constexpr int kNarrowKC = 128;             // k per staged chunk (four K steps)
constexpr int kNarrowLS = kNarrowKC + 8;   // LDS row stride: 136 = 8 x odd (mod 64): the fastest fragment reads

// W fragment of one K step for the wave's 16-column tile, laid out as the LDS
// tile reads of mma_step give them: lane l holds W row n0 + l%16 (row N-1
// past N: output columns that are never stored) at k0 + 4*(l/16) .. +3 and
// k0 + 16 + 4*(l/16) .. +3 (fp32 math) or k0 + 8*(l/16) .. +7 (bf16 math).
// With `clamp` (aligned rows, K % 4 == 0) offsets past K read the row's last
// four values instead: their products meet staged x values of zero.
template <int MATH>
__device__ __forceinline__ void load_wfrag(const GemmArgs& g, int n0, int k0, int lane, bool clamp, float (&w)[8]) {
  const int rl = lane & 15, ks = lane >> 4;
  const int ka = MATH == kMathBF16 ? k0 + 8 * ks : k0 + 4 * ks;
  const int kb = MATH == kMathBF16 ? ka + 4 : ka + 16;
  const int n = n0 + rl;
  const float* p = g.w + static_cast<int64_t>(n < g.N ? n : g.N - 1) * g.K;
  float lo[4], hi[4];
  if (clamp) {
    gload_fast<float, 4>(p, min(ka, g.K - 4), lo);
    gload_fast<float, 4>(p, min(kb, g.K - 4), hi);
  } else {
    gload<float, 4>(p, true, ka, g.K, false, lo);
    gload<float, 4>(p, true, kb, g.K, false, hi);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    w[q] = lo[q];
    w[4 + q] = hi[q];
  }
}

// The MFMAs of one K step for one 16-column tile (mma_step's products, W the
// first operand); bf16 math rounds both operands to bf16 here.
template <int MATH>
__device__ __forceinline__ void mma_direct(const XStep& a, const float (&w)[8], f32x4 (&acc)[2][1]) {
  if constexpr (MATH == kMathBF16) {
    bf16x8 wb;
#pragma unroll
    for (int q = 0; q < 8; ++q) wb[q] = static_cast<__bf16>(w[q]);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      bf16x8 xa;
#pragma unroll
      for (int q = 0; q < 8; ++q) xa[q] = static_cast<__bf16>(a.v[r][q]);
      acc[r][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb, xa, acc[r][0], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          acc[r][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[4 * h + q], a.v[r][4 * h + q], acc[r][0], 0, 0, 0);
  }
}

// Four x values of the staged tile as fp32 (zero past M or K).
template <typename TX>
__device__ __forceinline__ void xload4(const TX* p, bool vec, int64_t m, int64_t M, int k, int K, float (&v)[4]) {
  if constexpr (std::is_same_v<TX, float>) {
    if (vec && m < M && k + 4 <= K) {
      const float4 t = *reinterpret_cast<const float4*>(p);
      v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
      return;
    }
  } else {
    if (vec && m < M && k + 4 <= K) {
      const uint2 t = *reinterpret_cast<const uint2*>(p);
      v[0] = __uint_as_float(t.x << 16); v[1] = __uint_as_float(t.x & 0xffff0000u);
      v[2] = __uint_as_float(t.y << 16); v[3] = __uint_as_float(t.y & 0xffff0000u);
      return;
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = (m < M && k + q < K) ? to_f32(p[q]) : 0.0f;
}

// Four x values at k of row m for the aligned path (`vec`: rows 16-byte
// (fp32) or 8-byte (bf16) aligned, K % 4 == 0): the row is clamped to M - 1
// (its products land in output rows that are never stored) and the offset to
// K - 4; the LDS store writes zeros for k >= K (a select once the data is
// there: zeroing the registers here would wait for the load).
template <typename TX>
__device__ __forceinline__ void xload4_vec(const TX* x, int64_t m, int64_t M, int k, int K, float (&v)[4]) {
  const int64_t mc = m < M ? m : M - 1;
  const int kc = k < K ? k : K - 4;
  if constexpr (std::is_same_v<TX, float>) {
    const float4 t = *reinterpret_cast<const float4*>(x + mc * K + kc);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
    const uint2 t = *reinterpret_cast<const uint2*>(x + mc * K + kc);
    v[0] = __uint_as_float(t.x << 16); v[1] = __uint_as_float(t.x & 0xffff0000u);
    v[2] = __uint_as_float(t.y << 16); v[3] = __uint_as_float(t.y & 0xffff0000u);
  }
}

// The loop issues the next chunk's loads (its W fragments, then its x) before
// the current chunk's MFMAs, which read only LDS and W fragments that arrived
// during the previous chunk: the loads wait once per chunk, at the LDS store,
// so a chunk's memory latency overlaps the previous chunk's MFMAs. (Loads
// return in issue order, so a W fragment issued after the x loads could not
// be waited for without them.) VEC: the aligned path (g.vec), branch-free.
template <typename TX, int MATH, int EPI, bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_nt_narrow_kernel(GemmArgs g) {
  __shared__ __align__(16) float xs[2][kNarrowRows * kNarrowLS];  // 34.8 KB
  constexpr int SPC = kNarrowKC / kBK;                             // K steps per chunk (4)
  const int lane = lane_id();
  const int n0 = 16 * __builtin_amdgcn_readfirstlane(wave_id());  // wave-uniform
  const int rl = lane & 15, ks = lane >> 4;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kNarrowRows;
  const TX* x = static_cast<const TX*>(g.x);
  // g.vec: x and W rows start 16-byte (fp32) / 8-byte (bf16) aligned and
  // K % 4 == 0, so W offsets clamp to the row's last aligned quad
  const bool clamp = VEC || (g.vec && g.K % 4 == 0);
  constexpr int CPT = kNarrowRows * kNarrowKC / 4 / kThreads;  // four-value chunks per thread and chunk (4)
  float st[CPT][4];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id / (kNarrowKC / 4), k = c * kNarrowKC + 4 * (id % (kNarrowKC / 4));
      const int64_t m = row0 + r;
      if constexpr (VEC)
        xload4_vec<TX>(x, m, g.M, k, g.K, st[i]);
      else
        xload4<TX>(x + (m < g.M ? m : 0) * g.K + k, g.vec, m, g.M, k, g.K, st[i]);
    }
  };
  auto store_chunk = [&](int c, float* d) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id / (kNarrowKC / 4), k = 4 * (id % (kNarrowKC / 4));
      const bool in = !VEC || c * kNarrowKC + k < g.K;
      *reinterpret_cast<float4*>(d + r * kNarrowLS + k) =
          in ? make_float4(st[i][0], st[i][1], st[i][2], st[i][3]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  // the W fragments of chunk c's K steps (offsets past K clamped or zero)
  auto load_w = [&](int c, float (&w)[SPC][8]) {
#pragma unroll
    for (int t = 0; t < SPC; ++t) load_wfrag<MATH>(g, n0, (c * SPC + t) * kBK, lane, clamp, w[t]);
  };
  f32x4 acc[2][1];
  acc[0][0] = acc[1][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int nk = (g.K + kBK - 1) / kBK;
  const int nchunks = (g.K + kNarrowKC - 1) / kNarrowKC;
  // chunk c's MFMAs; `tail`: the last chunk, whose K steps past K are skipped
  auto compute = [&](int c, const float (&w)[SPC][8], bool tail) {
    const float* X = xs[c & 1];
#pragma unroll
    for (int t = 0; t < SPC; ++t) {
      if (!tail || c * SPC + t < nk) {  // uniform
        XStep a;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const float* xr = X + (16 * r + rl) * kNarrowLS + t * kBK;
          const int ka = MATH == kMathBF16 ? 8 * ks : 4 * ks;
          const int kb = MATH == kMathBF16 ? ka + 4 : ka + 16;
          const float4 lo = *reinterpret_cast<const float4*>(xr + ka);
          const float4 hi = *reinterpret_cast<const float4*>(xr + kb);
          a.v[r][0] = lo.x; a.v[r][1] = lo.y; a.v[r][2] = lo.z; a.v[r][3] = lo.w;
          a.v[r][4] = hi.x; a.v[r][5] = hi.y; a.v[r][6] = hi.z; a.v[r][7] = hi.w;
        }
        mma_direct<MATH>(a, w[t], acc);
      }
    }
  };
  // a chunk that is not the last: the next chunk's loads in flight, this
  // chunk's MFMAs, then the next chunk's x into the other buffer. No branch
  // around the loads, so the only wait on them is at the LDS store.
  auto step = [&](int c, const float (&wcur)[SPC][8], float (&wnext)[SPC][8]) {
    load_w(c + 1, wnext);
    load_chunk(c + 1);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
    compute(c, wcur, false);
    __builtin_amdgcn_sched_barrier(0);  // the store's wait for x after the MFMAs
    store_chunk(c + 1, xs[(c + 1) & 1]);
    __syncthreads();
  };
  float wa[SPC][8], wb[SPC][8];
  load_w(0, wa);
  load_chunk(0);
  store_chunk(0, xs[0]);
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  int c = 0;
  for (; c + 2 < nchunks; c += 2) {
    step(c, wa, wb);
    step(c + 1, wb, wa);
  }
  if (c + 1 < nchunks) {
    step(c, wa, wb);
    compute(c + 1, wb, true);
  } else {
    compute(c, wa, true);
  }
  if (n0 < g.N) epilogue_swapped<EPI, 1>(g, acc, row0, n0, lane);
}

// ---- Narrow fp32 projections with W in registers (128 <= K <= 304)
// The kernel above reads each workgroup's W fragments from L2 per K step and
// syncs per chunk. Here each wavefront loads the W fragments of its
// 16-column tile for all of K once (NB = K/16 rounded up float4 per lane:
// lane l holds W[16 w + l%16][16 b + 4*(l/16) .. +3] for block b) and keeps
// them in registers, and the workgroup walks 16-row x tiles t = blockIdx.x,
// + gridDim.x, ..., double-buffered in LDS: the next tile's loads are issued
// before the current tile's MFMAs, which read one float4 of LDS per four
// 16 x 16 x 4 MFMAs (x value q of the lane's quad is k-slot l/16 of MFMA q,
// as in the W fragment, so the products pair up; two accumulators). Three
// workgroups per CU (three wavefronts per SIMD) cover one another's
// stores, epilogues and barriers. K is zero-padded to whole 16-k blocks; W
// rows past N are zero. Needs g.vec (rows 16-byte aligned, K % 4 == 0).
// Measured at the c2 lin (24,492 x 300 -> 64, fp32): 17.3 us against 18.3
// for the kernel above; variants with W staged once per CU in LDS (one
// workgroup of eight wavefronts, or x fragments in registers with one
// wavefront per SIMD) took 18.2-19.3 us. The floor is the fp32 MFMA work
// (7.1 us at the 2.06 GHz this kernel runs at) behind a first x round that
// no wavefront can compute without.
constexpr int kNrRows = 16;
constexpr int kNrMinK = 128;
constexpr int kNrMaxK = 304;
// LDS row stride: 8 x odd (mod 64 floats). Measured ds_read_b128 rates of
// this fragment pattern (lane l: row l%16, column 4*(l/16)) on MI355X: 166-175
// B/clk per CU for strides of 8 x odd mod 64, as fast as linear reads; about
// 123 for 4 x odd, 63 for 32 mod 64, 31 for 0 mod 64.
// Under bf16 math K is padded to 32-k blocks (up to 320 values a row).
template <int MATH>
constexpr int nr_stride() { return MATH == kMathBF16 ? 320 + 8 : kNrMaxK + 8; }
constexpr int kNrXq = 5;      // x float4 per thread and tile: 16 lanes per row, quads slot + 16 j, j < 5
constexpr int kNrPerCu = 3;  // workgroups per CU (VGPR-bound)

// MATH: fp32 (NB 16-k blocks, 16 x 16 x 4 MFMAs) or bf16 (NB 32-k blocks:
// lane l's fragments are k = 32 b + 8*(l/16) .. +7 of its row, both operands
// rounded to bf16, one 16 x 16 x 32 MFMA per block).
template <int EPI, int NB, int MATH>
__global__ __launch_bounds__(kThreads) void gemm_nt_narrow_r_kernel(GemmArgs g, int ntiles) {
  constexpr int kNrS = nr_stride<MATH>();
  constexpr int KB = MATH == kMathBF16 ? 32 : 16;  // k per block
  __shared__ __align__(16) float xs[2][kNrRows * kNrS];  // 39.9 KB (fp32), 42.0 KB (bf16)
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int ct = __builtin_amdgcn_readfirstlane(wave_id());  // the wave's 16-column tile
  const int rl = lane & 15, ks = lane >> 4;
  const int K = g.K;
  const int Q = K / 4;  // data quads per row
  constexpr int QP = KB / 4 * NB;
  static_assert(QP <= 16 * kNrXq && 4 * QP <= kNrS, "x tile slots");
  const float* x = static_cast<const float*>(g.x);
  // x tile slots: row xrow, quads xslot + 16 j (16 lanes read 256 contiguous bytes)
  const int xrow = tid >> 4, xslot = tid & 15;
  float4 st[kNrXq];
  auto load_x = [&](int t) {
    const int64_t m = static_cast<int64_t>(t) * kNrRows + xrow;
    const float* p = x + (m < g.M ? m : g.M - 1) * K;  // rows past M: outputs never stored
#pragma unroll
    for (int j = 0; j < kNrXq; ++j) {
      const int q = xslot + 16 * j;
      st[j] = *reinterpret_cast<const float4*>(p + 4 * (q < Q ? q : Q - 1));
    }
  };
  auto store_x = [&](float* d) {
#pragma unroll
    for (int j = 0; j < kNrXq; ++j) {
      const int q = xslot + 16 * j;
      if (q < QP) *reinterpret_cast<float4*>(d + xrow * kNrS + 4 * q) = q < Q ? st[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  // W fragments (loads first, so waiting for them does not wait for x)
  const int wn = 16 * ct + rl;
  constexpr int WQ = KB / 16;  // float4 of W per lane and block
  float4 w[NB][WQ];
  {
    const float* p = g.w + static_cast<int64_t>(wn < g.N ? wn : g.N - 1) * K;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int h = 0; h < WQ; ++h) {
        const int k = KB * b + 4 * WQ * ks + 4 * h;
        w[b][h] = *reinterpret_cast<const float4*>(p + (k < K ? k : K - 4));
      }
  }
  int t = blockIdx.x;
  load_x(t);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int h = 0; h < WQ; ++h)
      if (wn >= g.N || KB * b + 4 * WQ * ks + 4 * h >= K) w[b][h] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  [[maybe_unused]] bf16x8 wb16[MATH == kMathBF16 ? NB : 1];
  if constexpr (MATH == kMathBF16) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
      wb16[b] = bf16x8{static_cast<__bf16>(w[b][0].x), static_cast<__bf16>(w[b][0].y), static_cast<__bf16>(w[b][0].z),
                       static_cast<__bf16>(w[b][0].w), static_cast<__bf16>(w[b][1].x), static_cast<__bf16>(w[b][1].y),
                       static_cast<__bf16>(w[b][1].z), static_cast<__bf16>(w[b][1].w)};
  }
  store_x(xs[0]);
  // the lane's output columns nc0 .. nc0 + 3: bias and attention vectors
  const int nc0 = 16 * ct + 4 * ks;
  const bool cols = 16 * ct < g.N;
  const bool full4 = g.vec4 && nc0 + 4 <= g.N;
  const int H = EPI == kEpiLogits ? g.N / g.C : 0;
  float bv[4], as[4], ad[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int n = nc0 + q;
    // autocast casts the bias to bf16 with the other operands
    const float bq = (g.bias && n < g.N) ? g.bias[n] : 0.0f;
    bv[q] = g.round_bf16 ? round_bf16(bq) : bq;
    as[q] = ad[q] = 0.0f;
    if constexpr (EPI == kEpiLogits) {
      if (n < g.N) {
        as[q] = g.att_src[n];  // head ct (C == 16), channel n - 16 ct: offset ct * C + (n - ct * C) = n
        ad[q] = g.att_dst[n];
      }
    }
  }
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  for (int i = 0; t < ntiles; ++i, t += gridDim.x) {
    // the next tile's x (the last tile re-reads itself, from L2: no branch
    // around the loads, whose only wait is at the LDS store)
    const int tn = t + static_cast<int>(gridDim.x) < ntiles ? t + static_cast<int>(gridDim.x) : t;
    load_x(tn);
    __builtin_amdgcn_sched_barrier(0);  // the next tile's loads ahead of the MFMAs
    const float* xp = xs[i & 1] + rl * kNrS + 4 * WQ * ks;
    f32x4 a0 = {0.0f, 0.0f, 0.0f, 0.0f}, a1 = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (MATH == kMathBF16) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float4 lo = *reinterpret_cast<const float4*>(xp + KB * b);
        const float4 hi = *reinterpret_cast<const float4*>(xp + KB * b + 4);
        const bf16x8 xb{static_cast<__bf16>(lo.x), static_cast<__bf16>(lo.y), static_cast<__bf16>(lo.z),
                        static_cast<__bf16>(lo.w), static_cast<__bf16>(hi.x), static_cast<__bf16>(hi.y),
                        static_cast<__bf16>(hi.z), static_cast<__bf16>(hi.w)};
        // one chain in block order: the sums of the narrow kernel above
        // (cign_linear_bwd_bf16gy's grad_x takes that kernel on bf16 storage
        // and must match cign_linear_bwd's bit for bit)
        a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb16[b], xb, a0, 0, 0, 0);
      }
    } else {
      float4 xv = *reinterpret_cast<const float4*>(xp);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const float4 xn = *reinterpret_cast<const float4*>(xp + 16 * (b + 1 < NB ? b + 1 : b));
        a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[b][0].x, xv.x, a0, 0, 0, 0);
        a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[b][0].y, xv.y, a1, 0, 0, 0);
        a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[b][0].z, xv.z, a0, 0, 0, 0);
        a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(w[b][0].w, xv.w, a1, 0, 0, 0);
        xv = xn;
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // the store's wait for x after the MFMAs
    store_x(xs[(i + 1) & 1]);
    // epilogue (epilogue_swapped's for one 16 x 16 tile, with the bias and
    // attention vectors loaded once per workgroup above)
    const int64_t m = static_cast<int64_t>(t) * kNrRows + rl;
    const f32x4 acc = a0 + a1;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = g.round_bf16 ? round_bf16(acc[q] + bv[q]) : acc[q] + bv[q];
    if (cols && m < g.M) {
      const int64_t o = m * g.N + nc0;
      if (g.y_bf16) {
        __bf16* yb = reinterpret_cast<__bf16*>(g.y);
        if (full4) {
          *reinterpret_cast<bf16x4*>(yb + o) = bf16x4{static_cast<__bf16>(v[0]), static_cast<__bf16>(v[1]),
                                                      static_cast<__bf16>(v[2]), static_cast<__bf16>(v[3])};
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (nc0 + q < g.N) yb[o + q] = static_cast<__bf16>(v[q]);
        }
      } else if (full4) {
        *reinterpret_cast<float4*>(g.y + o) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (nc0 + q < g.N) g.y[o + q] = v[q];
      }
    }
    if constexpr (EPI == kEpiLogits) {
      float ss = 0.0f, sd = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ss = fmaf(v[q], as[q], ss);
        sd = fmaf(v[q], ad[q], sd);
      }
#pragma unroll
      for (int o = 16; o < kWave; o <<= 1) {
        ss += shfl_xor(ss, o);
        sd += shfl_xor(sd, o);
      }
      if (cols && lane < 16 && ct < H && m < g.M) {
        g.alpha_src[m * H + ct] = ss;
        g.alpha_dst[m * H + ct] = sd;
      }
    }
    __syncthreads();
  }
}

template <int EPI, int MATH, int NB>
int launch_narrow_r(hipStream_t st, const GemmArgs& g, int grid, int ntiles) {
  constexpr int KB = MATH == kMathBF16 ? 32 : 16;
  if (NB == (g.K + KB - 1) / KB) {
    hipLaunchKernelGGL((gemm_nt_narrow_r_kernel<EPI, NB, MATH>), dim3(grid), dim3(kThreads), 0, st, g, ntiles);
    return check_launch("cign linear (narrow, W in registers)");
  }
  if constexpr (NB > kNrMinK / KB) return launch_narrow_r<EPI, MATH, NB - 1>(st, g, grid, ntiles);
  return set_error(kInvalid, "cign linear: K=%d outside the register-W kernel's range", g.K);
}

// grad_W partials of a narrow projection: a workgroup owns a row chunk, all
// (at most 64) outputs n and 64 inputs k0 .. k0 + 63; its four wavefronts
// take a quarter of the chunk's rows each for the whole 64 x 64 tile. The
// reduction dimension is m, and 16-byte loads feed the MFMAs directly: for
// four rows m .. m+3, lane l loads x[m + l/16][k0 + 4*(l%16) .. +3] and
// grad_y[m + l/16][4*(l%16) .. +3] (each load four rows x 256 contiguous
// bytes), and value i of the lane's x quad is operand row l%16 of "k tile" i,
// the sixteen inputs k0 + 4r + i, r < 16 (strided, which the products do not
// mind), likewise for n; the 4 x 4 tile pairs take sixteen 16 x 16 x 4 MFMAs
// per two loads. A lane then holds, per n tile j and row r of its result
// fragment, the four consecutive inputs k0 + 16*(l/16) + 4r .. +3 of output
// n = 4*(l%16) + j: one 16-byte store. Columns past N or K are clamped to the
// last aligned quad (outputs never stored); rows past the chunk read its last
// row and count zero. Under bf16 math both operands are rounded to bf16
// (exact products, fp32 sums, as the bf16 MFMA gives). The four wavefronts'
// tiles are added in LDS in wave order and written as the chunk's partial;
// colsum_kernel adds the chunks in order. Needs N and K multiples of 4 and
// 16-byte (fp32) / 8-byte (bf16 grad_y) aligned rows.
constexpr int kWnK = 64;          // k per workgroup tile
constexpr int kWnChunkRows = 64;  // row chunks: four wavefronts x whole batches
constexpr int kWnUnroll = 2;       // four-row groups per batch (two batches in flight; 4 measured slower)

template <typename TG>
__device__ __forceinline__ void load_quad(const TG* p, float (&v)[4]) {
  if constexpr (std::is_same_v<TG, float>) {
    const float4 t = *reinterpret_cast<const float4*>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
    const uint2 t = *reinterpret_cast<const uint2*>(p);
    v[0] = __uint_as_float(t.x << 16); v[1] = __uint_as_float(t.x & 0xffff0000u);
    v[2] = __uint_as_float(t.y << 16); v[3] = __uint_as_float(t.y & 0xffff0000u);
  }
}

template <int MATH, typename TG>
struct WnBatch {
  float x[kWnUnroll][4], g[kWnUnroll][4];
  // four-row groups m .. m + 4U - 1; rows past m1 read row m1 - 1
  __device__ __forceinline__ void load(const TG* gy, const float* xs, int N, int K, int64_t m, int64_t m1, int kc,
                                       int nc, int lane) {
    const int ks = lane >> 4;
#pragma unroll
    for (int u = 0; u < kWnUnroll; ++u) {
      const int64_t mr = m + 4 * u + ks;
      const int64_t mc = mr < m1 ? mr : m1 - 1;
      load_quad<float>(xs + mc * K + kc, x[u]);
      load_quad<TG>(gy + mc * N + nc, g[u]);
    }
  }
  __device__ __forceinline__ void mma(f32x4 (&acc)[4][4], int64_t m, int64_t m1, int lane) const {
    const int ks = lane >> 4;
#pragma unroll
    for (int u = 0; u < kWnUnroll; ++u) {
      const bool ok = m + 4 * u + ks < m1;
      float xv[4], gv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        xv[i] = ok ? (MATH == kMathBF16 ? round_bf16(x[u][i]) : x[u][i]) : 0.0f;
        gv[i] = MATH == kMathBF16 ? round_bf16(g[u][i]) : g[u][i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], gv[j], acc[i][j], 0, 0, 0);
    }
  }
};

template <int MATH, typename TG = float>
__global__ __launch_bounds__(kThreads) void wgrad_narrow_kernel(const TG* gy, const float* x, int64_t M, int N, int K,
                                                                int64_t chunk, int nchunks, int ntk, float* part) {
  __shared__ f32x4 red[3][16][kWave];  // waves 1..3: 16 accumulator tiles x 64 lanes (48 KB)
  const int lane = lane_id();
  // wave-uniform (the compiler cannot tell from threadIdx.x), so the row loop
  // below is a scalar loop and the accumulators stay in place
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  int tile, cy;
  if (!wg_tile_chunk(ntk, nchunks, true, tile, cy)) return;  // whole workgroup
  const int k0 = tile * kWnK;
  const int64_t c0 = static_cast<int64_t>(cy) * chunk;
  const int64_t c1 = c0 + chunk < M ? c0 + chunk : M;
  const int64_t q = chunk / 4;  // the wave's quarter of the chunk (a multiple of the batch rows)
  const int64_t m0 = c0 + wave * q;
  const int64_t m1 = m0 + q < c1 ? m0 + q : c1;
  const int rl = lane & 15, ks = lane >> 4;
  const int kc = min(k0 + 4 * rl, K - 4), nc = min(4 * rl, N - 4);
  f32x4 acc[4][4];  // [k tile][n tile]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int B = 4 * kWnUnroll;  // rows per batch
  if (m0 < m1) {
    // Two batches in flight. Each batch's loads are issued right after its
    // MFMAs and held there by scheduling barriers (the scheduler otherwise
    // sinks them to their use, one memory round trip per batch); a batch
    // past m1 (the last pair of a short quarter) counts zero.
    WnBatch<MATH, TG> b0, b1;
    b0.load(gy, x, N, K, m0, m1, kc, nc, lane);
    b1.load(gy, x, N, K, m0 + B, m1, kc, nc, lane);
    __builtin_amdgcn_sched_barrier(0);
    for (int64_t m = m0; m < m1; m += 2 * B) {
      b0.mma(acc, m, m1, lane);
      __builtin_amdgcn_sched_barrier(0);
      b0.load(gy, x, N, K, m + 2 * B, m1, kc, nc, lane);
      __builtin_amdgcn_sched_barrier(0);
      b1.mma(acc, m + B, m1, lane);
      __builtin_amdgcn_sched_barrier(0);
      b1.load(gy, x, N, K, m + 3 * B, m1, kc, nc, lane);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave - 1][4 * i + j][lane] = acc[i][j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] += red[w][4 * i + j][lane];
  float* out = part + static_cast<int64_t>(cy) * N * K;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = 4 * rl + j;
    if (n >= N) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = k0 + 16 * ks + 4 * r;
      if (k >= K) continue;  // K % 4 == 0: the quad is whole or past K
      *reinterpret_cast<float4*>(out + static_cast<int64_t>(n) * K + k) =
          make_float4(acc[0][j][r], acc[1][j][r], acc[2][j][r], acc[3][j][r]);
    }
  }
}

// ---- Weight gradient of the GAT lin with its attention logits (narrow):
// the logits' backward fused into wgrad_narrow_kernel. The projection's
// output gradient is gy = g + g_src (x) att_src + g_dst (x) att_dst (per
// head h: gy[m, h, c] = g[m, h, c] + g_src[m, h] att_src[h, c] + g_dst[m, h]
// att_dst[h, c], the sum attn_bwd_kernel forms), built per 4-column quad as
// the batches load, so it is never stored; and the attention gradients
// sum_m g_src[m, h] x_proj[m, h, c] (likewise g_dst) are summed by every
// workgroup of a row chunk over its share of the chunk's rows after its
// GEMM loop, into partial rows of their own (N for att_src, N for att_dst);
// one colsum launch reduces both partial arrays. Under bf16 math gy and x are rounded to bf16 before
// their products (gy after the fp32 sum, as cign_linear_bwd_bf16gy reads the
// stored sum). Needs N, K, C multiples of 4, N <= 64.
struct WlArgs {
  const float* gf;     // gradient of x_proj from the GAT [M, N]
  const float* gs;     // gradient of alpha_src [M, H]
  const float* gd;     // gradient of alpha_dst [M, H]
  const void* xp;      // x_proj [M, N]: fp32, or bf16 (TXP)
  const float* att_s;  // [N]
  const float* att_d;  // [N]
  const float* x;      // [M, K]
  int64_t M;
  int N, K, C, H;
  int64_t chunk;
  int nchunks, ntk;
  float* part;   // grad_W partials [nchunks][N K]
  float* part2;  // attention partials [nchunks ntk][2 N]
};

template <int MATH>
struct WlBatch {
  float x[kWnUnroll][4], g[kWnUnroll][4], s[kWnUnroll], d[kWnUnroll];
  __device__ __forceinline__ void load(const WlArgs& a, int64_t m, int64_t m1, int kc, int nc, int h, int lane) {
    const int ks = lane >> 4;
#pragma unroll
    for (int u = 0; u < kWnUnroll; ++u) {
      const int64_t mr = m + 4 * u + ks;
      const int64_t mc = mr < m1 ? mr : m1 - 1;
      load_quad<float>(a.x + mc * a.K + kc, x[u]);
      load_quad<float>(a.gf + mc * a.N + nc, g[u]);
      s[u] = a.gs[mc * a.H + h];
      d[u] = a.gd[mc * a.H + h];
    }
  }
  __device__ __forceinline__ void mma(f32x4 (&acc)[4][4], const float (&as)[4], const float (&ad)[4], int64_t m,
                                      int64_t m1, int lane) const {
    const int ks = lane >> 4;
#pragma unroll
    for (int u = 0; u < kWnUnroll; ++u) {
      const bool ok = m + 4 * u + ks < m1;
      float xv[4], gv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float o = s[u] * as[i] + d[u] * ad[i];  // attn_bwd_kernel's sum
        o = g[u][i] + o;
        gv[i] = MATH == kMathBF16 ? round_bf16(o) : o;
        xv[i] = ok ? (MATH == kMathBF16 ? round_bf16(x[u][i]) : x[u][i]) : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[i], gv[j], acc[i][j], 0, 0, 0);
    }
  }
};

// The attention gradients' sums over rows [m0, m1) for the lane's quad of
// columns nc (rows m + l/16), in a pass of their own after the GEMM loop
// (inside it, their registers cost the kernel its second wavefront per SIMD).
template <typename TXP>
__device__ __forceinline__ void wl_attn_rows(const WlArgs& a, int64_t m0, int64_t m1, int nc, int h, int lane,
                                             float (&accs)[4], float (&accd)[4]) {
  const int ks = lane >> 4;
  const TXP* xp = static_cast<const TXP*>(a.xp);
  constexpr int U = 4;  // row groups in flight
  for (int64_t m = m0; m < m1; m += 4 * U) {
    float p[U][4], sv[U], dv[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t mr = m + 4 * u + ks;
      ok[u] = mr < m1;
      const int64_t mc = ok[u] ? mr : m1 - 1;
      load_quad<TXP>(xp + mc * a.N + nc, p[u]);
      sv[u] = a.gs[mc * a.H + h];
      dv[u] = a.gd[mc * a.H + h];
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (ok[u]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          accs[i] = fmaf(sv[u], p[u][i], accs[i]);
          accd[i] = fmaf(dv[u], p[u][i], accd[i]);
        }
      }
  }
}

template <int MATH, typename TXP>
__global__ __launch_bounds__(kThreads) void wgrad_logits_narrow_kernel(WlArgs a) {
  __shared__ f32x4 red[3][16][kWave];  // waves 1..3: 16 accumulator tiles x 64 lanes (48 KB)
  __shared__ float ared[4][2][kNarrowN];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  int tile, cy;
  if (!wg_tile_chunk(a.ntk, a.nchunks, true, tile, cy)) return;  // whole workgroup
  const int N = a.N, K = a.K;
  const int k0 = tile * kWnK;
  const int64_t c0 = static_cast<int64_t>(cy) * a.chunk;
  const int64_t c1 = c0 + a.chunk < a.M ? c0 + a.chunk : a.M;
  const int64_t q = a.chunk / 4;
  const int64_t m0 = c0 + wave * q;
  const int64_t m1 = m0 + q < c1 ? m0 + q : c1;
  const int rl = lane & 15, ks = lane >> 4;
  const int kc = min(k0 + 4 * rl, K - 4), nc = min(4 * rl, N - 4);
  const int h = nc / a.C;  // C % 4 == 0: the quad lies in one head
  float as[4], ad[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    as[i] = a.att_s[nc + i];
    ad[i] = a.att_d[nc + i];
  }
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float accs[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int B = 4 * kWnUnroll;
  if (m0 < m1) {
    WlBatch<MATH> b0, b1;
    b0.load(a, m0, m1, kc, nc, h, lane);
    b1.load(a, m0 + B, m1, kc, nc, h, lane);
    __builtin_amdgcn_sched_barrier(0);
    for (int64_t m = m0; m < m1; m += 2 * B) {
      b0.mma(acc, as, ad, m, m1, lane);
      __builtin_amdgcn_sched_barrier(0);
      b0.load(a, m + 2 * B, m1, kc, nc, h, lane);
      __builtin_amdgcn_sched_barrier(0);
      b1.mma(acc, as, ad, m + B, m1, lane);
      __builtin_amdgcn_sched_barrier(0);
      b1.load(a, m + 3 * B, m1, kc, nc, h, lane);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  float* out = a.part + static_cast<int64_t>(cy) * N * K;
  {
    // the attention sums over this workgroup's share of the chunk: tile t
    // of ntk takes rows c0 + t R .. (R a multiple of 16), the wave a quarter
    const int64_t R = (a.chunk / a.ntk + 15) / 16 * 16;
    const int64_t r0 = c0 + tile * R;
    const int64_t r1 = r0 + R < c1 ? r0 + R : c1;
    const int64_t wa0 = r0 + wave * (R / 4);
    const int64_t wa1 = wa0 + R / 4 < r1 ? wa0 + R / 4 : r1;
    if (wa0 < wa1) wl_attn_rows<TXP>(a, wa0, wa1, nc, h, lane, accs, accd);
    // the wave's sums over its four row slots, then the waves in order
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int o = 16; o < kWave; o <<= 1) {
        accs[i] += shfl_xor(accs[i], o);
        accd[i] += shfl_xor(accd[i], o);
      }
    if (ks == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        ared[wave][0][4 * rl + i] = accs[i];
        ared[wave][1][4 * rl + i] = accd[i];
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave - 1][4 * i + j][lane] = acc[i][j];
  }
  __syncthreads();
  if (wave != 0) return;
  {
    float* out2 = a.part2 + (static_cast<int64_t>(cy) * a.ntk + tile) * 2 * N;
    for (int f = lane; f < 2 * N; f += kWave) {
      const int which = f >= N, c = f - which * N;
      float v = ared[0][which][c];
#pragma unroll
      for (int w = 1; w < 4; ++w) v += ared[w][which][c];
      out2[f] = v;
    }
  }
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] += red[w][4 * i + j][lane];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = 4 * rl + j;
    if (n >= N) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = k0 + 16 * ks + 4 * r;
      if (k >= K) continue;
      *reinterpret_cast<float4*>(out + static_cast<int64_t>(n) * K + k) =
          make_float4(acc[0][j][r], acc[1][j][r], acc[2][j][r], acc[3][j][r]);
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
#pragma unroll
  for (int q = 0; q < 4; ++q) acc[q] = rb_if(RB, acc[q]);
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
// Clifford pack inside the projection (weighting old). The block's
//   G[m, kk*2D + j]     = alpha[m,kk] W(bhr, brh),
//   G[m, kk*2D + D + j] = alpha[m,kk] D(bhr, brh),   bhr = H[m,j] P_kk[m,D+j],
//                                                   brh = C[m,j] P_kk[m,j]
// (packk::interact, the pack kernels' own formula) feeds proj only, so the
// kernels below build G's tiles from H, C, the hops and alpha where the
// projection GEMMs load their operands, and G [n, 2KD] is never stored:
//   forward   g = G Wp^T + bp, out = h + gamma * drop(g)  (the gamma epilogue);
//   backward  grad_G = grad_g Wp per 32-channel block of every hop and half,
//             consumed by the pack's backward in the epilogue (grad_H, grad_C,
//             grad_P_k, grad_alpha), and grad_Wp = grad_g^T G with G rebuilt
//             in the reduction's operand load.
// The reduction over G's columns runs hop by hop over 16 (forward) or 64
// (grad_Wp) channels at a time, W half then D half, so one load of H, C and
// the hop's two halves yields both halves' values.
constexpr int kPackMaxHops = 4;
constexpr int kPpBM = 64;  // rows per workgroup of the pack-projection kernels

struct PackArgs {
  int64_t M;
  int D, K, mode;  // mode: interaction code (packk::interact)
  const float* H;
  const float* C;
  const float* P[kPackMaxHops];
  int64_t p_stride;  // row stride of the hops (>= 2D)
  const float* alpha;
  int64_t a_stride;  // row stride of alpha: K, or 0 for one row shared by all nodes
  const __bf16* w16;  // bf16 math: Wp rounded to bf16 once per call [D, 2KD]
};

// Forward A tile of one K step (hop kk, channels j0 .. j0+15): BM rows x 32
// columns, tile column c < 16 = W value of channel j0 + c, c >= 16 = D value
// of channel j0 + c - 16. Thread: row tid / (16/CPT), CPT = BM/16 channels.
template <int BM>
struct PackAStage {
  static constexpr int CPT = BM / 16;  // channels per thread: 4 (64 rows) or 2 (32 rows)
  static constexpr int TPR = 16 / CPT; // threads per row
  float hv[CPT], cv[CPT], th[CPT], tc[CPT], al;

  template <int N>
  __device__ __forceinline__ static void ld(const float* p, int j, float (&v)[N]) {
    if constexpr (N == 4) {
      gload_fast<float, 4>(p, j, v);
    } else {
      const float2 u = *reinterpret_cast<const float2*>(p + j);
      v[0] = u.x;
      v[1] = u.y;
    }
  }

  __device__ __forceinline__ void load(const PackArgs& a, int64_t m0, int kk, int j0) {
    const int r = threadIdx.x / TPR, j = j0 + CPT * (threadIdx.x % TPR);
    const int64_t m = m0 + r < a.M ? m0 + r : a.M - 1;  // rows past M: outputs never stored
    ld(a.H + m * a.D, j, hv);
    ld(a.C + m * a.D, j, cv);
    const float* pk = a.P[kk] + m * a.p_stride;
    ld(pk, j, th);
    ld(pk, a.D + j, tc);
    al = a.alpha[m * a.a_stride + kk];
  }

  template <typename T>
  __device__ __forceinline__ void store(T* As, int S, int mode) const {
    const int r = threadIdx.x / TPR, c = CPT * (threadIdx.x % TPR);
    float w[CPT], d[CPT];
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const packk::DW e = packk::interact(hv[q] * tc[q], cv[q] * th[q], mode);
      w[q] = al * e.Wv;
      d[q] = al * e.Dv;
    }
    st_lds<T, CPT>(As + r * S + c, w);
    st_lds<T, CPT>(As + r * S + 16 + c, d);
  }
};

// Forward W tile of the same K step: BN rows (all D outputs) x 32, tile
// column c < 16 from Wp column kk*2D + j0 + c, c >= 16 from kk*2D + D + j0 +
// c - 16. fp32 math reads Wp; bf16 math its bf16 copy (half the bytes, no
// conversion per step), 16-byte chunks either way.
template <int MATH, int BN>
struct PackBStage {
  static constexpr int CHUNKS = BN * kBK / 4 / kThreads;
  float b[CHUNKS][4];

  __device__ __forceinline__ void load(const GemmArgs& g, const PackArgs&, int kk, int j0, int D, int n0) {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id >> 3, c = id & 7;
      const int col = kk * 2 * D + (c < 4 ? j0 + 4 * c : D + j0 + 4 * (c - 4));
      gload_fast<float, 4>(g.w + static_cast<int64_t>(n0 + r) * g.K, col, b[i]);
    }
  }
  template <typename T>
  __device__ __forceinline__ void store(T* Bs, int S) const {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      st_lds<T, 4>(Bs + (id >> 3) * S + 4 * (id & 7), b[i]);
    }
  }
};

template <int BN>
struct PackBStage<kMathBF16, BN> {
  static constexpr int CHUNKS = BN * kBK / 8 / kThreads;
  bf16x8 b[CHUNKS];

  __device__ __forceinline__ void load(const GemmArgs& g, const PackArgs& a, int kk, int j0, int D, int n0) {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      const int r = id >> 2, c = id & 3;
      const int col = kk * 2 * D + (c < 2 ? j0 + 8 * c : D + j0 + 8 * (c - 2));
      b[i] = *reinterpret_cast<const bf16x8*>(a.w16 + static_cast<int64_t>(n0 + r) * g.K + col);
    }
  }
  __device__ __forceinline__ void store(__bf16* Bs, int S) const {
#pragma unroll
    for (int i = 0; i < CHUNKS; ++i) {
      const int id = threadIdx.x + i * kThreads;
      *reinterpret_cast<bf16x8*>(Bs + (id >> 2) * S + 8 * (id & 3)) = b[i];
    }
  }
};

// MFMAs of one K step: the wave's columns [wave*TNW*16, +TNW*16) of all four
// 16-row tiles (W tile first operand: the swapped accumulator layout).
template <int MATH, int TNW, int RT>
__device__ __forceinline__ void mma_step_pp(const typename Op<MATH>::T* As, const typename Op<MATH>::T* Bs, int wave,
                                            int lane, f32x4 (&acc)[RT][TNW]) {
  constexpr int S = lds_stride<MATH>();
  const int rl = lane & 15, ks = lane >> 4;
  const int nb = wave * TNW * 16;
  if constexpr (MATH == kMathBF16) {
    bf16x8 a[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) a[r] = *reinterpret_cast<const bf16x8*>(As + (16 * r + rl) * S + ks * 8);
#pragma unroll
    for (int f = 0; f < TNW; ++f) {
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(Bs + (nb + 16 * f + rl) * S + ks * 8);
#pragma unroll
      for (int r = 0; r < RT; ++r) mma_bf16<kLdsAsm>(acc[r][f], b, a[r]);
    }
  } else {
#pragma unroll
    for (int hk = 0; hk < kBK; hk += 16) {
      float4 a[RT];
#pragma unroll
      for (int r = 0; r < RT; ++r) a[r] = *reinterpret_cast<const float4*>(As + (16 * r + rl) * S + hk + ks * 4);
#pragma unroll
      for (int f = 0; f < TNW; ++f) {
        const float4 b = *reinterpret_cast<const float4*>(Bs + (nb + 16 * f + rl) * S + hk + ks * 4);
#pragma unroll
        for (int r = 0; r < RT; ++r) mma_f32x4<kLdsAsm>(acc[r][f], b, a[r]);
      }
    }
  }
}

// g = G Wp^T + bp and the gamma epilogue; a workgroup owns BM rows and BN of
// the D outputs (each wavefront BN/4 of them); the next K step's rows and W
// tile load while the current one runs. With BN < D the D/BN workgroups of a
// row tile each build its G tiles: with one workgroup per 64 rows, c2's 383
// workgroups left the GPU at 1.5 wavefronts per SIMD, too few to cover each
// K step's load latency. One-dimensional grid of 8 ceil(row_tiles / 8) x
// D/BN workgroups, the column blocks of a row tile on one XCD one after
// another (ids go round-robin over the 8 XCDs), so they share its rows in L2.
// The host checks D in {64, 128, 256}, K <= kPackMaxHops, 16-byte aligned
// rows (H, C, hops, Wp, g_out, h, out).
template <int MATH, int BN, int BM>
__global__ __launch_bounds__(kThreads) void pack_proj_fwd_kernel(GemmArgs g, PackArgs a, int row_tiles) {
  using T = typename Op<MATH>::T;
  constexpr int S = lds_stride<MATH>();
  constexpr int TNW = BN / 64;
  constexpr int RT = BM / 16;
  __shared__ __align__(16) T As[2][BM * S];
  __shared__ __align__(16) T Bs[2][BN * S];
  const int ncb = a.D / BN;
  const int xcd = blockIdx.x % 8, jw = blockIdx.x / 8;
  const int rt = (jw / ncb) * 8 + xcd;
  const int n0 = (jw % ncb) * BN;
  if (rt >= row_tiles) return;  // whole workgroup, before any barrier
  const int lane = lane_id();
  const int wave = wave_id();
  const int64_t m0 = static_cast<int64_t>(rt) * BM;

  f32x4 acc[RT][TNW];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int f = 0; f < TNW; ++f) acc[r][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (kLdsAsm) mfma_settle(acc);

  const int jq = a.D / 16;
  const int steps = a.K * jq;
  PackAStage<BM> pa;
  PackBStage<MATH, BN> pb;
  pa.load(a, m0, 0, 0);
  pb.load(g, a, 0, 0, a.D, n0);
  pa.store(As[0], S, a.mode);
  pb.store(Bs[0], S);
  __syncthreads();
  int buf = 0;
  for (int s = 0; s < steps; ++s) {
    const bool more = s + 1 < steps;
    if (more) {
      const int kk = (s + 1) / jq, j0 = ((s + 1) % jq) * 16;
      pa.load(a, m0, kk, j0);
      pb.load(g, a, kk, j0, a.D, n0);
    }
    mma_step_pp<MATH, TNW, RT>(As[buf], Bs[buf], wave, lane, acc);
    if (more) {
      pa.store(As[buf ^ 1], S, a.mode);
      pb.store(Bs[buf ^ 1], S);
    }
    __syncthreads();
    buf ^= 1;
  }
  if constexpr (kLdsAsm) mfma_settle(acc);
  epilogue_swapped<kEpiGamma, TNW, RT>(g, acc, m0, n0 + wave * TNW * 16, lane);
}

// dst[i] = bf16(src[i]) (round to nearest even, as the MFMA operand stores)
__global__ void to_bf16_kernel(const float* src, int64_t n, __bf16* dst) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    dst[i] = static_cast<__bf16>(src[i]);
}

// ---- backward: grad_G and the pack's backward --------------------------------
struct PackBwdArgs {
  PackArgs a;
  const float* gg;     // grad_g [M, D]
  const void* wt;      // Wp^T [2KD, D]: bf16 with bf16 math, else fp32
  float* gH;
  float* gC;
  float* gP[kPackMaxHops];
  int64_t gp_stride;
  float* galpha_part;  // [M, K, D/CBW]: grad_alpha per channel block
};

// A workgroup owns 64 rows (a wavefront 16) and one block cb of CBW channels:
// grad_G for the 2K groups (hop kk, half) of those channels, 2K x CBW
// columns, over the D-long reduction, taken in phases of at most 128: each
// phase stages the Wp^T rows of the block's columns for its K range in LDS
// and loads the wavefront's grad_g fragments for it (about 52 KB of LDS at
// D = 256 bf16, where the whole reduction's rows took 101 KB and left one
// workgroup per CU). The last phase also issues the loads of the rows of H,
// C and the hops the epilogue needs. The epilogue is the pack's backward:
// the lane holds, for its row, channels cb*CBW + 16 fh + 4*(lane/16) + q of
// every group. CBW = 32 (bf16) writes whole 128-byte row segments of every
// gradient; fp32 takes CBW = 16. One-dimensional grid of 8 ceil(row_tiles /
// 8) x D/CBW workgroups: workgroup ids go round-robin over the 8 XCDs, and
// the mapping below gives the D/CBW channel blocks of a row tile to one XCD
// one after another, so the tile's grad_g rows, read by each of them, come
// from that XCD's L2 after the first.
template <int MATH, int KC, int DD>
__global__ __launch_bounds__(kThreads) void pack_proj_bwd_kernel(PackBwdArgs b, int row_tiles) {
  using T = typename Op<MATH>::T;
  constexpr int CBW = MATH == kMathBF16 ? 32 : 16;  // channels per block
  constexpr int NCB = DD / CBW;                     // channel blocks
  constexpr int NFH = CBW / 16;                     // 16-column tiles per group
  constexpr int TF = 2 * KC * NFH;                  // tile f = group * NFH + fh
  constexpr int NCOL = TF * 16;
  constexpr int CE = 16 / sizeof(T);                // elements per 16-byte chunk
  constexpr int KP = DD < 128 ? DD : 128;           // K per phase
  constexpr int PH = DD / KP;
  constexpr int SB = KP + CE;                       // LDS row stride, padded by 16 bytes
  constexpr int NTP = KP / kBK;                     // K steps per phase
  constexpr int CHUNKS = NCOL * KP / CE / kThreads;
  static_assert(NCOL * KP % (CE * kThreads) == 0, "whole staging rounds");
  // loads per round: the largest of 8, 6, 4, 3, 2, 1 dividing CHUNKS
  constexpr int ROUND = CHUNKS % 8 == 0 ? 8 : CHUNKS % 6 == 0 ? 6 : CHUNKS % 4 == 0 ? 4 : CHUNKS % 3 == 0 ? 3
                        : CHUNKS % 2 == 0 ? 2 : 1;
  __shared__ __align__(16) T Bs[NCOL * SB];
  const int xcd = blockIdx.x % 8, jw = blockIdx.x / 8;
  const int rt = (jw / NCB) * 8 + xcd;
  const int cb = jw % NCB;
  if (rt >= row_tiles) return;  // whole workgroup, before any barrier
  const PackArgs& a = b.a;
  const int lane = lane_id(), wave = wave_id();
  const int rl = lane & 15, ks = lane >> 4;
  const int64_t mrow = static_cast<int64_t>(rt) * kPpBM + 16 * wave + rl;
  const bool valid = mrow < a.M;
  const int64_t mr = valid ? mrow : a.M - 1;

  float h[NFH][4], c[NFH][4], th[KC][NFH][4], tc[KC][NFH][4], al[KC];
  f32x4 acc[TF];
#pragma unroll
  for (int f = 0; f < TF; ++f) acc[f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  using XF = std::conditional_t<MATH == kMathBF16, bf16x8, float[8]>;
#pragma unroll
  for (int ph = 0; ph < PH; ++ph) {
    // grad_g fragments of the wavefront's 16 rows over the phase's K range
    // (MFMA second operand), in the operand type: bf16 k = 32t + 8*(lane/16)
    // .. +7; fp32 k = 32t + 4*(lane/16) .. +3 and 32t + 16 + 4*(lane/16) .. +3.
    XF xf[NTP];
#pragma unroll
    for (int t = 0; t < NTP; ++t) {
      float lo[4], hi[4];
      const int k0 = ph * KP + kBK * t;
      const int ka = MATH == kMathBF16 ? k0 + 8 * ks : k0 + 4 * ks;
      const int kb = MATH == kMathBF16 ? ka + 4 : ka + 16;
      gload_fast<float, 4>(b.gg + mr * DD, ka, lo);
      gload_fast<float, 4>(b.gg + mr * DD, kb, hi);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if constexpr (MATH == kMathBF16) {
          xf[t][q] = static_cast<__bf16>(lo[q]);
          xf[t][4 + q] = static_cast<__bf16>(hi[q]);
        } else {
          xf[t][q] = lo[q];
          xf[t][4 + q] = hi[q];
        }
      }
    }
    if (ph == PH - 1) {
      // the epilogue's rows, in flight during the last phase's products
#pragma unroll
      for (int fh = 0; fh < NFH; ++fh) {
        const int j = cb * CBW + 16 * fh + 4 * ks;
        gload_fast<float, 4>(a.H + mr * DD, j, h[fh]);
        gload_fast<float, 4>(a.C + mr * DD, j, c[fh]);
#pragma unroll
        for (int k = 0; k < KC; ++k) {
          const float* pk = a.P[k] + mr * a.p_stride;
          gload_fast<float, 4>(pk, j, th[k][fh]);
          gload_fast<float, 4>(pk, DD + j, tc[k][fh]);
        }
      }
#pragma unroll
      for (int k = 0; k < KC; ++k) al[k] = a.alpha[mr * a.a_stride + k];
    }
    if (ph > 0) __syncthreads();  // the previous phase's products have read Bs
    // Wp^T rows of the block's columns over the phase's K range: tile column
    // col = CBW gi + cc is group gi (hop gi/2, half gi%2), channel cb*CBW + cc.
    {
      const T* wt = static_cast<const T*>(b.wt);
      constexpr int CPR = KP / CE;  // chunks per row
#pragma unroll 1
      for (int r0 = 0; r0 < CHUNKS; r0 += ROUND) {
        uint4 v[ROUND];
#pragma unroll
        for (int i = 0; i < ROUND; ++i) {
          const int id = threadIdx.x + (r0 + i) * kThreads;
          const int col = id / CPR, k = ph * KP + (id % CPR) * CE;
          const int gi = col / CBW;
          const int64_t gcol = (gi >> 1) * 2 * DD + (gi & 1) * DD + cb * CBW + (col % CBW);
          v[i] = *reinterpret_cast<const uint4*>(wt + gcol * DD + k);
        }
#pragma unroll
        for (int i = 0; i < ROUND; ++i) {
          const int id = threadIdx.x + (r0 + i) * kThreads;
          *reinterpret_cast<uint4*>(Bs + (id / CPR) * SB + (id % CPR) * CE) = v[i];
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NTP; ++t) {
      if constexpr (MATH == kMathBF16) {
#pragma unroll
        for (int f = 0; f < TF; ++f) {
          const bf16x8 wb = *reinterpret_cast<const bf16x8*>(Bs + (16 * f + rl) * SB + kBK * t + ks * 8);
          acc[f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wb, xf[t], acc[f], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int f = 0; f < TF; ++f) {
            const float4 wb = *reinterpret_cast<const float4*>(Bs + (16 * f + rl) * SB + kBK * t + 16 * hh + ks * 4);
            const float* xv = xf[t] + 4 * hh;
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.x, xv[0], acc[f], 0, 0, 0);
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.y, xv[1], acc[f], 0, 0, 0);
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.z, xv[2], acc[f], 0, 0, 0);
            acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb.w, xv[3], acc[f], 0, 0, 0);
          }
      }
    }
  }

  // the pack's backward (fused_clifford_cign_pack backward_main_kernel, as
  // cign_pack_gate_bwd); acc[gi * NFH + fh][q] = grad_G[mrow, channel
  // cb*CBW + 16 fh + 4 ks + q of group gi]
  float gsum[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) gsum[k] = 0.0f;
#pragma unroll
  for (int fh = 0; fh < NFH; ++fh) {
    const int j = cb * CBW + 16 * fh + 4 * ks;
    float gh[4], gc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) gh[q] = gc[q] = 0.0f;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      float gpt[4], gpc[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // bf16 math: grad_G is the bf16 output of autocast's Linear backward
        const float goW = MATH == kMathBF16 ? round_bf16(acc[(2 * k) * NFH + fh][q]) : acc[(2 * k) * NFH + fh][q];
        const float goD =
            MATH == kMathBF16 ? round_bf16(acc[(2 * k + 1) * NFH + fh][q]) : acc[(2 * k + 1) * NFH + fh][q];
        const packk::DW e = packk::interact(h[fh][q] * tc[k][fh][q], c[fh][q] * th[k][fh][q], a.mode);
        const float gD = goD * al[k];
        const float gW = goW * al[k];
        const float gbhr = gD * e.dD_bhr + gW * e.dW_bhr;
        const float gbrh = gD * e.dD_brh + gW * e.dW_brh;
        gh[q] += gbhr * tc[k][fh][q];
        gc[q] += gbrh * th[k][fh][q];
        gpt[q] = gbrh * c[fh][q];
        gpc[q] = gbhr * h[fh][q];
        gsum[k] += goW * e.Wv + goD * e.Dv;
      }
      if (valid) {
        float* gp = b.gP[k] + mrow * b.gp_stride;
        *reinterpret_cast<float4*>(gp + j) = make_float4(gpt[0], gpt[1], gpt[2], gpt[3]);
        *reinterpret_cast<float4*>(gp + DD + j) = make_float4(gpc[0], gpc[1], gpc[2], gpc[3]);
      }
    }
    if (valid) {
      *reinterpret_cast<float4*>(b.gH + mrow * DD + j) = make_float4(gh[0], gh[1], gh[2], gh[3]);
      *reinterpret_cast<float4*>(b.gC + mrow * DD + j) = make_float4(gc[0], gc[1], gc[2], gc[3]);
    }
  }
  // grad_alpha of the block: the four lane groups of a row
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    gsum[k] += shfl_xor(gsum[k], 16);
    gsum[k] += shfl_xor(gsum[k], 32);
  }
  if (valid && ks == 0)
#pragma unroll
    for (int k = 0; k < KC; ++k) b.galpha_part[(mrow * a.K + k) * (DD / CBW) + cb] = gsum[k];
}

// grad_alpha[m, k] = sum of the nb channel blocks' partials, in block order.
__global__ void galpha_sum_kernel(const float* part, int64_t mk, int nb, float* galpha) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= mk) return;
  float s = 0.0f;
  for (int q = 0; q < nb; ++q) s += part[i * nb + q];
  galpha[i] = s;
}

// W^T in bf16 for the backward's operand tiles: wt [K, N] = bf16(w [N, K])^T.
__global__ void __launch_bounds__(256) transpose_w_bf16_kernel(const float* __restrict__ w, int N, int K,
                                                              __bf16* __restrict__ wt) {
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
    if (k0 + r < K && n0 + c < N) wt[static_cast<int64_t>(k0 + r) * N + n0 + c] = static_cast<__bf16>(tile[c][r]);
  }
}

// grad_Wp [D, 2KD] partials: the wgrad kernel's tiling (128 x 128 tile of
// grad_Wp per workgroup, a chunk of rows) with the x operand = G rebuilt per
// 32-row step: tile k = kt covers hop kk = kt / (D/64), channels j0 = 64 *
// (kt % (D/64)) .. +63, tile column c < 64 = W value of channel j0 + c,
// c >= 64 = D value of channel j0 + c - 64. Rows past the chunk are zero.
template <int MATH>
struct PackWgStage : WgStage<MATH> {
  // WgStage's register layout: row tid / 8, tile column quads (tid % 8 + 8 i) * 4
  using WgStage<MATH>::v;
  // The raw inputs of a step, loaded before the current step's MFMAs and
  // packed after them (finish), so the loads' latency overlaps the MFMAs.
  float h[2][4], c[2][4], th[2][4], tc[2][4];
  float al;
  bool ok;

  __device__ __forceinline__ void load_pack(const PackArgs& a, int64_t m0, int64_t m1, int kk, int j0) {
    const int r = threadIdx.x / 8;
    const int64_t m = m0 + r;
    ok = m < m1;
    const int64_t mm = ok ? m : m1 - 1;  // a row past m1 reads row m1 - 1 (m0 < m1), packed as zeros
    al = a.alpha[mm * a.a_stride + kk];
    const float* pk = a.P[kk] + mm * a.p_stride;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int j = j0 + ((threadIdx.x % 8) + 8 * i) * 4;
      gload_fast<float, 4>(a.H + mm * a.D, j, h[i]);
      gload_fast<float, 4>(a.C + mm * a.D, j, c[i]);
      gload_fast<float, 4>(pk, j, th[i]);
      gload_fast<float, 4>(pk, a.D + j, tc[i]);
    }
  }
  __device__ __forceinline__ void finish(int mode) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const packk::DW e = packk::interact(h[i][q] * tc[i][q], c[i][q] * th[i][q], mode);
        v[i][q] = ok ? al * e.Wv : 0.0f;
        v[i + 2][q] = ok ? al * e.Dv : 0.0f;
      }
  }
};

template <int MATH>
__global__ __launch_bounds__(kThreads) void pack_wgrad_kernel(const float* gy, PackArgs a, int64_t chunk, int nchunks,
                                                              int ntk, float* part) {
  using T = typename Op<MATH>::T;
  using Lay = WgLayout<MATH>;
  __shared__ __align__(16) T Gs[2][kWgT * kWgM];
  __shared__ __align__(16) T Xs[2][kWgT * kWgM];
  const int N = a.D, KW = 2 * a.K * a.D;
  const int lane = lane_id();
  const int wave = wave_id();
  int tile, cy;
  if (!wg_tile_chunk(((N + kWgT - 1) / kWgT) * ntk, nchunks, MATH == kMathBF16, tile, cy)) return;  // whole workgroup
  const int kt = tile % ntk;
  const int n0 = (tile / ntk) * kWgT;
  const int kk = kt / (a.D / 64), j0 = 64 * (kt % (a.D / 64));
  const int64_t m0 = static_cast<int64_t>(cy) * chunk;
  const int64_t m1 = m0 + chunk < a.M ? m0 + chunk : a.M;
  const int wn = (wave >> 1) * 64, wk = (wave & 1) * 64;
  const int rl = lane & 15, ks = lane >> 4;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (kLdsAsm) mfma_settle(acc);

  WgStage<MATH> sg;
  PackWgStage<MATH> sx;
  sg.load(gy, N, m0, m1, n0, N, true);
  sx.load_pack(a, m0, m1, kk, j0);
  sx.finish(a.mode);
  sg.store(Gs[0]);
  sx.store(Xs[0]);
  __syncthreads();
  int buf = 0;
  for (int64_t mb = m0; mb < m1; mb += kWgM) {
    const bool more = mb + kWgM < m1;
    if (more) {
      sg.load(gy, N, mb + kWgM, m1, n0, N, true);
      sx.load_pack(a, mb + kWgM, m1, kk, j0);
    }
    __builtin_amdgcn_sched_barrier(0);  // the next step's loads ahead of the MFMAs
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
        for (int j = 0; j < 4; ++j) mma_bf16<kLdsAsm>(acc[i][j], gb, xb[j]);
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
          for (int j = 0; j < 4; ++j) mma_f32x4<kLdsAsm>(acc[i][j], gb, xb[j]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // and its packing after them
    if (more) {
      sg.store(Gs[buf ^ 1]);
      sx.finish(a.mode);
      sx.store(Xs[buf ^ 1]);
    }
    __syncthreads();
    buf ^= 1;
  }
  // lane holds grad_Wp rows n = n0 + wn + 16i + 4*(lane/16) + q of tile
  // column wk + 16j + lane%16: G column kk*2D + (wk/64)*D + j0 + 16j + lane%16
  if constexpr (kLdsAsm) mfma_settle(acc);
  float* out = part + static_cast<int64_t>(cy) * N * KW;
  const int gbase = kk * 2 * a.D + (wk / 64) * a.D + j0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = gbase + 16 * j + rl;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn + 16 * i + 4 * ks + q;
        if (n < N) out[static_cast<int64_t>(n) * KW + k] = acc[i][j][q];
      }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
inline bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
inline bool aligned8(const void* p) { return reinterpret_cast<uintptr_t>(p) % 8 == 0; }

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

template <typename TX, int MATH, int EPI, bool FULL>
void launch_nt_bn(hipStream_t st, const GemmArgs& g, int bn, int64_t blocks, int nrt, int nct) {
  const dim3 grid(static_cast<unsigned>(blocks));
  if constexpr (MATH == kMathBF16) {
    if (bn == 64)
      hipLaunchKernelGGL((gemm_nt_lds_kernel<TX, MATH, 64, EPI, FULL>), grid, dim3(kThreads), 0, st, g, nrt, nct);
    else
      hipLaunchKernelGGL((gemm_nt_lds_kernel<TX, MATH, 128, EPI, FULL>), grid, dim3(kThreads), 0, st, g, nrt, nct);
  } else {
    if (bn == 64)
      hipLaunchKernelGGL((gemm_nt_kernel<TX, MATH, 64, EPI, FULL>), grid, dim3(kThreads), 0, st, g, nrt, nct);
    else
      hipLaunchKernelGGL((gemm_nt_kernel<TX, MATH, 128, EPI, FULL>), grid, dim3(kThreads), 0, st, g, nrt, nct);
  }
}

template <typename TX, int MATH, int EPI>
int launch_nt(hipStream_t st, const GemmArgs& g, int bn) {
  if (g.N <= kNarrowN && (EPI != kEpiLogits || g.C == 16)) {
    // at most 64 outputs: 32-row tiles, a 16-column tile per wavefront (the
    // logits epilogue needs each head inside one wavefront's columns)
    const int64_t blocks = (g.M + kNarrowRows - 1) / kNarrowRows;
    if (blocks == 0) return kOk;
    if (blocks > 0x7fffffff) return set_error(kInvalid, "cign linear: too many tiles");
    if constexpr (std::is_same_v<TX, float> && EPI != kEpiGamma) {
      if (g.vec && g.K >= kNrMinK && g.K <= kNrMaxK) {
        // W in registers over 16-row tiles, kNrPerCu workgroups per CU
        const int64_t ntiles = (g.M + kNrRows - 1) / kNrRows;
        if (ntiles > 0x7fffffff) return set_error(kInvalid, "cign linear: too many tiles");
        const int grid = static_cast<int>(std::min<int64_t>(ntiles, static_cast<int64_t>(kNrPerCu) * device_cus()));
        constexpr int KB = MATH == kMathBF16 ? 32 : 16;
        return launch_narrow_r<EPI, MATH, (kNrMaxK + KB - 1) / KB>(st, g, grid, static_cast<int>(ntiles));
      }
    }
    if (g.vec)
      hipLaunchKernelGGL((gemm_nt_narrow_kernel<TX, MATH, EPI, true>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kThreads), 0, st, g);
    else
      hipLaunchKernelGGL((gemm_nt_narrow_kernel<TX, MATH, EPI, false>), dim3(static_cast<unsigned>(blocks)),
                         dim3(kThreads), 0, st, g);
    return check_launch("cign linear (narrow)");
  }
  if (g.M == 0) return kOk;
  if constexpr (MATH == kMathBF16 && EPI == kEpiStore) {
    if (g.vec && g.K % kXrKC == 0 && g.K <= kXrMaxK && xres_enabled()) return launch_xres<TX>(st, g);
  }
  const int nrt = static_cast<int>((g.M + kBM - 1) / kBM);
  const int nct = (g.N + bn - 1) / bn;
  const int64_t blocks = static_cast<int64_t>(nrt) * nct;
  if (blocks == 0) return kOk;
  if (blocks > 0x7fffffff) return set_error(kInvalid, "cign linear: too many tiles");
  // every K step takes the unguarded loads
  if (g.vec && g.K % kBK == 0) launch_nt_bn<TX, MATH, EPI, true>(st, g, bn, blocks, nrt, nct);
  else launch_nt_bn<TX, MATH, EPI, false>(st, g, bn, blocks, nrt, nct);
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

// xcd: the chunking of bf16 operands (wg_tile_chunk); the workspace size
// query takes it (the larger layout) for either math.
inline BwdWs bwd_ws(int64_t M, int N, int K, bool bias, bool xcd = true) {
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
  if (!small && N <= kNarrowN) {
    // wgrad_narrow_kernel: 64-wide k tiles, chunks of a multiple of 64 rows
    // (16-row batches per wavefront), about 512 workgroups, every tile of a
    // chunk on one XCD
    const int64_t ntk = (K + kWnK - 1) / kWnK;
    // (about 512: fewer workgroups left the chip short, more spent longer
    // on the chunk partials and their sums than they saved, at the c2 lin)
    int64_t wgc = wg_chunk_count(M, std::max<int64_t>(1, 512 / ntk), true);
    L.wg_chunk = std::max<int64_t>(kWnChunkRows,
                                   ((M + wgc - 1) / wgc + kWnChunkRows - 1) / kWnChunkRows * kWnChunkRows);
    wgc = M > 0 ? (M + L.wg_chunk - 1) / L.wg_chunk : 1;
    L.wg_chunks = static_cast<int>(wgc);
    L.part_w = off; off = al(off + 4LL * wgc * N * K);
    L.wt = off; off = al(off + 4LL * N * K);
    L.total = off;
    return L;
  }
  const int64_t tiles = static_cast<int64_t>((N + kWgT - 1) / kWgT) * ((K + kWgT - 1) / kWgT);
  int64_t wgc = wg_chunk_count(M, std::max<int64_t>(1, 512 / tiles), xcd);
  L.wg_chunk = std::max<int64_t>(kWgM, ((M + wgc - 1) / wgc + kWgM - 1) / kWgM * kWgM);
  wgc = M > 0 ? (M + L.wg_chunk - 1) / L.wg_chunk : 1;
  L.wg_chunks = static_cast<int>(wgc);
  L.part_w = off; off = al(off + 4LL * (small ? chunks : wgc) * N * K);
  // grad_x = grad_y W runs on the forward NT kernel against W^T [K, N]
  L.wt = off; off = al(off + (small ? 0 : 4LL * N * K));
  L.total = off;
  return L;
}


// ---- pack projection (host) --------------------------------------------------
// Workspace of cign_pack_proj_bwd: Wp^T [2KD, D] (fp32, or bf16 in its
// first half) | grad_Wp partials per row chunk | grad_b partials per row
// chunk | grad_alpha partials per 16-channel block | the node gate's backward.
struct PpWs {
  int wg_chunks, b_chunks;
  int64_t wg_chunk, b_chunk, wt, part_w, part_b, part_a, gate, total;
};

inline int pp_ntk(int D, int K) { return K * (D / 64); }

inline PpWs pp_ws(int64_t M, int D, int K, bool xcd = true) {
  PpWs L;
  auto al = [](int64_t v) { return (v + 255) & ~int64_t(255); };
  const int64_t kw = 2LL * K * D;
  const int64_t tiles = static_cast<int64_t>((D + kWgT - 1) / kWgT) * pp_ntk(D, K);
  int64_t wgc = wg_chunk_count(M, std::max<int64_t>(1, 512 / tiles), xcd);
  L.wg_chunk = std::max<int64_t>(kWgM, ((M + wgc - 1) / wgc + kWgM - 1) / kWgM * kWgM);
  L.wg_chunks = static_cast<int>(M > 0 ? (M + L.wg_chunk - 1) / L.wg_chunk : 1);
  int64_t bc = std::max<int64_t>(1, std::min<int64_t>(1024, (M + 63) / 64));
  L.b_chunk = std::max<int64_t>(1, (M + bc - 1) / bc);
  L.b_chunks = static_cast<int>(M > 0 ? (M + L.b_chunk - 1) / L.b_chunk : 1);
  int64_t off = 0;
  L.wt = off; off = al(off + 4 * kw * D);
  L.part_w = off; off = al(off + 4LL * L.wg_chunks * D * kw);
  L.part_b = off; off = al(off + 4LL * L.b_chunks * D);
  L.part_a = off; off = al(off + 4LL * M * K * (D / 16));
  L.gate = off; off = al(off + gate::node_gate_ws_bytes(M, D, K));
  L.total = off;
  return L;
}

inline int pp_check(const char* who, int64_t n, int D, int K, int interaction, int math, const float* H,
                    const float* C, const float* const* props, int64_t prop_stride, const float* alpha,
                    int64_t alpha_stride, const float* w) {
  if (n < 0) return set_error(kInvalid, "%s: n=%lld", who, static_cast<long long>(n));
  if (D != 64 && D != 128 && D != 256)
    return set_error(kInvalid, "%s: D=%d; the fused pack projection takes D = 64, 128 or 256 (else cign_pack_gate_fwd "
                     "+ cign_linear_gamma_fwd)", who, D);
  if (K < 1 || K > kPackMaxHops) return set_error(kInvalid, "%s: K=%d outside [1, %d]", who, K, kPackMaxHops);
  if (interaction < 0 || interaction > 2) return set_error(kInvalid, "%s: interaction must be 0, 1 or 2", who);
  if (math != kMathF32 && math != kMathBF16) return set_error(kInvalid, "%s: math must be 0 or 1", who);
  if (n > 0x7fffffffLL * kPpBM) return set_error(kInvalid, "%s: n too large", who);
  if (!w || !alpha || !props || (n > 0 && (!H || !C))) return set_error(kInvalid, "%s: null pointer", who);
  if (alpha_stride != 0 && alpha_stride < K) return set_error(kInvalid, "%s: alpha_stride must be 0 or >= K", who);
  if (prop_stride < 2LL * D || prop_stride % 4 != 0)
    return set_error(kInvalid, "%s: prop_stride must be a multiple of 4 and >= 2D", who);
  bool ok = aligned16(H) && aligned16(C) && aligned16(w);
  for (int k = 0; k < K; ++k) ok = ok && props[k] && aligned16(props[k]);
  if (!ok) return set_error(kInvalid, "%s: H, C, every hop and the weight must be 16-byte aligned, non-null", who);
  return kOk;
}

inline PackArgs pp_args(int64_t n, int D, int K, int interaction, const float* H, const float* C,
                        const float* const* props, int64_t prop_stride, const float* alpha, int64_t alpha_stride) {
  PackArgs a{};
  a.M = n; a.D = D; a.K = K; a.mode = interaction; a.H = H; a.C = C; a.p_stride = prop_stride;
  a.alpha = alpha; a.a_stride = alpha_stride;
  for (int k = 0; k < K; ++k) a.P[k] = props[k];
  return a;
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

// cign_linear_fwd / cign_linear_logits_fwd with bf16 math whose y is stored
// as bf16: the values the float32 output would hold (they are bf16-rounded),
// in half the bytes.
int cign_linear_fwd_bf16y(void* stream, int64_t M, int32_t N, int32_t K, int32_t x_dtype, const void* x,
                          const float* w, const float* bias, void* y) {
  int rc = check_common("cign_linear_fwd_bf16y", M, N, K, x, w, y);
  if (rc) return rc;
  if (M == 0) return kOk;
  GemmArgs g{};
  g.M = M; g.N = N; g.K = K; g.x = x; g.w = w; g.bias = bias; g.y = static_cast<float*>(y);
  g.vec = rows_aligned(x, x_dtype, w, K);
  g.vec4 = N % 4 == 0 && aligned16(y);
  g.round_bf16 = true;
  g.y_bf16 = true;
  return dispatch_nt<kEpiStore>(static_cast<hipStream_t>(stream), g, x_dtype, kMathBF16, pick_bn(N, 0, kMathBF16));
}

int cign_linear_logits_fwd_bf16y(void* stream, int64_t M, int32_t heads, int32_t channels, int32_t K,
                                 int32_t x_dtype, const void* x, const float* w, const float* att_src,
                                 const float* att_dst, void* y, float* alpha_src, float* alpha_dst) {
  const int N = heads * channels;
  int rc = check_common("cign_linear_logits_fwd_bf16y", M, N, K, x, w, y);
  if (rc) return rc;
  if (!att_src || !att_dst || (M > 0 && (!alpha_src || !alpha_dst)))
    return set_error(kInvalid, "cign_linear_logits_fwd_bf16y: null pointer");
  const int bn = pick_bn(N, channels, kMathBF16);
  if (bn == 0)
    return set_error(kInvalid, "cign_linear_logits_fwd_bf16y: channels=%d must be 16, 32, 64 or 128 (use "
                     "cign_linear_fwd_bf16y + cign_attn_logits_fwd_bf16)", channels);
  if (M == 0) return kOk;
  GemmArgs g{};
  g.M = M; g.N = N; g.K = K; g.x = x; g.w = w; g.y = static_cast<float*>(y);
  g.vec = rows_aligned(x, x_dtype, w, K);
  g.vec4 = N % 4 == 0 && aligned16(y);
  g.round_bf16 = true;
  g.y_bf16 = true;
  g.C = channels; g.att_src = att_src; g.att_dst = att_dst; g.alpha_src = alpha_src; g.alpha_dst = alpha_dst;
  return dispatch_nt<kEpiLogits>(static_cast<hipStream_t>(stream), g, x_dtype, kMathBF16, bn);
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

// Row chunks of cign_lin_logits_wgrad (wgrad_narrow_kernel's) and its
// workspace: a grad_W partial row (N K floats) per chunk, then an attention
// partial row (2 N) per workgroup.
struct WlWs {
  int64_t chunk, part2, total;
  int chunks, ntk;
};

inline WlWs wl_ws(int64_t M, int N, int K) {
  WlWs L;
  L.ntk = (K + kWnK - 1) / kWnK;
  int64_t wgc = wg_chunk_count(M, std::max<int64_t>(1, 512 / L.ntk), true);
  L.chunk = std::max<int64_t>(kWnChunkRows, ((M + wgc - 1) / wgc + kWnChunkRows - 1) / kWnChunkRows * kWnChunkRows);
  wgc = M > 0 ? (M + L.chunk - 1) / L.chunk : 1;
  L.chunks = static_cast<int>(wgc);
  auto al = [](int64_t v) { return (v + 255) & ~int64_t(255); };
  L.part2 = al(4LL * wgc * N * K);
  L.total = al(L.part2 + 4LL * wgc * L.ntk * 2 * N);
  return L;
}

int64_t cign_lin_logits_wgrad_workspace_bytes(int64_t M, int32_t N, int32_t K) {
  if (M < 0 || N <= 0 || K <= 0) return 0;
  return wl_ws(M, N, K).total;
}

int cign_lin_logits_wgrad(void* stream, int64_t M, int32_t heads, int32_t channels, int32_t K, int32_t xp_dtype,
                          int32_t math, const float* grad_xp, const float* grad_src, const float* grad_dst,
                          const void* xp, const float* att_src, const float* att_dst, const float* x, float* grad_w,
                          float* grad_att_src, float* grad_att_dst, void* workspace, int64_t workspace_bytes) {
  const char* who = "cign_lin_logits_wgrad";
  const int H = heads, C = channels;
  if (M < 0 || H < 1 || C < 1 || K <= 0) return set_error(kInvalid, "%s: bad sizes", who);
  const int N = H * C;
  if (N > kNarrowN || N <= kSmallN || C % 4 != 0 || K % 4 != 0)
    return set_error(kInvalid, "%s: needs %d < heads*channels <= %d, channels and K multiples of 4 (N=%d C=%d K=%d)",
                     who, kSmallN, kNarrowN, N, C, K);
  if (math != kMathF32 && math != kMathBF16) return set_error(kInvalid, "%s: math must be 0 or 1", who);
  if (xp_dtype != kF32 && xp_dtype != kBF16) return set_error(kInvalid, "%s: xp_dtype must be 0 or 1", who);
  if (!grad_w || !grad_att_src || !grad_att_dst || !att_src || !att_dst ||
      (M > 0 && (!grad_xp || !grad_src || !grad_dst || !xp || !x)))
    return set_error(kInvalid, "%s: null pointer", who);
  if (M > 0x7fffffff) return set_error(kInvalid, "%s: M too large", who);
  if (M > 0 && !(aligned16(grad_xp) && aligned16(x) && (xp_dtype == kF32 ? aligned16(xp) : aligned8(xp))))
    return set_error(kInvalid, "%s: grad_xp, x and xp rows must start 16-byte (bf16 xp: 8-byte) aligned", who);
  const WlWs L = wl_ws(M, N, K);
  if (workspace_bytes < L.total || !workspace)
    return set_error(kInvalid, "%s: workspace too small (%lld < %lld)", who, static_cast<long long>(workspace_bytes),
                     static_cast<long long>(L.total));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (M == 0) {
    int rc = rowops::zero_outputs(st, grad_w, N * K, grad_att_src, N, who);
    return rc ? rc : rowops::zero_outputs(st, grad_att_dst, N, nullptr, 0, who);
  }
  WlArgs a{};
  a.gf = grad_xp; a.gs = grad_src; a.gd = grad_dst; a.xp = xp; a.att_s = att_src; a.att_d = att_dst; a.x = x;
  a.M = M; a.N = N; a.K = K; a.C = C; a.H = H;
  a.chunk = L.chunk; a.nchunks = L.chunks; a.ntk = L.ntk;
  a.part = static_cast<float*>(workspace);
  a.part2 = reinterpret_cast<float*>(static_cast<char*>(workspace) + L.part2);
  const dim3 grid(wg_grid(L.ntk, L.chunks, true));
  if (math == kMathBF16) {
    if (xp_dtype == kBF16)
      hipLaunchKernelGGL((wgrad_logits_narrow_kernel<kMathBF16, bf16h>), grid, dim3(kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((wgrad_logits_narrow_kernel<kMathBF16, float>), grid, dim3(kThreads), 0, st, a);
  } else {
    if (xp_dtype == kBF16)
      hipLaunchKernelGGL((wgrad_logits_narrow_kernel<kMathF32, bf16h>), grid, dim3(kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((wgrad_logits_narrow_kernel<kMathF32, float>), grid, dim3(kThreads), 0, st, a);
  }
  int rc = check_launch(who);
  if (rc) return rc;
  // grad_W under bf16 math is the bf16 output of autocast's Linear backward;
  // the attention vectors' gradients stay float32 (cign_attn_logits_bwd_acc's)
  return rowops::launch_colsum_split(st, a.part, L.chunks, N * K, grad_w, a.part2, L.chunks * L.ntk, N, grad_att_src,
                                     grad_att_dst, who, math == kMathBF16);
}

// cign_linear_bwd with bf16 math (no bias) whose grad_y is bf16 storage: the
// values bf16 math rounds it to, in half the bytes (the GAT lin's backward,
// whose gradient the logits backward writes rounded).
int cign_linear_bwd_bf16gy(void* stream, int64_t M, int32_t N, int32_t K, const void* grad_y, const float* x,
                           const float* w, float* grad_x, float* grad_w, void* workspace, int64_t workspace_bytes) {
  if (M < 0 || N <= kSmallN || K <= 0)
    return set_error(kInvalid, "cign_linear_bwd_bf16gy: bad sizes (N must exceed %d)", kSmallN);
  if (!w || !grad_w || (M > 0 && (!grad_y || !x))) return set_error(kInvalid, "cign_linear_bwd_bf16gy: null pointer");
  if (M > 0x7fffffff) return set_error(kInvalid, "cign_linear_bwd_bf16gy: M too large");
  const BwdWs L = bwd_ws(M, N, K, false, true);
  if (workspace_bytes < L.total || (L.total > 0 && !workspace))
    return set_error(kInvalid, "cign_linear_bwd_bf16gy: workspace too small (%lld < %lld)",
                     static_cast<long long>(workspace_bytes), static_cast<long long>(L.total));
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int rc;
  if (M == 0) return rowops::zero_outputs(st, grad_w, N * K, nullptr, 0, "cign_linear_bwd_bf16gy");
  const bf16h* gy = static_cast<const bf16h*>(grad_y);
  if (N <= kNarrowN && N % 4 == 0 && K % 4 == 0 && aligned16(grad_y) && aligned16(x)) {
    const int ntk = (K + kWnK - 1) / kWnK;
    float* part = reinterpret_cast<float*>(ws + L.part_w);
    hipLaunchKernelGGL((wgrad_narrow_kernel<kMathBF16, bf16h>), dim3(wg_grid(ntk, L.wg_chunks, true)), dim3(kThreads),
                       0, st, gy, x, M, N, K, L.wg_chunk, L.wg_chunks, ntk, part);
    if ((rc = check_launch("cign_linear_bwd_bf16gy (grad_W partials, narrow)"))) return rc;
    if ((rc = rowops::launch_colsum(st, part, L.wg_chunks, N * K, 1, grad_w, nullptr,
                                    "cign_linear_bwd_bf16gy (grad_W)", true)))
      return rc;
  } else {
    const int ntk = (K + kWgT - 1) / kWgT;
    const dim3 grid(wg_grid(((N + kWgT - 1) / kWgT) * ntk, L.wg_chunks, true));
    const bool vec = N % 4 == 0 && K % 4 == 0 && aligned16(grad_y) && aligned16(x);
    float* part = reinterpret_cast<float*>(ws + L.part_w);
    hipLaunchKernelGGL((wgrad_kernel<kMathBF16, bf16h>), grid, dim3(kThreads), 0, st, gy, x, M, N, K, L.wg_chunk,
                       L.wg_chunks, ntk, vec, part);
    if ((rc = check_launch("cign_linear_bwd_bf16gy (grad_W partials)"))) return rc;
    if ((rc = rowops::launch_colsum(st, part, L.wg_chunks, N * K, 1, grad_w, nullptr,
                                    "cign_linear_bwd_bf16gy (grad_W)", true)))
      return rc;
  }
  if (!grad_x) return kOk;
  float* wt = reinterpret_cast<float*>(ws + L.wt);
  hipLaunchKernelGGL(transpose_w_kernel, dim3((K + 31) / 32, (N + 31) / 32), dim3(256), 0, st, w, N, K, wt);
  if ((rc = check_launch("cign_linear_bwd_bf16gy (W^T)"))) return rc;
  GemmArgs g{};
  g.M = M; g.N = K; g.K = N; g.x = grad_y; g.w = wt; g.y = grad_x;
  g.vec = rows_aligned(grad_y, kBF16, wt, N);
  g.vec4 = K % 4 == 0 && aligned16(grad_x);
  g.round_bf16 = true;  // grad_x is the bf16 output of autocast's Linear backward
  return dispatch_nt<kEpiStore>(st, g, kBF16, kMathBF16, pick_bn(K, 0, kMathBF16));
}

int cign_linear_bwd(void* stream, int64_t M, int32_t N, int32_t K, int32_t math, const float* grad_y, const float* x,
                    const float* w, float* grad_x, float* grad_w, float* grad_b, void* workspace,
                    int64_t workspace_bytes) {
  if (M < 0 || N <= 0 || K <= 0) return set_error(kInvalid, "cign_linear_bwd: bad sizes");
  if (!w || !grad_w || (M > 0 && (!grad_y || !x))) return set_error(kInvalid, "cign_linear_bwd: null pointer");
  if (math != kMathF32 && math != kMathBF16) return set_error(kInvalid, "cign_linear_bwd: math must be 0 or 1");
  if (M > 0x7fffffff) return set_error(kInvalid, "cign_linear_bwd: M too large");
  const BwdWs L = bwd_ws(M, N, K, grad_b != nullptr, math == kMathBF16);
  if (workspace_bytes < L.total || (L.total > 0 && !workspace))
    return set_error(kInvalid, "cign_linear_bwd: workspace too small (%lld < %lld)",
                     static_cast<long long>(workspace_bytes), static_cast<long long>(L.total));
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int rc;
  if (M == 0) return rowops::zero_outputs(st, grad_w, N * K, grad_b, grad_b ? N : 0, "cign_linear_bwd");
  // Under bf16 math (autocast) grad_x, grad_W and grad_b are rounded to bf16:
  // they are the bf16 outputs of the autocast Linear's backward.
  const bool rb = math == kMathBF16;
  auto bias_grad = [&]() -> int {
    if (!grad_b) return kOk;
    float* part = reinterpret_cast<float*>(ws + L.part_b);
    hipLaunchKernelGGL(bias_grad_kernel, dim3((N + 63) / 64, L.chunks), dim3(kThreads), 0, st, grad_y, M, N, L.chunk,
                       part, rb);
    const int r = check_launch("cign_linear_bwd (bias partials)");
    return r ? r : rowops::launch_colsum(st, part, L.chunks, N, 1, grad_b, nullptr, "cign_linear_bwd (bias)", rb);
  };
  if (N <= kSmallN) {
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
    if ((rc = rowops::launch_colsum(st, part, L.chunks, N * K, 1, grad_w, nullptr, "cign_linear_bwd (grad_W)", rb)))
      return rc;
    return bias_grad();
  }
  // grad_W [N,K] = grad_y^T x: split-M MFMA partials, then chunk sums.
  if (N <= kNarrowN && N % 4 == 0 && K % 4 == 0 && aligned16(grad_y) && aligned16(x)) {
    const int ntk = (K + kWnK - 1) / kWnK;
    float* part = reinterpret_cast<float*>(ws + L.part_w);
    const dim3 grid(wg_grid(ntk, L.wg_chunks, true));
    if (math == kMathBF16)
      hipLaunchKernelGGL(wgrad_narrow_kernel<kMathBF16>, grid, dim3(kThreads), 0, st, grad_y, x, M, N, K, L.wg_chunk,
                         L.wg_chunks, ntk, part);
    else
      hipLaunchKernelGGL(wgrad_narrow_kernel<kMathF32>, grid, dim3(kThreads), 0, st, grad_y, x, M, N, K, L.wg_chunk,
                         L.wg_chunks, ntk, part);
    if ((rc = check_launch("cign_linear_bwd (grad_W partials, narrow)"))) return rc;
    if ((rc = rowops::launch_colsum(st, part, L.wg_chunks, N * K, 1, grad_w, nullptr, "cign_linear_bwd (grad_W)",
                                    rb)))
      return rc;
  } else {
    const int ntk = (K + kWgT - 1) / kWgT;
    const dim3 grid(wg_grid(((N + kWgT - 1) / kWgT) * ntk, L.wg_chunks, math == kMathBF16));
    const bool vec = N % 4 == 0 && K % 4 == 0 && aligned16(grad_y) && aligned16(x);
    float* part = reinterpret_cast<float*>(ws + L.part_w);
    if (math == kMathBF16)
      hipLaunchKernelGGL(wgrad_kernel<kMathBF16>, grid, dim3(kThreads), 0, st, grad_y, x, M, N, K, L.wg_chunk,
                         L.wg_chunks, ntk, vec, part);
    else
      hipLaunchKernelGGL(wgrad_kernel<kMathF32>, grid, dim3(kThreads), 0, st, grad_y, x, M, N, K, L.wg_chunk,
                         L.wg_chunks, ntk, vec, part);
    if ((rc = check_launch("cign_linear_bwd (grad_W partials)"))) return rc;
    if ((rc = rowops::launch_colsum(st, part, L.wg_chunks, N * K, 1, grad_w, nullptr, "cign_linear_bwd (grad_W)",
                                    rb)))
      return rc;
  }
  if (!grad_x) return bias_grad();
  // grad_x [M,K] = grad_y [M,N] W [N,K] = grad_y (W^T)^T: the forward NT
  // kernel with W^T [K,N] as its weight. Under bf16 math it rounds both
  // operands to bf16 as autocast's backward GEMM reads them, and the output
  // to bf16.
  float* wt = reinterpret_cast<float*>(ws + L.wt);
  hipLaunchKernelGGL(transpose_w_kernel, dim3((K + 31) / 32, (N + 31) / 32), dim3(256), 0, st, w, N, K, wt);
  if ((rc = check_launch("cign_linear_bwd (W^T)"))) return rc;
  GemmArgs g{};
  g.M = M; g.N = K; g.K = N; g.x = grad_y; g.w = wt; g.y = grad_x;
  g.vec = rows_aligned(grad_y, kF32, wt, N);
  g.vec4 = K % 4 == 0 && aligned16(grad_x);
  g.round_bf16 = rb;
  if ((rc = dispatch_nt<kEpiStore>(st, g, kF32, math, pick_bn(K, 0, math)))) return rc;
  return bias_grad();
}

int64_t cign_pack_proj_fwd_workspace_bytes(int32_t D, int32_t K, int32_t math) {
  if (K < 1 || K > kPackMaxHops || (D != 64 && D != 128 && D != 256)) return 0;
  return math == kMathBF16 ? 2LL * D * 2 * K * D : 0;
}

int cign_pack_proj_fwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t math,
                       const float* H, const float* C, const float* const* props, int64_t prop_stride,
                       const float* alpha, int64_t alpha_stride, const float* w, const float* bias, const float* h,
                       const float* gamma, float dropout_p, uint64_t seed, float* g_out, float* out, uint8_t* mask,
                       void* workspace, int64_t workspace_bytes) {
  const char* who = "cign_pack_proj_fwd";
  int rc = pp_check(who, n, D, K, interaction, math, H, C, props, prop_stride, alpha, alpha_stride, w);
  if (rc) return rc;
  const int64_t need = cign_pack_proj_fwd_workspace_bytes(D, K, math);
  if (workspace_bytes < need || (need > 0 && (!workspace || !aligned16(workspace))))
    return set_error(kInvalid, "%s: workspace too small or unaligned (%lld < %lld)", who,
                     static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  if (!gamma || (n > 0 && (!h || !g_out || !out || !mask))) return set_error(kInvalid, "%s: null pointer", who);
  if (!(dropout_p >= 0.0f && dropout_p < 1.0f)) return set_error(kInvalid, "%s: dropout_p must be in [0,1)", who);
  if (!aligned16(h) || !aligned16(g_out) || !aligned16(out) || reinterpret_cast<uintptr_t>(mask) % 4 != 0)
    return set_error(kInvalid, "%s: h, g_out and out must be 16-byte aligned, mask 4-byte", who);
  if (n == 0) return kOk;
  GemmArgs g{};
  g.M = n; g.N = D; g.K = 2 * K * D; g.w = w; g.bias = bias; g.y = g_out;
  g.vec = true; g.vec4 = true; g.round_bf16 = math == kMathBF16;
  g.h = h; g.gamma = gamma; g.p = dropout_p; g.seed = seed; g.out = out; g.mask = mask;
  PackArgs a = pp_args(n, D, K, interaction, H, C, props, prop_stride, alpha, alpha_stride);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (math == kMathBF16) {
    __bf16* w16 = static_cast<__bf16*>(workspace);
    const int64_t nw = 2LL * K * D * D;
    hipLaunchKernelGGL(to_bf16_kernel, dim3(static_cast<unsigned>(std::min<int64_t>((nw + 255) / 256, 2048))),
                       dim3(256), 0, st, w, nw, w16);
    if ((rc = check_launch("cign_pack_proj_fwd (bf16 weight)"))) return rc;
    a.w16 = w16;
  }
  // 64-row tiles: at the c2 block (24.5K rows, D = 256, bf16) 119 us against
  // 146 us with 32-row tiles (twice the workgroups, twice the W tile loads)
  auto go = [&](auto MC) {
    constexpr int M_ = decltype(MC)::value;
    const int row_tiles = static_cast<int>((n + kPpBM - 1) / kPpBM);
    auto launch = [&](auto BNC) {
      constexpr int BN = decltype(BNC)::value;
      const dim3 grid1(static_cast<unsigned>((row_tiles + 7) / 8 * 8 * (D / BN)));
      hipLaunchKernelGGL((pack_proj_fwd_kernel<M_, BN, kPpBM>), grid1, dim3(kThreads), 0, st, g, a, row_tiles);
    };
    // Column block: all D outputs with bf16 math (at the production block
    // 120 us against 122 us with 128 and 153 us with 64), 64 with fp32 math,
    // whose double-buffered fp32 tiles of all 256 outputs took 92 KB of LDS
    // and one workgroup per CU (229 us against 237 us with 128 and 317 us
    // with 256).
    if (D == 64 || M_ == kMathF32) launch(std::integral_constant<int, 64>());
    else if (D == 128) launch(std::integral_constant<int, 128>());
    else launch(std::integral_constant<int, 256>());
  };
  if (math == kMathBF16) go(std::integral_constant<int, kMathBF16>());
  else go(std::integral_constant<int, kMathF32>());
  return check_launch(who);
}

int64_t cign_pack_proj_bwd_workspace_bytes(int64_t n, int32_t D, int32_t K) {
  if (n < 0 || K < 1 || K > kPackMaxHops || (D != 64 && D != 128 && D != 256)) return 0;
  return pp_ws(n, D, K).total;
}

int cign_pack_proj_bwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t math,
                       const float* grad_g, const float* H, const float* C, const float* const* props,
                       int64_t prop_stride, const float* alpha, int64_t alpha_stride, const float* w,
                       int32_t score_mode, const float* gate_weight, float* grad_H, float* grad_C,
                       float* const* grad_props, int64_t grad_prop_stride, float* grad_alpha, float* grad_w,
                       float* grad_b, float* grad_gate_weight, float* grad_gate_bias, void* workspace,
                       int64_t workspace_bytes) {
  const char* who = "cign_pack_proj_bwd";
  int rc = pp_check(who, n, D, K, interaction, math, H, C, props, prop_stride, alpha, alpha_stride, w);
  if (rc) return rc;
  if (!grad_w || !grad_props || (n > 0 && (!grad_g || !grad_H || !grad_C || !grad_alpha)))
    return set_error(kInvalid, "%s: null pointer", who);
  if (gate_weight && (!grad_gate_weight || !grad_gate_bias || alpha_stride != K))
    return set_error(kInvalid, "%s: the node gate needs its gradient outputs and a per-node alpha (stride K)", who);
  if (grad_prop_stride < 2LL * D || grad_prop_stride % 4 != 0)
    return set_error(kInvalid, "%s: grad_prop_stride must be a multiple of 4 and >= 2D", who);
  bool ok = aligned16(grad_g) && aligned16(grad_H) && aligned16(grad_C);
  for (int k = 0; k < K; ++k) ok = ok && grad_props[k] && aligned16(grad_props[k]);
  if (!ok) return set_error(kInvalid, "%s: grad_g, grad_H, grad_C and every grad_prop must be 16-byte aligned", who);
  const PpWs L = pp_ws(n, D, K, math == kMathBF16);
  if (workspace_bytes < L.total || !workspace)
    return set_error(kInvalid, "%s: workspace too small (%lld < %lld)", who, static_cast<long long>(workspace_bytes),
                     static_cast<long long>(L.total));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int kw = 2 * K * D;
  if (n == 0) {
    if ((rc = rowops::zero_outputs(st, grad_w, D * kw, grad_b, grad_b ? D : 0, who))) return rc;
    return gate_weight ? rowops::zero_outputs(st, grad_gate_weight, K * 2 * D, grad_gate_bias, K, who) : kOk;
  }
  char* ws = static_cast<char*>(workspace);
  const dim3 tgrid((kw + 31) / 32, (D + 31) / 32);
  if (math == kMathBF16)
    hipLaunchKernelGGL(transpose_w_bf16_kernel, tgrid, dim3(256), 0, st, w, D, kw,
                       reinterpret_cast<__bf16*>(ws + L.wt));
  else
    hipLaunchKernelGGL(transpose_w_kernel, tgrid, dim3(256), 0, st, w, D, kw, reinterpret_cast<float*>(ws + L.wt));
  if ((rc = check_launch("cign_pack_proj_bwd (Wp^T)"))) return rc;
  PackBwdArgs b{};
  b.a = pp_args(n, D, K, interaction, H, C, props, prop_stride, alpha, alpha_stride);
  b.gg = grad_g; b.wt = ws + L.wt; b.gH = grad_H; b.gC = grad_C; b.gp_stride = grad_prop_stride;
  b.galpha_part = reinterpret_cast<float*>(ws + L.part_a);
  for (int k = 0; k < K; ++k) b.gP[k] = grad_props[k];
  const int cbw = math == kMathBF16 ? 32 : 16;  // channel block of pack_proj_bwd_kernel
  const int row_tiles = static_cast<int>((n + kPpBM - 1) / kPpBM);
  const dim3 grid(static_cast<unsigned>((row_tiles + 7) / 8 * 8 * (D / cbw)));
  auto go = [&](auto MC) {
    constexpr int M_ = decltype(MC)::value;
    auto with_d = [&](auto KC) {
      constexpr int K_ = decltype(KC)::value;
      if (D == 64) hipLaunchKernelGGL((pack_proj_bwd_kernel<M_, K_, 64>), grid, dim3(kThreads), 0, st, b, row_tiles);
      else if (D == 128)
        hipLaunchKernelGGL((pack_proj_bwd_kernel<M_, K_, 128>), grid, dim3(kThreads), 0, st, b, row_tiles);
      else hipLaunchKernelGGL((pack_proj_bwd_kernel<M_, K_, 256>), grid, dim3(kThreads), 0, st, b, row_tiles);
    };
    switch (K) {
      case 1: with_d(std::integral_constant<int, 1>()); break;
      case 2: with_d(std::integral_constant<int, 2>()); break;
      case 3: with_d(std::integral_constant<int, 3>()); break;
      default: with_d(std::integral_constant<int, 4>()); break;
    }
    const int64_t mk = n * K;
    hipLaunchKernelGGL(galpha_sum_kernel, dim3(static_cast<unsigned>((mk + 255) / 256)), dim3(256), 0, st,
                       b.galpha_part, mk, D / cbw, grad_alpha);
    const int ntk = pp_ntk(D, K);
    const dim3 wgrid(wg_grid(((D + kWgT - 1) / kWgT) * ntk, L.wg_chunks, math == kMathBF16));
    hipLaunchKernelGGL((pack_wgrad_kernel<M_>), wgrid, dim3(kThreads), 0, st, grad_g, b.a, L.wg_chunk, L.wg_chunks, ntk,
                       reinterpret_cast<float*>(ws + L.part_w));
  };
  if (math == kMathBF16) go(std::integral_constant<int, kMathBF16>());
  else go(std::integral_constant<int, kMathF32>());
  if ((rc = check_launch(who))) return rc;
  // bf16 math: grad_Wp and grad_b are the bf16 outputs of autocast's backward
  const bool rb = math == kMathBF16;
  if ((rc = rowops::launch_colsum(st, reinterpret_cast<float*>(ws + L.part_w), L.wg_chunks, D * kw, 1, grad_w,
                                  nullptr, "cign_pack_proj_bwd (grad_Wp)", rb)))
    return rc;
  if (grad_b) {
    float* part = reinterpret_cast<float*>(ws + L.part_b);
    hipLaunchKernelGGL(bias_grad_kernel, dim3((D + 63) / 64, L.b_chunks), dim3(kThreads), 0, st, grad_g, n, D,
                       L.b_chunk, part, rb);
    if ((rc = check_launch("cign_pack_proj_bwd (bias partials)"))) return rc;
    if ((rc = rowops::launch_colsum(st, part, L.b_chunks, D, 1, grad_b, nullptr, "cign_pack_proj_bwd (bias)", rb)))
      return rc;
  }
  if (!gate_weight) return kOk;
  // the node gate's backward, its input gradients added to the pack's
  return gate::node_gate_bwd(st, n, D, K, score_mode, H, C, gate_weight, alpha, grad_alpha, grad_H, grad_C,
                             grad_gate_weight, grad_gate_bias, ws + L.gate, L.total - L.gate, true,
                             "cign_pack_proj_bwd (node gate)");
}

}  // extern "C"
