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
//   backward                               grad_x = grad_y W, grad_W = grad_y^T x,
//                                          grad_b = sum_n grad_y
//
// Math: fp32 (v_mfma_f32_16x16x4_f32, exact fp32 products) or bf16
// (v_mfma_f32_16x16x32_bf16, the autocast path of _local_amp_linear: inputs
// rounded to bf16 in registers, fp32 accumulation, output rounded to bf16 and
// returned as fp32). The skinny shapes of the block (N <= 1536 outputs, K <=
// 1536, M = nodes) are HBM-bound in bf16 and MFMA-bound in fp32.
//
// Forward tiling: a workgroup is 4 wavefronts x 32 rows = 128 rows and BN =
// 16*NF (64 or 128) columns; a wavefront holds 2 x NF 16x16 accumulator tiles and, per K
// chunk (16 in fp32, 32 in bf16), loads its A fragments (16 bytes per lane per
// row tile) and its B fragments straight from global memory (W is small and
// stays in L2), prefetching the next chunk before the current chunk's MFMAs.
// Fragment layouts (16x16xK MFMA, lane l): A supplies row l%16 and k-slice
// l/16, B supplies column l%16 and the same k-slice, D holds rows 4*(l/16)+i,
// i < 4, of column l%16.
//
// Backward: grad_x is the same kernel on the transposed weight (one small
// transpose into the workspace); grad_W and grad_b are split over row chunks
// of M (fp32 MFMA, deterministic partials summed in chunk order).
#include <algorithm>
#include <type_traits>

#include "common.h"

namespace cign {
namespace gemm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum Epi : int { kEpiStore = 0, kEpiLogits = 1, kEpiGamma = 2 };
enum Math : int { kMathF32 = 0, kMathBF16 = 1 };

constexpr int kWaves = 4;
constexpr int kRowsPerWave = 32;
constexpr int kBM = kWaves * kRowsPerWave;

struct GemmArgs {
  int64_t M;
  int N, K;
  const void* x;      // [M, K] fp32 or bf16 (x_bf16)
  bool x_bf16;
  bool vec;           // rows of x and w are 16-byte aligned (vector loads)
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

__device__ __forceinline__ float round_bf16(float v) { return to_f32(from_f32<bf16>(v)); }

// One lane's share of a K chunk for one 16-wide fragment: VK consecutive k
// values of one row (zeros past K or past the last row).
template <int MATH>
struct Frag;

template <>
struct Frag<kMathF32> {
  static constexpr int KC = 16;  // k per chunk (4 lanes groups x 4)
  static constexpr int VK = 4;
  float4 v;
};

template <>
struct Frag<kMathBF16> {
  static constexpr int KC = 32;  // 4 lane groups x 8
  static constexpr int VK = 8;
  bf16x8 v;
};

__device__ __forceinline__ __bf16 to_bf16(float f) {
  const bf16 b = from_f32<bf16>(f);
  return __builtin_bit_cast(__bf16, b.bits);
}

// Loads VK values of a row starting at k (row pointer p, row valid, K bound).
template <int MATH>
__device__ __forceinline__ void load_frag(const float* p, bool valid, int k, int K, bool vec, Frag<MATH>& f) {
  constexpr int VK = Frag<MATH>::VK;
  float t[VK];
  if (vec && valid && k + VK <= K) {
#pragma unroll
    for (int q = 0; q < VK; q += 4) {
      const float4 u = *reinterpret_cast<const float4*>(p + k + q);
      t[q] = u.x;
      t[q + 1] = u.y;
      t[q + 2] = u.z;
      t[q + 3] = u.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < VK; ++q) t[q] = (valid && k + q < K) ? p[k + q] : 0.0f;
  }
  if constexpr (MATH == kMathF32) {
    f.v = make_float4(t[0], t[1], t[2], t[3]);
  } else {
#pragma unroll
    for (int q = 0; q < VK; ++q) f.v[q] = to_bf16(t[q]);
  }
}

template <int MATH>
__device__ __forceinline__ void load_frag(const bf16* p, bool valid, int k, int K, bool vec, Frag<MATH>& f) {
  static_assert(MATH == kMathBF16, "bf16 inputs feed the bf16 MFMA");
  if (vec && valid && k + 8 <= K) {
    const uint4 u = *reinterpret_cast<const uint4*>(p + k);
    f.v = __builtin_bit_cast(bf16x8, u);
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint16_t b = (valid && k + q < K) ? p[k + q].bits : 0;
      f.v[q] = __builtin_bit_cast(__bf16, b);
    }
  }
}

template <int MATH>
__device__ __forceinline__ void mma(f32x4& acc, const Frag<MATH>& a, const Frag<MATH>& b) {
  if constexpr (MATH == kMathF32) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v.x, b.v.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v.y, b.v.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v.z, b.v.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v.w, b.v.w, acc, 0, 0, 0);
  } else {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
  }
}

// The fragments of one K chunk for a wavefront: 2 row tiles x NF column tiles.
template <typename TX, int MATH, int NF>
struct ChunkFrags {
  Frag<MATH> a[2];
  Frag<MATH> b[NF];

  __device__ __forceinline__ void load(const GemmArgs& g, const TX* x, int64_t row0, int n0, int k0, int lane) {
    constexpr int VK = Frag<MATH>::VK;
    const int kk = k0 + (lane >> 4) * VK;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int64_t row = row0 + 16 * r + (lane & 15);
      load_frag<MATH>(x + row * g.K, row < g.M, kk, g.K, g.vec, a[r]);
    }
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int n = n0 + 16 * f + (lane & 15);
      load_frag<MATH>(g.w + static_cast<int64_t>(n) * g.K, n < g.N, kk, g.K, g.vec, b[f]);
    }
  }
};

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

template <typename TX, int MATH, int NF, int EPI>
__global__ __launch_bounds__(kWaves * kWave) void gemm_nt_kernel(GemmArgs g, int nrt, int nct) {
  const int lane = lane_id();
  const int wave = wave_id();
  int rt, ct;
  tile_of(nrt, nct, rt, ct);
  const int64_t row0 = static_cast<int64_t>(rt) * kBM + wave * kRowsPerWave;
  const int n0 = ct * (16 * NF);
  const TX* x = static_cast<const TX*>(g.x);
  constexpr int KC = Frag<MATH>::KC;

  f32x4 acc[2][NF];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[r][f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  ChunkFrags<TX, MATH, NF> cur;
  cur.load(g, x, row0, n0, 0, lane);
  for (int k0 = 0; k0 < g.K; k0 += KC) {
    ChunkFrags<TX, MATH, NF> nxt;
    if (k0 + KC < g.K) nxt.load(g, x, row0, n0, k0 + KC, lane);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int f = 0; f < NF; ++f) mma<MATH>(acc[r][f], cur.a[r], cur.b[f]);
    cur = nxt;
  }

  // Epilogue: lane holds rows row0 + 16r + 4*(lane/16) + i of column
  // n0 + 16f + lane%16.
  const int cl = lane & 15;
  const int rq = (lane >> 4) * 4;
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int n = n0 + 16 * f + cl;
    const bool nv = n < g.N;
    const float bv = (g.bias && nv) ? g.bias[n] : 0.0f;
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = acc[r][f][i] + bv;
        if (g.round_bf16) v = round_bf16(v);
        acc[r][f][i] = v;
        const int64_t m = row0 + 16 * r + rq + i;
        if (!nv || m >= g.M) continue;
        const int64_t o = m * g.N + n;
        g.y[o] = v;
        if constexpr (EPI == kEpiGamma) {
          const bool keep = block_keep(g.seed, static_cast<uint64_t>(o), g.p);
          const float dv = keep ? (g.p > 0.0f ? v / (1.0f - g.p) : v) : 0.0f;
          g.out[o] = g.h[o] + g.gamma[n] * dv;
          g.mask[o] = keep ? 1 : 0;
        }
      }
  }
  if constexpr (EPI == kEpiLogits) {
    // Heads of C columns lie whole inside the tile (host: BN % C == 0,
    // C % 16 == 0). Sum over a head's fragments in the lane, then over the 16
    // column lanes.
    const int H = g.N / g.C;
    const int fph = g.C / 16;
    for (int h0 = 0; h0 < NF; h0 += fph) {
      const int head = (n0 + 16 * h0) / g.C;
      float ss[2][4], sd[2][4];
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) ss[r][i] = sd[r][i] = 0.0f;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        if (f < h0 || f >= h0 + fph) continue;
        const int n = n0 + 16 * f + cl;
        const int c = n - head * g.C;
        const float as = n < g.N ? g.att_src[static_cast<int64_t>(head) * g.C + c] : 0.0f;
        const float ad = n < g.N ? g.att_dst[static_cast<int64_t>(head) * g.C + c] : 0.0f;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            ss[r][i] = fmaf(acc[r][f][i], as, ss[r][i]);
            sd[r][i] = fmaf(acc[r][f][i], ad, sd[r][i]);
          }
      }
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int o = 1; o < 16; o <<= 1) {
            ss[r][i] += shfl_xor(ss[r][i], o);
            sd[r][i] += shfl_xor(sd[r][i], o);
          }
      if (cl == 0 && head < H) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int64_t m = row0 + 16 * r + rq + i;
            if (m < g.M) {
              g.alpha_src[m * H + head] = ss[r][i];
              g.alpha_dst[m * H + head] = sd[r][i];
            }
          }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// grad_W / grad_b: partial[c] = grad_y[rows of chunk c]^T x[rows of chunk c].
// A workgroup computes a 64 (outputs) x 64 (inputs) tile over one row chunk:
// wave w owns outputs [16w, 16w + 16) and the tile's 4 input fragments. Per
// group of 16 rows, lane l reads grad_y[m][o] and x[m][k] for rows
// m = m0 + 4j + l/16 (j < 4): column slices of 16 consecutive values, fed to
// 16x16x4 fp32 MFMAs whose k dimension is the row index.
// ---------------------------------------------------------------------------
struct WgradArgs {
  int64_t M;
  int N, K;
  int64_t chunk;        // rows per chunk
  const float* gy;      // [M, N]
  const float* x;       // [M, K]
  float* part_w;        // [chunks, N, K]
  float* part_b;        // [chunks, N] or null
};

__global__ __launch_bounds__(kWaves * kWave) void wgrad_kernel(WgradArgs g, int nkt) {
  const int lane = lane_id();
  const int wave = wave_id();
  const int ot = blockIdx.x / nkt, kt = blockIdx.x % nkt;
  const int c = blockIdx.y;
  const int o = ot * 64 + wave * 16 + (lane & 15);
  const int kbase = kt * 64;
  const int64_t mb = c * g.chunk, me = min(g.M, mb + g.chunk);
  f32x4 acc[4];
#pragma unroll
  for (int f = 0; f < 4; ++f) acc[f] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float bsum = 0.0f;
  const bool ov = o < g.N;
  for (int64_t m0 = mb; m0 < me; m0 += 16) {
    float av[4], bvv[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + 4 * j + (lane >> 4);
      const bool mv = m < me;
      av[j] = (mv && ov) ? g.gy[m * g.N + o] : 0.0f;
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const int k = kbase + 16 * f + (lane & 15);
        bvv[f][j] = (mv && k < g.K) ? g.x[m * g.K + k] : 0.0f;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bsum += av[j];
#pragma unroll
      for (int f = 0; f < 4; ++f) acc[f] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], bvv[f][j], acc[f], 0, 0, 0);
    }
  }
  // acc[f] lane l: rows (outputs) 4*(l/16)+i of this wave's 16, column
  // (input) kbase + 16f + l%16.
  const int rq = (lane >> 4) * 4;
  float* pw = g.part_w + static_cast<int64_t>(c) * g.N * g.K;
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    const int k = kbase + 16 * f + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int oo = ot * 64 + wave * 16 + rq + i;
      if (oo < g.N && k < g.K) pw[static_cast<int64_t>(oo) * g.K + k] = acc[f][i];
    }
  }
  if (g.part_b && kt == 0) {
    bsum += shfl_xor(bsum, 16);
    bsum += shfl_xor(bsum, 32);
    if (lane < 16 && ov) g.part_b[static_cast<int64_t>(c) * g.N + o] = bsum;
  }
}

// out[i] = sum_c part[c * len + i], c = 0 .. chunks-1 (in order).
__global__ void sum_chunks_kernel(const float* part, int chunks, int64_t len, float* out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < len;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    float t = 0.0f;
    for (int c = 0; c < chunks; ++c) t += part[c * len + i];
    out[i] = t;
  }
}

// wt[k, n] = w[n, k]
__global__ void transpose_kernel(const float* w, int N, int K, float* wt) {
  __shared__ float tile[32][33];
  const int k0 = blockIdx.x * 32, n0 = blockIdx.y * 32;
  const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;
  for (int j = ty; j < 32; j += 8) {
    const int n = n0 + j, k = k0 + tx;
    tile[j][tx] = (n < N && k < K) ? w[static_cast<int64_t>(n) * K + k] : 0.0f;
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    const int k = k0 + j, n = n0 + tx;
    if (k < K && n < N) wt[static_cast<int64_t>(k) * N + n] = tile[tx][j];
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
inline bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Column tile of NF 16-wide fragments: 4 (64 columns) or 8 (128 columns;
// wider tiles leave one wavefront per SIMD). For the logits epilogue the tile
// must hold whole heads.
inline int pick_nf(int N, int C) {
  int nf = N <= 64 ? 4 : 8;
  if (C > 0) {
    while (nf < 8 && (16 * nf) % C != 0) nf *= 2;
    if ((16 * nf) % C != 0) return 0;
  }
  return nf;
}

template <typename TX, int MATH, int EPI>
int launch_nt(hipStream_t st, const GemmArgs& g, int nf) {
  const int nrt = static_cast<int>((g.M + kBM - 1) / kBM);
  const int nct = (g.N + 16 * nf - 1) / (16 * nf);
  const int64_t blocks = static_cast<int64_t>(nrt) * nct;
  if (blocks == 0) return kOk;
  if (blocks > 0x7fffffff) return set_error(kInvalid, "cign linear: too many tiles");
#define CIGN_NT(NF) \
  hipLaunchKernelGGL((gemm_nt_kernel<TX, MATH, NF, EPI>), dim3(static_cast<unsigned>(blocks)), dim3(kWaves * kWave), 0, st, g, nrt, nct)
  if (nf == 4) CIGN_NT(4);
  else CIGN_NT(8);
#undef CIGN_NT
  return check_launch("cign linear");
}

template <int EPI>
int dispatch_nt(hipStream_t st, const GemmArgs& g, int x_dtype, int math, int nf) {
  if (x_dtype == kBF16) {
    if (math != kMathBF16) return set_error(kInvalid, "cign linear: bfloat16 inputs need math=1 (bf16 MFMA)");
    return launch_nt<bf16, kMathBF16, EPI>(st, g, nf);
  }
  if (x_dtype != kF32) return set_error(kInvalid, "cign linear: unsupported x dtype %d", x_dtype);
  if (math == kMathF32) return launch_nt<float, kMathF32, EPI>(st, g, nf);
  if (math == kMathBF16) return launch_nt<float, kMathBF16, EPI>(st, g, nf);
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
  int chunks;
  int64_t chunk, wt, part_w, part_b, total;
};

inline BwdWs bwd_ws(int64_t M, int N, int K, bool bias) {
  BwdWs L;
  const int tiles = ((N + 63) / 64) * ((K + 63) / 64);
  // about 4 x 256 workgroups, chunks of at least 256 rows
  int chunks = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>((1024 + tiles - 1) / tiles, (M + 255) / 256)));
  chunks = std::min(chunks, 256);
  L.chunks = chunks;
  L.chunk = (M + chunks - 1) / chunks;
  L.chunk = ((L.chunk + 15) / 16) * 16;
  auto al = [](int64_t v) { return (v + 255) & ~int64_t(255); };
  int64_t off = 0;
  L.wt = off; off = al(off + 4LL * N * K);
  L.part_w = off; off = al(off + 4LL * chunks * N * K);
  L.part_b = off; off = al(off + (bias ? 4LL * chunks * N : 0));
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
  g.M = M; g.N = N; g.K = K; g.x = x; g.x_bf16 = x_dtype == kBF16; g.w = w; g.bias = bias; g.y = y;
  g.vec = rows_aligned(x, x_dtype, w, K);
  g.round_bf16 = math == kMathBF16;
  return dispatch_nt<kEpiStore>(static_cast<hipStream_t>(stream), g, x_dtype, math, pick_nf(N, 0));
}

int cign_linear_logits_fwd(void* stream, int64_t M, int32_t heads, int32_t channels, int32_t K, int32_t x_dtype,
                           int32_t math, const void* x, const float* w, const float* att_src, const float* att_dst,
                           float* y, float* alpha_src, float* alpha_dst) {
  const int N = heads * channels;
  int rc = check_common("cign_linear_logits_fwd", M, N, K, x, w, y);
  if (rc) return rc;
  if (!att_src || !att_dst || (M > 0 && (!alpha_src || !alpha_dst)))
    return set_error(kInvalid, "cign_linear_logits_fwd: null pointer");
  const int nf = channels % 16 == 0 ? pick_nf(N, channels) : 0;
  if (nf == 0)
    return set_error(kInvalid, "cign_linear_logits_fwd: channels=%d must be 16, 32, 64 or 128 (use cign_linear_fwd + "
                     "cign_attn_logits_fwd)", channels);
  if (M == 0) return kOk;
  GemmArgs g{};
  g.M = M; g.N = N; g.K = K; g.x = x; g.x_bf16 = x_dtype == kBF16; g.w = w; g.y = y;
  g.vec = rows_aligned(x, x_dtype, w, K);
  g.round_bf16 = math == kMathBF16;
  g.C = channels; g.att_src = att_src; g.att_dst = att_dst; g.alpha_src = alpha_src; g.alpha_dst = alpha_dst;
  return dispatch_nt<kEpiLogits>(static_cast<hipStream_t>(stream), g, x_dtype, math, nf);
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
  g.M = M; g.N = N; g.K = K; g.x = x; g.x_bf16 = x_dtype == kBF16; g.w = w; g.bias = bias; g.y = g_out;
  g.vec = rows_aligned(x, x_dtype, w, K);
  g.round_bf16 = math == kMathBF16;
  g.h = h; g.gamma = gamma; g.p = dropout_p; g.seed = seed; g.out = y; g.mask = mask;
  return dispatch_nt<kEpiGamma>(static_cast<hipStream_t>(stream), g, x_dtype, math, pick_nf(N, 0));
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
  const BwdWs L = bwd_ws(M, N, K, grad_b != nullptr);
  if (!workspace || workspace_bytes < L.total)
    return set_error(kInvalid, "cign_linear_bwd: workspace too small (%lld < %lld)",
                     static_cast<long long>(workspace_bytes), static_cast<long long>(L.total));
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* wt = reinterpret_cast<float*>(ws + L.wt);
  float* part_w = reinterpret_cast<float*>(ws + L.part_w);
  float* part_b = grad_b ? reinterpret_cast<float*>(ws + L.part_b) : nullptr;
  // grad_x = grad_y W : the forward kernel on W^T ([K, N]).
  if (grad_x && M > 0) {
    hipLaunchKernelGGL(transpose_kernel, dim3((K + 31) / 32, (N + 31) / 32), dim3(256), 0, st, w, N, K, wt);
    int rc = check_launch("cign_linear_bwd (transpose)");
    if (rc) return rc;
    GemmArgs g{};
    g.M = M; g.N = K; g.K = N; g.x = grad_y; g.w = wt; g.y = grad_x;
    g.vec = rows_aligned(grad_y, kF32, wt, N);
    g.round_bf16 = false;
    rc = dispatch_nt<kEpiStore>(st, g, kF32, math, pick_nf(K, 0));
    if (rc) return rc;
  }
  // grad_W, grad_b: split over row chunks, partials summed in chunk order.
  WgradArgs a{};
  a.M = M; a.N = N; a.K = K; a.chunk = L.chunk; a.gy = grad_y; a.x = x; a.part_w = part_w; a.part_b = part_b;
  const int nkt = (K + 63) / 64;
  const int chunks = M > 0 ? static_cast<int>((M + L.chunk - 1) / L.chunk) : 0;
  if (chunks > 0) {
    hipLaunchKernelGGL(wgrad_kernel, dim3(((N + 63) / 64) * nkt, chunks), dim3(kWaves * kWave), 0, st, a, nkt);
    int rc = check_launch("cign_linear_bwd (grad_w)");
    if (rc) return rc;
  }
  const int64_t len = static_cast<int64_t>(N) * K;
  hipLaunchKernelGGL(sum_chunks_kernel, dim3(static_cast<unsigned>(std::min<int64_t>((len + 255) / 256, 4096))),
                     dim3(256), 0, st, part_w, chunks, len, grad_w);
  int rc = check_launch("cign_linear_bwd (sum)");
  if (rc) return rc;
  if (grad_b) {
    hipLaunchKernelGGL(sum_chunks_kernel, dim3((N + 255) / 256), dim3(256), 0, st, part_b, chunks,
                       static_cast<int64_t>(N), grad_b);
    rc = check_launch("cign_linear_bwd (bias)");
  }
  return rc;
}

}  // extern "C"
