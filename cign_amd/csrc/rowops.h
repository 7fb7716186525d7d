// Row-parallel building blocks of the per-node kernels (GAT side ops, block
// ops, Clifford packs).
//
// A row of QC chunks (a chunk is W = 4 floats, one 16-byte access, or W = 1)
// is spread over LPR lanes, a power of two <= 64, so the lanes of a row sit in
// one wavefront and per-row sums are butterflies. Each lane owns V chunks
// (q, q + LPR, ..., q + (V-1)*LPR); a 256-thread workgroup covers RPB =
// 256 / LPR rows at a time.
//
// Sums over rows (parameter gradients) are deterministic and atomic-free:
// each workgroup owns a fixed range of rows and writes one partial row per
// column tile (block_colsum), and colsum_kernel adds the partials in a fixed
// order.
#pragma once

#include <type_traits>

#include "common.h"

namespace cign {
namespace rowops {

template <int N>
using IC = std::integral_constant<int, N>;

// Number of row blocks (partial rows) of a reduction over n rows: about 8
// rows per block, at most 1024 blocks (4 per CU); the workspace of such a
// reduction is quantities * colsum_blocks(n) * width floats.
inline int colsum_blocks(int64_t n) {
  const int64_t b = (n + 7) / 8;
  return static_cast<int>(b < 1 ? 1 : (b < 1024 ? b : 1024));
}

// Threads of the colsum_kernel workgroup (16 or 64 columns x 64 or 16
// partial slices).
constexpr int kColsumThreads = 1024;

template <int LPR>
struct Geo {
  static constexpr int RPB = kBlock / LPR;
  int q;   // lane within the row
  int rl;  // row slot within the workgroup
  __device__ Geo() : q(threadIdx.x & (LPR - 1)), rl(threadIdx.x / LPR) {}
};

template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) v += shfl_xor(v, o);
  return v;
}

// Rows [r0, r1) of row block b out of nb.
__device__ __forceinline__ void block_rows(int64_t n, int nb, int b, int64_t& r0, int64_t& r1) {
  const int64_t rb = (n + nb - 1) / nb;
  r0 = static_cast<int64_t>(b) * rb;
  r1 = r0 + rb < n ? r0 + rb : n;
}

// Adds the per-thread column partials acc[v][w] (tile column (q + v*LPR)*W + w)
// over the RPB row slots of the workgroup and stores the first `ncols` tile
// columns to dst. `lds` holds kBlock * V * W floats.
template <int LPR, int V, int W>
__device__ __forceinline__ void block_colsum(const float (&acc)[V][W], float* lds, float* dst, int ncols) {
  constexpr int NC = LPR * V * W;
  constexpr int RPB = kBlock / LPR;
  const int q = threadIdx.x & (LPR - 1);
  const int rl = threadIdx.x / LPR;
#pragma unroll
  for (int v = 0; v < V; ++v)
#pragma unroll
    for (int w = 0; w < W; ++w) lds[rl * NC + (q + v * LPR) * W + w] = acc[v][w];
  __syncthreads();
  for (int c = threadIdx.x; c < ncols; c += kBlock) {
    float s = 0.0f;
    for (int r = 0; r < RPB; ++r) s += lds[r * NC + c];
    dst[c] = s;
  }
  __syncthreads();
}

// Zero-fills a[0..na) and b[0..nbv) (b may be null): the parameter
// gradients of an empty row set.
int zero_outputs(hipStream_t st, float* a, int na, float* b, int nbv, const char* who);

// out_y[c] = sum over b < nb of part[(y * nb + b) * width + c] for
// `quantities` (1 or 2) outputs y, in a fixed order (colsum_kernel or
// colsum_wide_kernel by shape), each sum rounded to bf16 when round_bf16_out.
int launch_colsum(hipStream_t st, const float* part, int nb, int width, int quantities, float* out0, float* out1,
                  const char* who, bool round_bf16_out = false);

// Two reductions in one launch: out[c] = sum_b part[b][c] over nb partial
// rows of split columns (split % 16 == 0; rounded to bf16 when
// round_bf16_out), and tail0[j] = sum_b tail_part[b][j], tail1[j] =
// sum_b tail_part[b][tn + j] over tail_nb rows of 2 tn columns, each in
// colsum_kernel's fixed order.
int launch_colsum_split(hipStream_t st, const float* part, int nb, int split, float* out, const float* tail_part,
                        int tail_nb, int tn, float* tail0, float* tail1, const char* who, bool round_bf16_out);

// Calls f(IC<LPR>, IC<V>) for a row of qc chunks: LPR = next power of two
// >= qc up to 64, then V = 2 or 4 chunks per lane (qc <= 256). Returns -1 when
// qc > 256 (the caller tiles or rejects).
template <class F>
int with_geo(int qc, F&& f) {
  if (qc <= 1) return f(IC<1>(), IC<1>());
  if (qc <= 2) return f(IC<2>(), IC<1>());
  if (qc <= 4) return f(IC<4>(), IC<1>());
  if (qc <= 8) return f(IC<8>(), IC<1>());
  if (qc <= 16) return f(IC<16>(), IC<1>());
  if (qc <= 32) return f(IC<32>(), IC<1>());
  if (qc <= 64) return f(IC<64>(), IC<1>());
  if (qc <= 128) return f(IC<64>(), IC<2>());
  if (qc <= 256) return f(IC<64>(), IC<4>());
  return -1;
}

inline bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// Runs f(IC<KT>()) with KT = K for the common hop counts 2..4 (kernels
// specialised on the hop count: per-hop state in registers, hop loops
// unrolled), KT = 0 (a runtime loop over K) otherwise.
template <class F>
void with_hops(int K, F&& f) {
  switch (K) {
    case 2: f(IC<2>()); break;
    case 3: f(IC<3>()); break;
    case 4: f(IC<4>()); break;
    default: f(IC<0>()); break;
  }
}

// Grid of a grid-stride loop over `items` units of `per_block` each.
inline int grid_for(int64_t items, int per_block) {
  const int64_t g = (items + per_block - 1) / per_block;
  return static_cast<int>(g < 1 ? 1 : (g > 65536 ? 65536 : g));
}

}  // namespace rowops
}  // namespace cign
