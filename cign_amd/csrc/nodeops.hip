// Per-node kernels of the GAT side ops and the block ops, and their C-ABI.
//
// GAT side ops (fused_gat_sideops_ext/fused_gat_sideops_cuda.cu:25-337):
//   attention logits  alpha_src[n,h] = <x[n,h,:], att_src[h,:]>, alpha_dst
//                     likewise; backward g_x = gs*att_src + gd*att_dst,
//                     g_att[h,c] = sum_n g[n,h] x[n,h,c];
//   head mean + bias + SiLU   pre = sum_h out[n,h,:] / H + bias, y = SiLU(pre);
//                     backward g_out = g_y SiLU'(pre) / H per head, g_bias = sum_n.
// Block ops (fused_block_ops.py:15 inline kernels, fused_block_ops_ext/
// fused_block_ops_cuda.cu:45-322), rows of D <= 256:
//   dropout + LayerNorm, add + LayerNorm, dropout-gamma-residual, with their
//   backward passes (dx / dz, weight, bias and gamma gradients).
// Row reductions are butterflies over a row's lanes; sums over nodes go
// through deterministic per-row-block partials (rowops.h).
#include "rowops.h"

namespace cign {
namespace rowops {

// v rounded to bf16 (nearest even), as a float: parameter gradients under
// bf16 autocast are the bf16 outputs of its Linear backward.
__device__ __forceinline__ float bf16_rounded(float v) { return to_f32(from_f32<bf16>(v)); }

// out[c] = sum_b part[b][c] over the nb row-block partials, in a fixed order
// (rounded to bf16 when rb):
// a workgroup of kColsumThreads covers kCols columns (16 or 64) in
// kColsumThreads / kCols slices; thread (c, s) sums the partials b = s,
// s + slices, ... with eight independent accumulators (combined in a fixed
// order), then the slices are added through an LDS tree.
//
// Split outputs (a TailSum): workgroups past the first split / kCols (split
// a multiple of kCols) reduce a second partial array instead, tail.part
// [tail.nb][2 tn], whose columns j < tn go to tail.out0 and the rest to
// tail.out1 (never rounded): two reductions in one launch.
struct TailSum {
  const float* part = nullptr;
  int nb = 0, tn = 0;
  float* out0 = nullptr;
  float* out1 = nullptr;
};

template <int kCols>
__global__ __launch_bounds__(kColsumThreads) void colsum_kernel(const float* part, int nb, int width, float* out0,
                                                                float* out1, bool rb, int split = 0x7fffffff,
                                                                TailSum tail = TailSum()) {
  // kCols columns x kSlices partial slices per workgroup; a slice thread
  // keeps eight partial rows in flight, then the slices meet in an LDS tree
  // (a fixed order, so the sums are deterministic).
  constexpr int kSlices = kColsumThreads / kCols;
  __shared__ float red[kColsumThreads];
  const bool in_tail = static_cast<int64_t>(blockIdx.x) * kCols >= split;  // whole workgroup
  const float* src = in_tail ? tail.part : part + static_cast<int64_t>(blockIdx.y) * nb * width;
  const int rows = in_tail ? tail.nb : nb;
  const int w = in_tail ? 2 * tail.tn : width;
  float* out = blockIdx.y == 0 ? out0 : out1;
  const int t = threadIdx.x;
  const int c = (in_tail ? static_cast<int>(blockIdx.x) * kCols - split : static_cast<int>(blockIdx.x) * kCols) +
                t % kCols;
  const int s = t / kCols;
  float acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = 0.0f;
  if (c < w) {
    int b = s;
    for (; b + 7 * kSlices < rows; b += 8 * kSlices)
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += src[static_cast<int64_t>(b + u * kSlices) * w + c];
    for (; b < rows; b += kSlices) acc[0] += src[static_cast<int64_t>(b) * w + c];
  }
  red[t] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  for (int h = kSlices / 2; h > 0; h >>= 1) {
    if (s < h) red[t] += red[t + h * kCols];
    __syncthreads();
  }
  if (s == 0 && c < w) {
    if (!in_tail)
      out[c] = rb ? bf16_rounded(red[t]) : red[t];
    else if (c < tail.tn)
      tail.out0[c] = red[t];
    else
      tail.out1[c - tail.tn] = red[t];
  }
}

// Wide outputs over many partial rows, four columns a thread: a workgroup
// (256 threads) covers 64 columns in 16 slices; slice s sums the partial rows
// b = s, s + 16, ... as float4 with eight independent accumulators (combined
// in a fixed order), then the slices meet in an LDS tree. Split outputs as in
// colsum_kernel (split a multiple of 64, the first split / 64 workgroups);
// the tail's workgroups cover 16 columns in 64 slices (its partial rows are
// many: one per workgroup of the producing kernel). Needs width % 4 == 0,
// tn % 4 == 0 and 16-byte aligned rows and outputs.
__global__ __launch_bounds__(kBlock) void colsum4_kernel(const float* part, int nb, int width, float* out, bool rb,
                                                         int split, TailSum tail) {
  __shared__ float4 red[kBlock];
  const int head_blocks = split / 64;
  const bool in_tail = static_cast<int>(blockIdx.x) >= head_blocks;  // whole workgroup
  const int quads = in_tail ? 4 : 16;
  const int slices = kBlock / quads;
  const float* src = in_tail ? tail.part : part;
  const int rows = in_tail ? tail.nb : nb;
  const int w = in_tail ? 2 * tail.tn : width;
  const int t = threadIdx.x;
  const int c = (in_tail ? (static_cast<int>(blockIdx.x) - head_blocks) * 16 : static_cast<int>(blockIdx.x) * 64) +
                4 * (t % quads);
  const int s = t / quads;
  float4 acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (c < w) {
    int b = s;
    for (; b + 7 * slices < rows; b += 8 * slices)
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float4 v = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(b + u * slices) * w + c);
        acc[u].x += v.x; acc[u].y += v.y; acc[u].z += v.z; acc[u].w += v.w;
      }
    for (; b < rows; b += slices) {
      const float4 v = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(b) * w + c);
      acc[0].x += v.x; acc[0].y += v.y; acc[0].z += v.z; acc[0].w += v.w;
    }
  }
#pragma unroll
  for (int h = 4; h > 0; h >>= 1)
#pragma unroll
    for (int u = 0; u < h; ++u) {
      acc[u].x += acc[u + h].x; acc[u].y += acc[u + h].y; acc[u].z += acc[u + h].z; acc[u].w += acc[u + h].w;
    }
  red[t] = acc[0];
  __syncthreads();
  for (int h = slices / 2; h > 0; h >>= 1) {
    if (s < h) {
      const float4 v = red[t + h * quads];
      red[t].x += v.x; red[t].y += v.y; red[t].z += v.z; red[t].w += v.w;
    }
    __syncthreads();
  }
  if (s == 0 && c < w) {
    float4 r = red[t];
    if (!in_tail) {
      if (rb) r = make_float4(bf16_rounded(r.x), bf16_rounded(r.y), bf16_rounded(r.z), bf16_rounded(r.w));
      *reinterpret_cast<float4*>(out + c) = r;
    } else {
      // tn % 4 == 0: the quad lies in one tail output
      float* o = c < tail.tn ? tail.out0 + c : tail.out1 + (c - tail.tn);
      *reinterpret_cast<float4*>(o) = r;
    }
  }
}

// Wide outputs over few partial rows (weight gradients): one thread per four
// columns walks every partial row in order, eight rows in flight.
__global__ __launch_bounds__(kBlock) void colsum_wide_kernel(const float* part, int nb, int width, float* out0,
                                                             float* out1, bool rb) {
  const int64_t c = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * 4;
  if (c >= width) return;
  const float* src = part + static_cast<int64_t>(blockIdx.y) * nb * width + c;
  float* out = blockIdx.y == 0 ? out0 : out1;
  float4 acc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) acc[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  int b = 0;
  for (; b + 8 <= nb; b += 8)
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float4 v = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(b + u) * width);
      acc[u].x += v.x; acc[u].y += v.y; acc[u].z += v.z; acc[u].w += v.w;
    }
  for (; b < nb; ++b) {
    const float4 v = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(b) * width);
    acc[0].x += v.x; acc[0].y += v.y; acc[0].z += v.z; acc[0].w += v.w;
  }
#pragma unroll
  for (int h = 4; h > 0; h >>= 1)
#pragma unroll
    for (int u = 0; u < h; ++u) {
      acc[u].x += acc[u + h].x; acc[u].y += acc[u + h].y; acc[u].z += acc[u + h].z; acc[u].w += acc[u + h].w;
    }
  if (rb)
    acc[0] = make_float4(bf16_rounded(acc[0].x), bf16_rounded(acc[0].y), bf16_rounded(acc[0].z), bf16_rounded(acc[0].w));
  *reinterpret_cast<float4*>(out + c) = acc[0];
}

__global__ void zero_kernel(float* a, int na, float* b, int nbv) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i < na) a[i] = 0.0f;
  if (b && i < nbv) b[i] = 0.0f;
}

int zero_outputs(hipStream_t st, float* a, int na, float* b, int nbv, const char* who) {
  const int m = na > nbv ? na : nbv;
  if (m <= 0) return kOk;
  hipLaunchKernelGGL(zero_kernel, dim3((m + kBlock - 1) / kBlock), dim3(kBlock), 0, st, a, na, b, nbv);
  return check_launch(who);
}

int launch_colsum_split(hipStream_t st, const float* part, int nb, int split, float* out, const float* tail_part,
                        int tail_nb, int tn, float* tail0, float* tail1, const char* who, bool round_bf16_out) {
  TailSum tail;
  tail.part = tail_part;
  tail.nb = tail_nb;
  tail.tn = tn;
  tail.out0 = tail0;
  tail.out1 = tail1;
  if (split % 64 == 0 && tn % 4 == 0 && aligned16(part) && aligned16(out) && aligned16(tail_part) &&
      aligned16(tail0) && aligned16(tail1)) {
    // four columns a thread (the c2 lin: 19,200 + 128 columns over 96 and
    // 480 partial rows: 7.9 us on colsum_kernel<16>)
    const int blocks = split / 64 + (2 * tn + 15) / 16;
    if (blocks == 0) return kOk;
    hipLaunchKernelGGL(colsum4_kernel, dim3(blocks), dim3(kBlock), 0, st, part, nb, split, out, round_bf16_out, split,
                       tail);
    return check_launch(who);
  }
  if (split % 16 != 0) return set_error(kInvalid, "%s: split colsum needs a multiple of 16 columns", who);
  const int blocks = split / 16 + (2 * tn + 15) / 16;
  if (blocks == 0) return kOk;
  hipLaunchKernelGGL(colsum_kernel<16>, dim3(blocks, 1), dim3(kColsumThreads), 0, st, part, nb, split, out, nullptr,
                     round_bf16_out, split, tail);
  return check_launch(who);
}

int launch_colsum(hipStream_t st, const float* part, int nb, int width, int quantities, float* out0, float* out1,
                  const char* who, bool round_bf16_out) {
  if (width <= 0) return kOk;
  // Three fixed-order paths: outputs of at least 65536 columns over at most
  // 128 partial rows (weight gradients) take colsum_wide_kernel, one thread
  // per four columns walking the rows in order (16K threads and more);
  // outputs of at most 4096 columns over at least 256 partial rows
  // (LayerNorm and bias gradients at large n), and mid-width outputs (the
  // 64 x 300 weight gradient of the c2 projection: 4800 threads of the wide
  // kernel walking 128 rows took 26 us), take 16 columns x 64 slices, so more
  // workgroups share the rows; the rest 64 columns x 16 slices.
  const bool vec = width % 4 == 0 && aligned16(part) && aligned16(out0) && (!out1 || aligned16(out1));
  if (width > 4096 && width < 65536 && nb >= 16 && quantities == 1 && vec) {
    // four columns a thread: 64 columns x 16 slices a workgroup
    hipLaunchKernelGGL(colsum4_kernel, dim3((width + 63) / 64), dim3(kBlock), 0, st, part, nb, width, out0,
                       round_bf16_out, 0x7fffffff, TailSum());
    return check_launch(who);
  }
  if (width > 4096 && width < 65536 && nb >= 16)
    hipLaunchKernelGGL(colsum_kernel<16>, dim3((width + 15) / 16, quantities), dim3(kColsumThreads), 0, st, part, nb,
                       width, out0, out1, round_bf16_out);
  else if (width > 4096 && nb <= 128 && vec)
    hipLaunchKernelGGL(colsum_wide_kernel, dim3((width / 4 + kBlock - 1) / kBlock, quantities), dim3(kBlock), 0, st,
                       part, nb, width, out0, out1, round_bf16_out);
  else if (width <= 4096 && nb >= 256)
    hipLaunchKernelGGL(colsum_kernel<16>, dim3((width + 15) / 16, quantities), dim3(kColsumThreads), 0, st, part, nb,
                       width, out0, out1, round_bf16_out);
  else
    hipLaunchKernelGGL(colsum_kernel<64>, dim3((width + 63) / 64, quantities), dim3(kColsumThreads), 0, st, part, nb,
                       width, out0, out1, round_bf16_out);
  return check_launch(who);
}

}  // namespace rowops

namespace nodeops {
using namespace rowops;

// ---------------------------------------------------------------------------
// Attention logits.
// ---------------------------------------------------------------------------
// Rows r of x viewed as [n*H, C]; head h = r % H. x is float32, or bf16
// storage (TX = bf16h: W values per 2W-byte load).
template <int LPR, int V, int W, typename TX = float>
__global__ __launch_bounds__(kBlock) void attn_fwd_kernel(int64_t rows, int H, int C, const TX* x,
                                                          const float* as, const float* ad, float* os, float* od) {
  const Geo<LPR> g;
  const int qc = C / W;
  const int64_t step = static_cast<int64_t>(gridDim.x) * Geo<LPR>::RPB;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * Geo<LPR>::RPB + g.rl; r < rows; r += step) {
    const int h = static_cast<int>(r % H);
    float ss = 0.0f, sd = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = g.q + v * LPR;
      if (c < qc) {
        float xv[W], av[W], dv[W];
        Chunk<TX, W>::load(x + r * C + c * W, xv);
        Chunk<float, W>::load(as + static_cast<int64_t>(h) * C + c * W, av);
        Chunk<float, W>::load(ad + static_cast<int64_t>(h) * C + c * W, dv);
#pragma unroll
        for (int w = 0; w < W; ++w) {
          ss = fmaf(xv[w], av[w], ss);
          sd = fmaf(xv[w], dv[w], sd);
        }
      }
    }
    ss = row_sum<LPR>(ss);
    sd = row_sum<LPR>(sd);
    if (g.q == 0) {
      os[r] = ss;
      od[r] = sd;
    }
  }
}

// Rows = nodes of width F = H*C; column tile blockIdx.y of LPR*V chunks.
// Writes g_x (plus gx_in, the gradient x receives from its other consumer,
// when not null; it may alias gx) and the tile's partial sums of gs*x and
// gd*x for row block blockIdx.x (part layout [2][nb][F]).
template <int LPR, int V, int W, typename TX = float, typename TO = float>
__global__ __launch_bounds__(kBlock) void attn_bwd_kernel(int64_t n, int H, int C, const float* gs, const float* gd,
                                                          const TX* x, const float* as, const float* ad,
                                                          const float* gx_in, TO* gx, float* part, int nb) {
  __shared__ float lds[kBlock * V * W];
  const Geo<LPR> g;
  const int F = H * C;
  const int qf = F / W;
  const int t0 = blockIdx.y * LPR * V;  // first chunk of the tile
  int64_t r0, r1;
  block_rows(n, nb, blockIdx.x, r0, r1);
  float av[V][W], dv[V][W], accs[V][W], accd[V][W];
  int hv[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int c = t0 + g.q + v * LPR;
    hv[v] = c < qf ? (c * W) / C : 0;
#pragma unroll
    for (int w = 0; w < W; ++w) accs[v][w] = accd[v][w] = av[v][w] = dv[v][w] = 0.0f;
    if (c < qf) {
      Chunk<float, W>::load(as + c * W, av[v]);
      Chunk<float, W>::load(ad + c * W, dv[v]);
    }
  }
  for (int64_t r = r0 + g.rl; r < r1; r += Geo<LPR>::RPB) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = t0 + g.q + v * LPR;
      if (c < qf) {
        const float s = gs[r * H + hv[v]];
        const float d = gd[r * H + hv[v]];
        float xv[W], o[W], gi[W];
        Chunk<TX, W>::load(x + r * F + c * W, xv);
        if (gx_in) Chunk<float, W>::load(gx_in + r * F + c * W, gi);
#pragma unroll
        for (int w = 0; w < W; ++w) {
          o[w] = s * av[v][w] + d * dv[v][w];
          if (gx_in) o[w] = gi[w] + o[w];
          accs[v][w] = fmaf(s, xv[w], accs[v][w]);
          accd[v][w] = fmaf(d, xv[w], accd[v][w]);
        }
        Chunk<TO, W>::store(gx + r * F + c * W, o);
      }
    }
  }
  const int ncols = min(LPR * V * W, F - t0 * W);
  block_colsum<LPR, V, W>(accs, lds, part + static_cast<int64_t>(blockIdx.x) * F + t0 * W, ncols);
  block_colsum<LPR, V, W>(accd, lds, part + (static_cast<int64_t>(nb) + blockIdx.x) * F + t0 * W, ncols);
}

// ---------------------------------------------------------------------------
// Head mean + bias + SiLU.
// ---------------------------------------------------------------------------
template <int W>
__global__ __launch_bounds__(kBlock) void head_silu_fwd_kernel(int64_t n, int H, int C, const float* out,
                                                               const float* bias, float* y, float* pre) {
  const int qc = C / W;
  const int64_t total = n * qc;
  const float hf = static_cast<float>(H);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t r = i / qc;
    const int c = static_cast<int>(i - r * qc);
    float s[W], b[W], p[W], o[W];
#pragma unroll
    for (int w = 0; w < W; ++w) s[w] = 0.0f;
    for (int h = 0; h < H; ++h) {
      float v[W];
      Chunk<float, W>::load(out + (r * H + h) * C + c * W, v);
#pragma unroll
      for (int w = 0; w < W; ++w) s[w] += v[w];
    }
    Chunk<float, W>::load(bias + c * W, b);
#pragma unroll
    for (int w = 0; w < W; ++w) {
      p[w] = s[w] / hf + b[w];
      o[w] = silu(p[w]);
    }
    Chunk<float, W>::store(pre + r * C + c * W, p);
    Chunk<float, W>::store(y + r * C + c * W, o);
  }
}

template <int LPR, int V, int W>
__global__ __launch_bounds__(kBlock) void head_silu_bwd_kernel(int64_t n, int H, int C, const float* gy,
                                                               const float* pre, float* gout, float* part, int nb) {
  __shared__ float lds[kBlock * V * W];
  const Geo<LPR> g;
  const int qc = C / W;
  const int t0 = blockIdx.y * LPR * V;
  const float hf = static_cast<float>(H);
  int64_t r0, r1;
  block_rows(n, nb, blockIdx.x, r0, r1);
  float acc[V][W];
#pragma unroll
  for (int v = 0; v < V; ++v)
#pragma unroll
    for (int w = 0; w < W; ++w) acc[v][w] = 0.0f;
  for (int64_t r = r0 + g.rl; r < r1; r += Geo<LPR>::RPB) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = t0 + g.q + v * LPR;
      if (c < qc) {
        float gv[W], pv[W], o[W];
        Chunk<float, W>::load(gy + r * C + c * W, gv);
        Chunk<float, W>::load(pre + r * C + c * W, pv);
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const float gp = gv[w] * silu_grad(pv[w]);
          acc[v][w] += gp;
          o[w] = gp / hf;
        }
        for (int h = 0; h < H; ++h) Chunk<float, W>::store(gout + (r * H + h) * C + c * W, o);
      }
    }
  }
  block_colsum<LPR, V, W>(acc, lds, part + static_cast<int64_t>(blockIdx.x) * C + t0 * W,
                          min(LPR * V * W, C - t0 * W));
}

// ---------------------------------------------------------------------------
// Block ops. MODE 0: dropout + LayerNorm of x; MODE 1: LayerNorm of a + b.
// ---------------------------------------------------------------------------
template <int W>
__device__ __forceinline__ void store_mask(uint8_t* m, const bool (&k)[W]) {
  if constexpr (W == 8) {
    uint32_t v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
      v[h] = (k[4 * h] ? 1u : 0u) | (k[4 * h + 1] ? 1u << 8 : 0u) | (k[4 * h + 2] ? 1u << 16 : 0u) |
             (k[4 * h + 3] ? 1u << 24 : 0u);
    *reinterpret_cast<uint2*>(m) = make_uint2(v[0], v[1]);
  } else if constexpr (W == 4) {
    const uint32_t v = (k[0] ? 1u : 0u) | (k[1] ? 1u << 8 : 0u) | (k[2] ? 1u << 16 : 0u) | (k[3] ? 1u << 24 : 0u);
    *reinterpret_cast<uint32_t*>(m) = v;
  } else {
    m[0] = k[0] ? 1 : 0;
  }
}

template <int W>
__device__ __forceinline__ void load_mask(const uint8_t* m, bool (&k)[W]) {
  if constexpr (W == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(m);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      k[w] = ((v.x >> (8 * w)) & 0xffu) != 0;
      k[4 + w] = ((v.y >> (8 * w)) & 0xffu) != 0;
    }
  } else if constexpr (W == 4) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(m);
#pragma unroll
    for (int w = 0; w < 4; ++w) k[w] = ((v >> (8 * w)) & 0xffu) != 0;
  } else {
    k[0] = m[0] != 0;
  }
}

template <int MODE, int LPR, int V, int W>
__global__ __launch_bounds__(kBlock) void ln_fwd_kernel(int64_t n, int D, const float* x, const float* x2,
                                                        const float* wt, const float* bs, float p, float eps,
                                                        uint64_t seed, float* y, float* mean, float* rstd,
                                                        uint8_t* mask, float* ycat) {
  const Geo<LPR> g;
  const int qd = D / W;
  const float scale = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
  const float df = static_cast<float>(D);
  // The lane's weight and bias chunks, loaded once (in flight with the first
  // row's loads) instead of after each row's two reductions.
  float wv[V][W], bv[V][W];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int c = g.q + v * LPR;
    Chunk<float, W>::load(wt + (c < qd ? c : 0) * W, wv[v]);
    Chunk<float, W>::load(bs + (c < qd ? c : 0) * W, bv[v]);
  }
  const int64_t step = static_cast<int64_t>(gridDim.x) * Geo<LPR>::RPB;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * Geo<LPR>::RPB + g.rl; r < n; r += step) {
    float qv[V][W];
    float s = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = g.q + v * LPR;
#pragma unroll
      for (int w = 0; w < W; ++w) qv[v][w] = 0.0f;
      if (c < qd) {
        const int64_t base = r * D + c * W;
        float xv[W];
        Chunk<float, W>::load(x + base, xv);
        if constexpr (MODE == 0) {
          bool keep[W];
#pragma unroll
          for (int w = 0; w < W; ++w) {
            keep[w] = block_keep(seed, static_cast<uint64_t>(base + w), p);
            qv[v][w] = keep[w] ? xv[w] * scale : 0.0f;
          }
          store_mask<W>(mask + base, keep);
        } else {
          float bv[W];
          Chunk<float, W>::load(x2 + base, bv);
#pragma unroll
          for (int w = 0; w < W; ++w) qv[v][w] = xv[w] + bv[w];
          if constexpr (MODE == 2) Chunk<float, W>::store(ycat + 2 * r * D + c * W, bv);
        }
#pragma unroll
        for (int w = 0; w < W; ++w) s += qv[v][w];
      }
    }
    const float mu = row_sum<LPR>(s) / df;
    float cs = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (g.q + v * LPR < qd)
#pragma unroll
        for (int w = 0; w < W; ++w) cs += (qv[v][w] - mu) * (qv[v][w] - mu);
    const float rs = 1.0f / sqrtf(row_sum<LPR>(cs) / df + eps);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = g.q + v * LPR;
      if (c < qd) {
        float o[W];
#pragma unroll
        for (int w = 0; w < W; ++w) o[w] = (qv[v][w] - mu) * rs * wv[v][w] + bv[v][w];
        Chunk<float, W>::store(y + r * D + c * W, o);
        if constexpr (MODE == 2) Chunk<float, W>::store(ycat + 2 * r * D + D + c * W, o);
      }
    }
    if (g.q == 0) {
      mean[r] = mu;
      rstd[r] = rs;
    }
  }
}

// dx (MODE 0) or dz (MODE 1) per row, and the row block's partial sums of
// gy*xhat (weight) and gy (bias): part layout [2][nb][D]. MODE 2 is MODE 1
// for an output also read as the right half of [x2 | y] ([n, 2D], gradient
// gcat): gy gains gcat's right half, and dx2 = dz + gcat's left half.
template <int MODE, int LPR, int V, int W>
__global__ __launch_bounds__(kBlock) void ln_bwd_kernel(int64_t n, int D, const float* gy, const float* x,
                                                        const float* x2, const float* wt, const float* mean,
                                                        const float* rstd, const uint8_t* mask, float p, float* dx,
                                                        float* part, int nb, const float* gcat, float* dx2) {
  __shared__ float lds[kBlock * V * W];
  const Geo<LPR> g;
  const int qd = D / W;
  const float scale = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
  const float df = static_cast<float>(D);
  int64_t r0, r1;
  block_rows(n, nb, blockIdx.x, r0, r1);
  float aw[V][W], ab[V][W], wv[V][W];
#pragma unroll
  for (int v = 0; v < V; ++v) {
#pragma unroll
    for (int w = 0; w < W; ++w) aw[v][w] = ab[v][w] = wv[v][w] = 0.0f;
    if (g.q + v * LPR < qd) Chunk<float, W>::load(wt + (g.q + v * LPR) * W, wv[v]);
  }
  // Every lane of a row runs the same trip count (the loop bound is per row).
  for (int64_t r = r0 + g.rl; r < r1; r += Geo<LPR>::RPB) {
    const float mu = mean[r];
    const float rs = rstd[r];
    float xh[V][W], dn[V][W], gv[V][W];
    float gleft[MODE == 2 ? V : 1][W];
    bool keep[V][W];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = g.q + v * LPR;
#pragma unroll
      for (int w = 0; w < W; ++w) {
        xh[v][w] = dn[v][w] = gv[v][w] = 0.0f;
        keep[v][w] = true;
      }
      if (c < qd) {
        const int64_t base = r * D + c * W;
        float xv[W];
        Chunk<float, W>::load(x + base, xv);
        Chunk<float, W>::load(gy + base, gv[v]);
        if constexpr (MODE == 2) {
          float gr[W];
          Chunk<float, W>::load(gcat + 2 * r * D + D + c * W, gr);
          Chunk<float, W>::load(gcat + 2 * r * D + c * W, gleft[v]);
#pragma unroll
          for (int w = 0; w < W; ++w) gv[v][w] += gr[w];
        }
        float qv[W];
        if constexpr (MODE == 0) {
          load_mask<W>(mask + base, keep[v]);
#pragma unroll
          for (int w = 0; w < W; ++w) qv[w] = keep[v][w] ? xv[w] * scale : 0.0f;
        } else {
          float bv[W];
          Chunk<float, W>::load(x2 + base, bv);
#pragma unroll
          for (int w = 0; w < W; ++w) qv[w] = xv[w] + bv[w];
        }
#pragma unroll
        for (int w = 0; w < W; ++w) {
          xh[v][w] = (qv[w] - mu) * rs;
          dn[v][w] = gv[v][w] * wv[v][w];
          s1 += dn[v][w];
          s2 += dn[v][w] * xh[v][w];
          aw[v][w] = fmaf(gv[v][w], xh[v][w], aw[v][w]);
          ab[v][w] += gv[v][w];
        }
      }
    }
    s1 = row_sum<LPR>(s1);
    s2 = row_sum<LPR>(s2);
    const float k = rs / df;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = g.q + v * LPR;
      if (c < qd) {
        float o[W];
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const float dq = k * (df * dn[v][w] - s1 - xh[v][w] * s2);
          o[w] = MODE == 0 ? (keep[v][w] ? dq * scale : 0.0f) : dq;
        }
        Chunk<float, W>::store(dx + r * D + c * W, o);
        if constexpr (MODE == 2) {
#pragma unroll
          for (int w = 0; w < W; ++w) o[w] += gleft[v][w];
          Chunk<float, W>::store(dx2 + r * D + c * W, o);
        }
      }
    }
  }
  block_colsum<LPR, V, W>(aw, lds, part + static_cast<int64_t>(blockIdx.x) * D, D);
  block_colsum<LPR, V, W>(ab, lds, part + (static_cast<int64_t>(nb) + blockIdx.x) * D, D);
}

template <int W>
__global__ __launch_bounds__(kBlock) void gamma_fwd_kernel(int64_t n, int D, const float* h, const float* gsrc,
                                                           const float* gamma, float p, uint64_t seed, float* y,
                                                           uint8_t* mask) {
  const int qd = D / W;
  const int64_t total = n * qd;
  const float scale = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t r = i / qd;
    const int c = static_cast<int>(i - r * qd);
    const int64_t base = r * D + c * W;
    float hv[W], gv[W], gm[W], o[W];
    bool keep[W];
    Chunk<float, W>::load(h + base, hv);
    Chunk<float, W>::load(gsrc + base, gv);
    Chunk<float, W>::load(gamma + c * W, gm);
#pragma unroll
    for (int w = 0; w < W; ++w) {
      keep[w] = block_keep(seed, static_cast<uint64_t>(base + w), p);
      const float gd = keep[w] ? gv[w] * scale : 0.0f;
      o[w] = hv[w] + gm[w] * gd;
    }
    store_mask<W>(mask + base, keep);
    Chunk<float, W>::store(y + base, o);
  }
}

// grad_g = gy * gamma * m and the row block's partial sum of gy * g * m
// (m = keep / (1 - p)).
template <int LPR, int V, int W>
__global__ __launch_bounds__(kBlock) void gamma_bwd_kernel(int64_t n, int D, const float* gy, const float* gsrc,
                                                           const float* gamma, const uint8_t* mask, float p,
                                                           float* grad_g, float* part, int nb) {
  __shared__ float lds[kBlock * V * W];
  const Geo<LPR> g;
  const int qd = D / W;
  const float scale = p > 0.0f ? 1.0f / (1.0f - p) : 1.0f;
  int64_t r0, r1;
  block_rows(n, nb, blockIdx.x, r0, r1);
  float acc[V][W], gm[V][W];
#pragma unroll
  for (int v = 0; v < V; ++v) {
#pragma unroll
    for (int w = 0; w < W; ++w) acc[v][w] = gm[v][w] = 0.0f;
    if (g.q + v * LPR < qd) Chunk<float, W>::load(gamma + (g.q + v * LPR) * W, gm[v]);
  }
  for (int64_t r = r0 + g.rl; r < r1; r += Geo<LPR>::RPB) {
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int c = g.q + v * LPR;
      if (c < qd) {
        const int64_t base = r * D + c * W;
        float go[W], gv[W], o[W];
        bool keep[W];
        Chunk<float, W>::load(gy + base, go);
        Chunk<float, W>::load(gsrc + base, gv);
        load_mask<W>(mask + base, keep);
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const float m = keep[w] ? scale : 0.0f;
          o[w] = go[w] * gm[v][w] * m;
          acc[v][w] += go[w] * gv[w] * m;
        }
        Chunk<float, W>::store(grad_g + base, o);
      }
    }
  }
  block_colsum<LPR, V, W>(acc, lds, part + static_cast<int64_t>(blockIdx.x) * D, D);
}

// ---------------------------------------------------------------------------
// Host helpers.
// ---------------------------------------------------------------------------
inline int chunk_width(int width, std::initializer_list<const void*> ptrs) {
  if (width % 4 != 0) return 1;
  for (const void* p : ptrs)
    if (!aligned16(p)) return 1;
  return 4;
}

// Rows of at least 128 aligned floats: eight values per lane (two 16-byte
// accesses), so a wavefront holds two rows of 256 instead of one.
inline int wide_chunks(int width, int w) { return w == 4 && width % 8 == 0 && width >= 128 ? 8 : w; }

int check_rows(const char* who, int64_t n, int D) {
  if (n < 0) return set_error(kInvalid, "%s: negative row count", who);
  if (D < 1 || D > 256) return set_error(kInvalid, "%s: requires 1<=D<=256, got %d", who, D);
  return kOk;
}

int64_t colsum_bytes(int64_t n, int width, int quantities) {
  return 4LL * quantities * colsum_blocks(n) * width;
}

// Attention logits over float32 or bf16-stored x (TX = bf16h).
template <typename TX>
int attn_fwd_impl(const char* who, void* stream, int64_t n, int32_t H, int32_t C, const TX* x, const float* att_src,
                  const float* att_dst, float* alpha_src, float* alpha_dst) {
  if (n < 0 || H < 1 || C < 1)
    return set_error(kInvalid, "%s: bad shape n=%lld H=%d C=%d", who, static_cast<long long>(n), H, C);
  if (n == 0) return kOk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t rows = n * H;
  if constexpr (std::is_same_v<TX, bf16h>) {
    // bf16 rows eight values (16 bytes) per lane
    if (C % 8 == 0 && aligned16(x) && aligned16(att_src) && aligned16(att_dst)) {
      const bf16* xb = reinterpret_cast<const bf16*>(x);
      const int rc = with_geo(C / 8, [&](auto LC, auto VC) {
        constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
        hipLaunchKernelGGL((attn_fwd_kernel<L, V, 8, bf16>), dim3(grid_for(rows, Geo<L>::RPB)), dim3(kBlock), 0, st,
                           rows, H, C, xb, att_src, att_dst, alpha_src, alpha_dst);
        return check_launch(who);
      });
      if (rc >= 0) return rc;
    }
  } else {
    // fp32 rows of at least 128 values eight per lane (two 16-byte loads):
    // two rows per wavefront instead of one
    if (C % 8 == 0 && C >= 128 && aligned16(x) && aligned16(att_src) && aligned16(att_dst)) {
      const int rc = with_geo(C / 8, [&](auto LC, auto VC) {
        constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
        hipLaunchKernelGGL((attn_fwd_kernel<L, V, 8, float>), dim3(grid_for(rows, Geo<L>::RPB)), dim3(kBlock), 0,
                           st, rows, H, C, x, att_src, att_dst, alpha_src, alpha_dst);
        return check_launch(who);
      });
      if (rc >= 0) return rc;
    }
  }
  const int W = chunk_width(C, {x, att_src, att_dst});
  const int rc = with_geo(C / W, [&](auto LC, auto VC) {
    constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
    const int grid = grid_for(rows, Geo<L>::RPB);
    if (W == 4)
      hipLaunchKernelGGL((attn_fwd_kernel<L, V, 4, TX>), dim3(grid), dim3(kBlock), 0, st, rows, H, C, x, att_src,
                         att_dst, alpha_src, alpha_dst);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<L, V, 1, TX>), dim3(grid), dim3(kBlock), 0, st, rows, H, C, x, att_src,
                         att_dst, alpha_src, alpha_dst);
    return check_launch(who);
  });
  if (rc < 0) return set_error(kInvalid, "%s: channels=%d too wide (max %d)", who, C, 256 * W);
  return rc;
}

// Attention logits backward; grad_x = grad_x_in (when not null; it may alias
// grad_x) + the logits' term.
template <typename TX>
int attn_bwd_impl(const char* who, void* stream, int64_t n, int32_t H, int32_t C, const float* grad_src,
                  const float* grad_dst, const TX* x, const float* att_src, const float* att_dst,
                  const float* grad_x_in, float* grad_x, float* grad_att_src, float* grad_att_dst, void* workspace,
                  int64_t workspace_bytes, bool grad_x_bf16 = false) {
  if (n < 0 || H < 1 || C < 1) return set_error(kInvalid, "%s: bad shape", who);
  const int F = H * C;
  if (workspace_bytes < colsum_bytes(n, F, 2)) return set_error(kInvalid, "%s: workspace too small", who);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = colsum_blocks(n);
  float* part = static_cast<float*>(workspace);
  if constexpr (std::is_same_v<TX, bf16h>) {
    // bf16 rows eight values (16 bytes) per lane
    if (n > 0 && C % 8 == 0 && aligned16(x) && aligned16(att_src) && aligned16(att_dst) && aligned16(grad_x) &&
        (!grad_x_in || aligned16(grad_x_in))) {
      const bf16* xb = reinterpret_cast<const bf16*>(x);
      const int qf8 = F / 8;
      auto launch8 = [&](auto LC, auto VC) {
        constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
        const dim3 grid(nb, (qf8 + L * V - 1) / (L * V));
        if (grad_x_bf16)
          hipLaunchKernelGGL((attn_bwd_kernel<L, V, 8, bf16, bf16>), grid, dim3(kBlock), 0, st, n, H, C, grad_src,
                             grad_dst, xb, att_src, att_dst, grad_x_in, reinterpret_cast<bf16*>(grad_x), part, nb);
        else
          hipLaunchKernelGGL((attn_bwd_kernel<L, V, 8, bf16>), grid, dim3(kBlock), 0, st, n, H, C, grad_src, grad_dst,
                             xb, att_src, att_dst, grad_x_in, grad_x, part, nb);
        return check_launch(who);
      };
      // rows of more than 128 chunks take column tiles of 128 (two chunks per
      // lane): four chunks of eight values held 197 VGPRs, two waves per SIMD
      const int rc = qf8 > 128 ? launch8(IC<64>(), IC<2>()) : with_geo(qf8, launch8);
      if (rc) return rc;
      return launch_colsum(st, part, nb, F, 2, grad_att_src, grad_att_dst, who);
    }
  }
  if (grad_x_bf16 && n > 0)
    return set_error(kInvalid, "%s: a bf16 grad_x needs bf16 x with channels a multiple of 8 and 16-byte aligned "
                     "rows", who);
  const int W = grad_x_in ? chunk_width(C, {x, att_src, att_dst, grad_x, grad_x_in})
                          : chunk_width(C, {x, att_src, att_dst, grad_x});
  const int qf = F / W;
  if (n > 0) {
    auto launch = [&](auto LC, auto VC) {
      constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
      const dim3 grid(nb, (qf + L * V - 1) / (L * V));
      if (W == 4)
        hipLaunchKernelGGL((attn_bwd_kernel<L, V, 4, TX>), grid, dim3(kBlock), 0, st, n, H, C, grad_src, grad_dst, x,
                           att_src, att_dst, grad_x_in, grad_x, part, nb);
      else
        hipLaunchKernelGGL((attn_bwd_kernel<L, V, 1, TX>), grid, dim3(kBlock), 0, st, n, H, C, grad_src, grad_dst, x,
                           att_src, att_dst, grad_x_in, grad_x, part, nb);
      return check_launch(who);
    };
    const int rc = qf > 256 ? launch(IC<64>(), IC<4>()) : with_geo(qf, launch);
    if (rc) return rc;
  } else {
    return zero_outputs(st, grad_att_src, F, grad_att_dst, F, who);
  }
  return launch_colsum(st, part, nb, F, 2, grad_att_src, grad_att_dst, who);
}

}  // namespace nodeops
}  // namespace cign

using namespace cign;
using namespace cign::rowops;
using namespace cign::nodeops;

extern "C" {

// Workspace bytes of a backward whose parameter gradient sums `quantities`
// vectors of `width` floats over n rows (see each entry point).
int64_t cign_colsum_workspace_bytes(int64_t n, int32_t width, int32_t quantities) {
  return colsum_bytes(n, width, quantities);
}

// ---- attention logits --------------------------------------------------------
int cign_attn_logits_fwd(void* stream, int64_t n, int32_t H, int32_t C, const float* x, const float* att_src,
                         const float* att_dst, float* alpha_src, float* alpha_dst) {
  return attn_fwd_impl("cign_attn_logits_fwd", stream, n, H, C, x, att_src, att_dst, alpha_src, alpha_dst);
}

int cign_attn_logits_fwd_bf16(void* stream, int64_t n, int32_t H, int32_t C, const void* x, const float* att_src,
                              const float* att_dst, float* alpha_src, float* alpha_dst) {
  return attn_fwd_impl("cign_attn_logits_fwd_bf16", stream, n, H, C, static_cast<const bf16h*>(x), att_src, att_dst,
                       alpha_src, alpha_dst);
}

int cign_attn_logits_bwd(void* stream, int64_t n, int32_t H, int32_t C, const float* grad_src, const float* grad_dst,
                         const float* x, const float* att_src, const float* att_dst, float* grad_x,
                         float* grad_att_src, float* grad_att_dst, void* workspace, int64_t workspace_bytes) {
  return attn_bwd_impl("cign_attn_logits_bwd", stream, n, H, C, grad_src, grad_dst, x, att_src, att_dst, nullptr,
                       grad_x, grad_att_src, grad_att_dst, workspace, workspace_bytes);
}

int cign_attn_logits_bwd_acc(void* stream, int64_t n, int32_t H, int32_t C, int32_t x_dtype, int32_t grad_x_dtype,
                             const float* grad_src, const float* grad_dst, const void* x, const float* att_src,
                             const float* att_dst, const float* grad_x_in, void* grad_x, float* grad_att_src,
                             float* grad_att_dst, void* workspace, int64_t workspace_bytes) {
  const char* who = "cign_attn_logits_bwd_acc";
  if (grad_x_dtype != kF32 && !(grad_x_dtype == kBF16 && x_dtype == kBF16))
    return set_error(kInvalid, "%s: grad_x_dtype must be 0 (float32), or 1 (bf16) with bf16 x", who);
  if (grad_x_dtype == kBF16 && grad_x_in == grad_x)
    return set_error(kInvalid, "%s: a bf16 grad_x cannot alias the float32 grad_x_in", who);
  float* gx = static_cast<float*>(grad_x);
  if (x_dtype == kF32)
    return attn_bwd_impl(who, stream, n, H, C, grad_src, grad_dst, static_cast<const float*>(x), att_src, att_dst,
                         grad_x_in, gx, grad_att_src, grad_att_dst, workspace, workspace_bytes);
  if (x_dtype == kBF16)
    return attn_bwd_impl(who, stream, n, H, C, grad_src, grad_dst, static_cast<const bf16h*>(x), att_src, att_dst,
                         grad_x_in, gx, grad_att_src, grad_att_dst, workspace, workspace_bytes,
                         grad_x_dtype == kBF16);
  return set_error(kInvalid, "%s: x_dtype must be 0 (float32) or 1 (bf16), got %d", who, x_dtype);
}

// ---- head mean + bias + SiLU ----------------------------------------------
int cign_head_silu_fwd(void* stream, int64_t n, int32_t H, int32_t C, const float* out, const float* bias, float* y,
                       float* pre) {
  if (n < 0 || H < 1 || C < 1) return set_error(kInvalid, "cign_head_silu_fwd: bad shape");
  if (n == 0) return kOk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int W = chunk_width(C, {out, bias, y, pre});
  const int grid = grid_for(n * (C / W), kBlock);
  if (W == 4)
    hipLaunchKernelGGL((head_silu_fwd_kernel<4>), dim3(grid), dim3(kBlock), 0, st, n, H, C, out, bias, y, pre);
  else
    hipLaunchKernelGGL((head_silu_fwd_kernel<1>), dim3(grid), dim3(kBlock), 0, st, n, H, C, out, bias, y, pre);
  return check_launch("cign_head_silu_fwd");
}

int cign_head_silu_bwd(void* stream, int64_t n, int32_t H, int32_t C, const float* grad_y, const float* pre,
                       float* grad_out, float* grad_bias, void* workspace, int64_t workspace_bytes) {
  if (n < 0 || H < 1 || C < 1) return set_error(kInvalid, "cign_head_silu_bwd: bad shape");
  if (workspace_bytes < colsum_bytes(n, C, 1)) return set_error(kInvalid, "cign_head_silu_bwd: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = colsum_blocks(n);
  float* part = static_cast<float*>(workspace);
  const int W = chunk_width(C, {grad_y, pre, grad_out});
  const int qc = C / W;
  if (n > 0) {
    auto launch = [&](auto LC, auto VC) {
      constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
      const dim3 grid(nb, (qc + L * V - 1) / (L * V));
      if (W == 4)
        hipLaunchKernelGGL((head_silu_bwd_kernel<L, V, 4>), grid, dim3(kBlock), 0, st, n, H, C, grad_y, pre, grad_out,
                           part, nb);
      else
        hipLaunchKernelGGL((head_silu_bwd_kernel<L, V, 1>), grid, dim3(kBlock), 0, st, n, H, C, grad_y, pre, grad_out,
                           part, nb);
      return check_launch("cign_head_silu_bwd");
    };
    const int rc = qc > 256 ? launch(IC<64>(), IC<4>()) : with_geo(qc, launch);
    if (rc) return rc;
  } else {
    return zero_outputs(st, grad_bias, C, nullptr, 0, "cign_head_silu_bwd");
  }
  return launch_colsum(st, part, nb, C, 1, grad_bias, nullptr, "cign_head_silu_bwd");
}

// ---- block ops ------------------------------------------------------------
static int ln_fwd(int mode, void* stream, int64_t n, int32_t D, const float* x, const float* x2, const float* w,
                  const float* b, float p, float eps, uint64_t seed, float* y, float* mean, float* rstd,
                  uint8_t* mask, const char* who, float* ycat = nullptr) {
  int rc = check_rows(who, n, D);
  if (rc) return rc;
  if (!(p >= 0.0f && p < 1.0f)) return set_error(kInvalid, "%s: dropout_p must be in [0,1)", who);
  if (n == 0) return kOk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int W = wide_chunks(D, chunk_width(D, {x, x2 ? x2 : x, w, b, y, mask ? static_cast<const void*>(mask) : x,
                                                ycat ? ycat : y}));
  return with_geo(D / W, [&](auto LC, auto VC) {
    constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
    const int grid = grid_for(n, Geo<L>::RPB);
#define CIGN_LN_FWD(M, WW)                                                                                          \
  hipLaunchKernelGGL((ln_fwd_kernel<M, L, V, WW>), dim3(grid), dim3(kBlock), 0, st, n, D, x, x2, w, b, p, eps, seed, \
                     y, mean, rstd, mask, ycat)
    if (mode == 0) {
      if (W == 8) CIGN_LN_FWD(0, 8); else if (W == 4) CIGN_LN_FWD(0, 4); else CIGN_LN_FWD(0, 1);
    } else if (mode == 1) {
      if (W == 8) CIGN_LN_FWD(1, 8); else if (W == 4) CIGN_LN_FWD(1, 4); else CIGN_LN_FWD(1, 1);
    } else {
      if (W == 8) CIGN_LN_FWD(2, 8); else if (W == 4) CIGN_LN_FWD(2, 4); else CIGN_LN_FWD(2, 1);
    }
#undef CIGN_LN_FWD
    return check_launch(who);
  });
}

static int ln_bwd(int mode, void* stream, int64_t n, int32_t D, const float* gy, const float* x, const float* x2,
                  const float* w, const float* mean, const float* rstd, const uint8_t* mask, float p, float* dx,
                  float* dw, float* db, void* workspace, int64_t workspace_bytes, const char* who,
                  const float* gcat = nullptr, float* dx2 = nullptr) {
  int rc = check_rows(who, n, D);
  if (rc) return rc;
  if (workspace_bytes < colsum_bytes(n, D, 2)) return set_error(kInvalid, "%s: workspace too small", who);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = colsum_blocks(n);
  float* part = static_cast<float*>(workspace);
  if (n > 0) {
    const int W = wide_chunks(D, chunk_width(D, {gy, x, x2 ? x2 : x, w, dx, mask ? static_cast<const void*>(mask) : x,
                                                 gcat ? gcat : gy, dx2 ? dx2 : dx}));
    rc = with_geo(D / W, [&](auto LC, auto VC) {
      constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
#define CIGN_LN_BWD(M, WW)                                                                                           \
  hipLaunchKernelGGL((ln_bwd_kernel<M, L, V, WW>), dim3(nb), dim3(kBlock), 0, st, n, D, gy, x, x2, w, mean, rstd, mask, \
                     p, dx, part, nb, gcat, dx2)
      if (mode == 0) {
        if (W == 8) CIGN_LN_BWD(0, 8); else if (W == 4) CIGN_LN_BWD(0, 4); else CIGN_LN_BWD(0, 1);
      } else if (mode == 1) {
        if (W == 8) CIGN_LN_BWD(1, 8); else if (W == 4) CIGN_LN_BWD(1, 4); else CIGN_LN_BWD(1, 1);
      } else {
        if (W == 8) CIGN_LN_BWD(2, 8); else if (W == 4) CIGN_LN_BWD(2, 4); else CIGN_LN_BWD(2, 1);
      }
#undef CIGN_LN_BWD
      return check_launch(who);
    });
    if (rc) return rc;
  } else {
    return zero_outputs(st, dw, D, db, D, who);
  }
  return launch_colsum(st, part, nb, D, 2, dw, db, who);
}

int cign_dropout_ln_fwd(void* stream, int64_t n, int32_t D, const float* x, const float* weight, const float* bias,
                        float dropout_p, float eps, uint64_t seed, float* y, float* mean, float* rstd, uint8_t* mask) {
  return ln_fwd(0, stream, n, D, x, nullptr, weight, bias, dropout_p, eps, seed, y, mean, rstd, mask,
                "cign_dropout_ln_fwd");
}

int cign_dropout_ln_bwd(void* stream, int64_t n, int32_t D, const float* grad_y, const float* x, const float* weight,
                        const float* mean, const float* rstd, const uint8_t* mask, float dropout_p, float* grad_x,
                        float* grad_weight, float* grad_bias, void* workspace, int64_t workspace_bytes) {
  return ln_bwd(0, stream, n, D, grad_y, x, nullptr, weight, mean, rstd, mask, dropout_p, grad_x, grad_weight,
                grad_bias, workspace, workspace_bytes, "cign_dropout_ln_bwd");
}

int cign_add_ln_fwd(void* stream, int64_t n, int32_t D, const float* a, const float* b, const float* weight,
                    const float* bias, float eps, float* y, float* mean, float* rstd) {
  return ln_fwd(1, stream, n, D, a, b, weight, bias, 0.0f, eps, 0, y, mean, rstd, nullptr, "cign_add_ln_fwd");
}

int cign_add_ln_bwd(void* stream, int64_t n, int32_t D, const float* grad_y, const float* a, const float* b,
                    const float* weight, const float* mean, const float* rstd, float* grad_z, float* grad_weight,
                    float* grad_bias, void* workspace, int64_t workspace_bytes) {
  return ln_bwd(1, stream, n, D, grad_y, a, b, weight, mean, rstd, nullptr, 0.0f, grad_z, grad_weight, grad_bias,
                workspace, workspace_bytes, "cign_add_ln_bwd");
}

int cign_add_ln_cat_fwd(void* stream, int64_t n, int32_t D, const float* a, const float* b, const float* weight,
                        const float* bias, float eps, float* y, float* cat, float* mean, float* rstd) {
  return ln_fwd(2, stream, n, D, a, b, weight, bias, 0.0f, eps, 0, y, mean, rstd, nullptr, "cign_add_ln_cat_fwd",
                cat);
}

int cign_add_ln_cat_bwd(void* stream, int64_t n, int32_t D, const float* grad_y, const float* grad_cat, const float* a,
                        const float* b, const float* weight, const float* mean, const float* rstd, float* grad_a,
                        float* grad_b, float* grad_weight, float* grad_bias, void* workspace, int64_t workspace_bytes) {
  return ln_bwd(2, stream, n, D, grad_y, a, b, weight, mean, rstd, nullptr, 0.0f, grad_a, grad_weight, grad_bias,
                workspace, workspace_bytes, "cign_add_ln_cat_bwd", grad_cat, grad_b);
}

int cign_gamma_residual_fwd(void* stream, int64_t n, int32_t D, const float* h, const float* g, const float* gamma,
                            float dropout_p, uint64_t seed, float* y, uint8_t* mask) {
  int rc = check_rows("cign_gamma_residual_fwd", n, D);
  if (rc) return rc;
  if (!(dropout_p >= 0.0f && dropout_p < 1.0f))
    return set_error(kInvalid, "cign_gamma_residual_fwd: dropout_p must be in [0,1)");
  if (n == 0) return kOk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int W = chunk_width(D, {h, g, gamma, y, mask});
  const int grid = grid_for(n * (D / W), kBlock);
  if (W == 4)
    hipLaunchKernelGGL((gamma_fwd_kernel<4>), dim3(grid), dim3(kBlock), 0, st, n, D, h, g, gamma, dropout_p, seed, y,
                       mask);
  else
    hipLaunchKernelGGL((gamma_fwd_kernel<1>), dim3(grid), dim3(kBlock), 0, st, n, D, h, g, gamma, dropout_p, seed, y,
                       mask);
  return check_launch("cign_gamma_residual_fwd");
}

int cign_gamma_residual_bwd(void* stream, int64_t n, int32_t D, const float* grad_y, const float* g,
                            const float* gamma, const uint8_t* mask, float dropout_p, float* grad_g, float* grad_gamma,
                            void* workspace, int64_t workspace_bytes) {
  int rc = check_rows("cign_gamma_residual_bwd", n, D);
  if (rc) return rc;
  if (workspace_bytes < colsum_bytes(n, D, 1))
    return set_error(kInvalid, "cign_gamma_residual_bwd: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int nb = colsum_blocks(n);
  float* part = static_cast<float*>(workspace);
  if (n > 0) {
    const int W = chunk_width(D, {grad_y, g, gamma, mask, grad_g});
    rc = with_geo(D / W, [&](auto LC, auto VC) {
      constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
      if (W == 4)
        hipLaunchKernelGGL((gamma_bwd_kernel<L, V, 4>), dim3(nb), dim3(kBlock), 0, st, n, D, grad_y, g, gamma, mask,
                           dropout_p, grad_g, part, nb);
      else
        hipLaunchKernelGGL((gamma_bwd_kernel<L, V, 1>), dim3(nb), dim3(kBlock), 0, st, n, D, grad_y, g, gamma, mask,
                           dropout_p, grad_g, part, nb);
      return check_launch("cign_gamma_residual_bwd");
    });
    if (rc) return rc;
  } else {
    return zero_outputs(st, grad_gamma, D, nullptr, 0, "cign_gamma_residual_bwd");
  }
  return launch_colsum(st, part, nb, D, 1, grad_gamma, nullptr, "cign_gamma_residual_bwd");
}

}  // extern "C"
