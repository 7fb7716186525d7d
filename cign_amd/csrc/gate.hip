// Node-mode hop gate of the Clifford block and its C-ABI.
//
// compute_hop_gate (generic_engine/model_cign.py:721-749), node mode:
//   score 0 (old): s = [H | C];  score 1 (new): s = [H + C | |H - C|]   (s: [n, 2D])
//   logits[n,k] = <s[n,:], weight[k,:]> + bias[k],  alpha[n,:] = softmax_k(logits)
// Backward:
//   gl[n,k] = alpha[n,k] (g[n,k] - sum_j alpha[n,j] g[n,j])       (softmax)
//   gs[n,:] = sum_k gl[n,k] weight[k,:]
//   score 0: gH = gs[:, :D], gC = gs[:, D:]
//   score 1: gH = gs1 + sgn(H-C) gs2, gC = gs1 - sgn(H-C) gs2       (sgn(0) = 0, torch's abs')
//   grad_weight[k,:] = sum_n gl[n,k] s[n,:],  grad_bias[k] = sum_n gl[n,k]
// The forward and the row part of the backward put a node's D-chunks on one
// lane group (rowops.h); the parameter gradients are deterministic row-block
// partials added by colsum_kernel.
#include "rowops.h"

namespace cign {
namespace gate {
using namespace rowops;

constexpr int kMaxGateHops = 16;

template <int W>
__device__ __forceinline__ void score_chunk(const float (&h)[W], const float (&c)[W], int mode, float (&s1)[W],
                                            float (&s2)[W]) {
#pragma unroll
  for (int w = 0; w < W; ++w) {
    if (mode == 0) {
      s1[w] = h[w];
      s2[w] = c[w];
    } else {
      s1[w] = h[w] + c[w];
      s2[w] = fabsf(h[w] - c[w]);
    }
  }
}

// The lane's chunks (q = q0 + v*LPR) of the gate weight rows k: [weight[k,
// :D] chunk, weight[k, D:] chunk]. With a compile-time hop count (KT > 0) they
// are loaded once per thread into registers (chunks past the row read chunk
// 0; they meet zero scores and are never stored); otherwise each use reads
// global memory. Per-row weight loads, each in its own guarded block, had
// made every row wait on K dependent loads.
template <int LPR, int V, int W, int KT>
struct GateW {
  static constexpr int KR = KT > 0 ? KT : 1;
  float a[KR][V][W], b[KR][V][W];
  const float* wt;
  int D, qd, q0;
  __device__ __forceinline__ GateW(const float* w, int d, int q) : wt(w), D(d), qd(d / W), q0(q) {
    if constexpr (KT > 0) {
#pragma unroll
      for (int k = 0; k < KT; ++k)
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int qq = q0 + v * LPR;
          const float* wk = wt + static_cast<int64_t>(k) * 2 * D + (qq < qd ? qq : 0) * W;
          Chunk<float, W>::load(wk, a[k][v]);
          Chunk<float, W>::load(wk + D, b[k][v]);
        }
    }
  }
  __device__ __forceinline__ void get(int k, int v, float (&x)[W], float (&y)[W]) const {
    if constexpr (KT > 0) {
#pragma unroll
      for (int w = 0; w < W; ++w) {
        x[w] = a[k][v][w];
        y[w] = b[k][v][w];
      }
    } else {
      const float* wk = wt + static_cast<int64_t>(k) * 2 * D + (q0 + v * LPR) * W;
      Chunk<float, W>::load(wk, x);
      Chunk<float, W>::load(wk + D, y);
    }
  }
};

// Hop counts with a compile-time kernel (loop bound KC, weights in registers).
template <int KT>
constexpr int gate_kc() {
  return KT > 0 ? KT : kMaxGateHops;
}

template <int LPR, int V, int W, int KT>
__global__ __launch_bounds__(kBlock) void hop_gate_fwd_kernel(int64_t n, int D, int K, int mode, const float* H,
                                                              const float* C, const float* wt, const float* bias,
                                                              float* alpha) {
  constexpr int KC = gate_kc<KT>();
  const Geo<LPR> g;
  const int qd = D / W;
  const GateW<LPR, V, W, KT> gw(wt, D, g.q);
  const int64_t step = static_cast<int64_t>(gridDim.x) * Geo<LPR>::RPB;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * Geo<LPR>::RPB + g.rl; r < n; r += step) {
    float s1[V][W], s2[V][W];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int q = g.q + v * LPR;
      float h[W], c[W];
#pragma unroll
      for (int w = 0; w < W; ++w) h[w] = c[w] = 0.0f;
      if (q < qd) {
        Chunk<float, W>::load(H + r * D + q * W, h);
        Chunk<float, W>::load(C + r * D + q * W, c);
      }
      score_chunk<W>(h, c, mode, s1[v], s2[v]);
    }
    float logit[KC];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      if (KT > 0 || k < K) {
        float d = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int q = g.q + v * LPR;
          if (KT > 0 || q < qd) {
            float a[W], b[W];
            gw.get(k, v, a, b);
#pragma unroll
            for (int w = 0; w < W; ++w) d = fmaf(s1[v][w], a[w], fmaf(s2[v][w], b[w], d));
          }
        }
        logit[k] = row_sum<LPR>(d) + bias[k];
        m = fmaxf(m, logit[k]);
      }
    }
    float tot = 0.0f;
#pragma unroll
    for (int k = 0; k < KC; ++k)
      if (KT > 0 || k < K) {
        logit[k] = expf(logit[k] - m);
        tot += logit[k];
      }
#pragma unroll
    for (int k = 0; k < KC; ++k)
      if ((KT > 0 || k < K) && g.q == (k % LPR)) alpha[r * K + k] = logit[k] / tot;
  }
}

// Row part of the backward: gl (to the workspace), grad_H, grad_C.
template <int LPR, int V, int W, int KT>
__global__ __launch_bounds__(kBlock) void hop_gate_bwd_rows_kernel(int64_t n, int D, int K, int mode, const float* H,
                                                                   const float* C, const float* wt, const float* alpha,
                                                                   const float* galpha, float* gl_out, float* gH,
                                                                   float* gC) {
  constexpr int KC = gate_kc<KT>();
  const Geo<LPR> g;
  const int qd = D / W;
  const GateW<LPR, V, W, KT> gw(wt, D, g.q);
  const int64_t step = static_cast<int64_t>(gridDim.x) * Geo<LPR>::RPB;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * Geo<LPR>::RPB + g.rl; r < n; r += step) {
    float gl[KC];
    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < KC; ++k)
      if (KT > 0 || k < K) dot += alpha[r * K + k] * galpha[r * K + k];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      gl[k] = 0.0f;
      if (KT > 0 || k < K) gl[k] = alpha[r * K + k] * (galpha[r * K + k] - dot);
    }
#pragma unroll
    for (int k = 0; k < KC; ++k)
      if ((KT > 0 || k < K) && g.q == (k % LPR)) gl_out[r * K + k] = gl[k];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int q = g.q + v * LPR;
      if (q < qd) {
        float g1[W], g2[W];
#pragma unroll
        for (int w = 0; w < W; ++w) g1[w] = g2[w] = 0.0f;
#pragma unroll
        for (int k = 0; k < KC; ++k) {
          if (KT > 0 || k < K) {
            float a[W], b[W];
            gw.get(k, v, a, b);
#pragma unroll
            for (int w = 0; w < W; ++w) {
              g1[w] = fmaf(gl[k], a[w], g1[w]);
              g2[w] = fmaf(gl[k], b[w], g2[w]);
            }
          }
        }
        float oh[W], oc[W];
        if (mode == 0) {
#pragma unroll
          for (int w = 0; w < W; ++w) {
            oh[w] = g1[w];
            oc[w] = g2[w];
          }
        } else {
          float h[W], c[W];
          Chunk<float, W>::load(H + r * D + q * W, h);
          Chunk<float, W>::load(C + r * D + q * W, c);
#pragma unroll
          for (int w = 0; w < W; ++w) {
            const float d = h[w] - c[w];
            const float sg = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
            oh[w] = g1[w] + sg * g2[w];
            oc[w] = g1[w] - sg * g2[w];
          }
        }
        Chunk<float, W>::store(gH + r * D + q * W, oh);
        Chunk<float, W>::store(gC + r * D + q * W, oc);
      }
    }
  }
}

// Column part: row block blockIdx.x, tile blockIdx.y of kBlock chunks of the
// 2D score columns. part_w [nb][K*2D] (column k*2D + j), part_b [nb][K].
// Rows go four at a time: their score chunks and gl values are all loaded
// before any is used.
template <int W, int KT>
__global__ __launch_bounds__(kBlock) void hop_gate_bwd_cols_kernel(int64_t n, int D, int K, int mode,
                                                                   const float* H, const float* C, const float* gl,
                                                                   float* part_w, float* part_b, int nb) {
  constexpr int KC = gate_kc<KT>();
  constexpr int R = 4;
  const int qs = 2 * D / W;  // score chunks (D % W == 0, so no chunk straddles the halves)
  const int q = blockIdx.y * kBlock + threadIdx.x;
  int64_t r0, r1;
  block_rows(n, nb, blockIdx.x, r0, r1);
  const bool col = q < qs;
  if (col) {
    float acc[KC][W];
#pragma unroll
    for (int k = 0; k < KC; ++k)
#pragma unroll
      for (int w = 0; w < W; ++w) acc[k][w] = 0.0f;
    const bool second = q * W >= D;
    const int d0 = second ? q * W - D : q * W;
    auto add_rows = [&](int64_t r, auto UC) {
      constexpr int U = decltype(UC)::value;
      float h[U][W], c[U][W], gk[U][KC];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        Chunk<float, W>::load(H + (r + u) * D + d0, h[u]);
        Chunk<float, W>::load(C + (r + u) * D + d0, c[u]);
#pragma unroll
        for (int k = 0; k < KC; ++k) gk[u][k] = (KT > 0 || k < K) ? gl[(r + u) * K + k] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float s1[W], s2[W];
        score_chunk<W>(h[u], c[u], mode, s1, s2);
#pragma unroll
        for (int k = 0; k < KC; ++k)
#pragma unroll
          for (int w = 0; w < W; ++w) acc[k][w] = fmaf(gk[u][k], second ? s2[w] : s1[w], acc[k][w]);
      }
    };
    int64_t r = r0;
    for (; r + R <= r1; r += R) add_rows(r, IC<R>());
    for (; r < r1; ++r) add_rows(r, IC<1>());
    float* dst = part_w + static_cast<int64_t>(blockIdx.x) * K * 2 * D + q * W;
#pragma unroll
    for (int k = 0; k < KC; ++k)
      if (KT > 0 || k < K)
#pragma unroll
        for (int w = 0; w < W; ++w) dst[static_cast<int64_t>(k) * 2 * D + w] = acc[k][w];
  }
  if (blockIdx.y == 0 && threadIdx.x < K) {
    float accb = 0.0f;
    for (int64_t r = r0; r < r1; ++r) accb += gl[r * K + threadIdx.x];
    part_b[static_cast<int64_t>(blockIdx.x) * K + threadIdx.x] = accb;
  }
}

int check_gate(const char* who, int64_t n, int D, int K, int mode) {
  if (n < 0 || D < 1) return set_error(kInvalid, "%s: bad shape n=%lld D=%d", who, static_cast<long long>(n), D);
  if (K < 1 || K > kMaxGateHops) return set_error(kInvalid, "%s: hop count %d outside [1, %d]", who, K, kMaxGateHops);
  if (mode != 0 && mode != 1) return set_error(kInvalid, "%s: score mode must be 0 (old) or 1 (new)", who);
  return kOk;
}

int gate_width(int D, std::initializer_list<const void*> ptrs) {
  if (D % 4 != 0) return 1;
  for (const void* p : ptrs)
    if (!aligned16(p)) return 1;
  return 4;
}

// Workspace layout of the backward: gl [n*K] | part_w [nb*K*2D] | part_b [nb*K].
int64_t gate_ws_floats(int64_t n, int D, int K) {
  const int64_t nb = colsum_blocks(n);
  return n * K + nb * K * 2LL * D + nb * K;
}

}  // namespace gate
}  // namespace cign

using namespace cign;
using namespace cign::rowops;
using namespace cign::gate;

extern "C" {

int64_t cign_hop_gate_bwd_workspace_bytes(int64_t n, int32_t D, int32_t K) {
  return 4LL * gate_ws_floats(n, D, K);
}

int cign_hop_gate_fwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t score_mode, const float* H,
                      const float* C, const float* weight, const float* bias, float* alpha) {
  int rc = check_gate("cign_hop_gate_fwd", n, D, K, score_mode);
  if (rc) return rc;
  if (n == 0) return kOk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int W = gate_width(D, {H, C, weight});
  rc = with_geo(D / W, [&](auto LC, auto VC) {
    constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
    const int grid = grid_for(n, Geo<L>::RPB);
    if (W == 4)
      with_hops(K, [&](auto KC) {
        hipLaunchKernelGGL((hop_gate_fwd_kernel<L, V, 4, decltype(KC)::value>), dim3(grid), dim3(kBlock), 0, st, n,
                           D, K, score_mode, H, C, weight, bias, alpha);
      });
    else
      hipLaunchKernelGGL((hop_gate_fwd_kernel<L, V, 1, 0>), dim3(grid), dim3(kBlock), 0, st, n, D, K, score_mode, H,
                         C, weight, bias, alpha);
    return check_launch("cign_hop_gate_fwd");
  });
  if (rc < 0) return set_error(kInvalid, "cign_hop_gate_fwd: D=%d too wide (max %d)", D, 256 * W);
  return rc;
}

int cign_hop_gate_bwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t score_mode, const float* H,
                      const float* C, const float* weight, const float* alpha, const float* grad_alpha, float* grad_H,
                      float* grad_C, float* grad_weight, float* grad_bias, void* workspace, int64_t workspace_bytes) {
  int rc = check_gate("cign_hop_gate_bwd", n, D, K, score_mode);
  if (rc) return rc;
  if (workspace_bytes < 4LL * gate_ws_floats(n, D, K))
    return set_error(kInvalid, "cign_hop_gate_bwd: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n == 0) return zero_outputs(st, grad_weight, K * 2 * D, grad_bias, K, "cign_hop_gate_bwd");
  const int nb = colsum_blocks(n);
  float* gl = static_cast<float*>(workspace);
  float* part_w = gl + n * K;
  float* part_b = part_w + static_cast<int64_t>(nb) * K * 2 * D;
  const int W = gate_width(D, {H, C, weight, grad_H, grad_C});
  rc = with_geo(D / W, [&](auto LC, auto VC) {
    constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
    const int grid = grid_for(n, Geo<L>::RPB);
    if (W == 4)
      with_hops(K, [&](auto KC) {
        hipLaunchKernelGGL((hop_gate_bwd_rows_kernel<L, V, 4, decltype(KC)::value>), dim3(grid), dim3(kBlock), 0, st,
                           n, D, K, score_mode, H, C, weight, alpha, grad_alpha, gl, grad_H, grad_C);
      });
    else
      hipLaunchKernelGGL((hop_gate_bwd_rows_kernel<L, V, 1, 0>), dim3(grid), dim3(kBlock), 0, st, n, D, K,
                         score_mode, H, C, weight, alpha, grad_alpha, gl, grad_H, grad_C);
    return check_launch("cign_hop_gate_bwd (rows)");
  });
  if (rc < 0) return set_error(kInvalid, "cign_hop_gate_bwd: D=%d too wide (max %d)", D, 256 * W);
  if (rc) return rc;
  const int qs = 2 * D / W;
  const dim3 cgrid(nb, (qs + kBlock - 1) / kBlock);
  if (W == 4)
    with_hops(K, [&](auto KC) {
      hipLaunchKernelGGL((hop_gate_bwd_cols_kernel<4, decltype(KC)::value>), cgrid, dim3(kBlock), 0, st, n, D, K,
                         score_mode, H, C, gl, part_w, part_b, nb);
    });
  else
    hipLaunchKernelGGL((hop_gate_bwd_cols_kernel<1, 0>), cgrid, dim3(kBlock), 0, st, n, D, K, score_mode, H, C, gl,
                       part_w, part_b, nb);
  if ((rc = check_launch("cign_hop_gate_bwd (cols)"))) return rc;
  if ((rc = launch_colsum(st, part_w, nb, K * 2 * D, 1, grad_weight, nullptr, "cign_hop_gate_bwd"))) return rc;
  return launch_colsum(st, part_b, nb, K, 1, grad_bias, nullptr, "cign_hop_gate_bwd");
}

}  // extern "C"
