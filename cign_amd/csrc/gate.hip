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
#include "clifford.h"
#include "gate.h"

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

// Row part of the backward: gl (to the workspace), grad_H, grad_C (added to
// what they hold when ACC).
template <int LPR, int V, int W, int KT, bool ACC>
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
        if constexpr (ACC) {
          float ph[W], pc[W];
          Chunk<float, W>::load(gH + r * D + q * W, ph);
          Chunk<float, W>::load(gC + r * D + q * W, pc);
#pragma unroll
          for (int w = 0; w < W; ++w) {
            oh[w] = ph[w] + oh[w];
            oc[w] = pc[w] + oc[w];
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

// ===========================================================================
// The node-mode gate fused into the Clifford pack (the block's only use of
// alpha is the pack, model_cign.py:803-846): the forward computes a row's
// alpha from the H/C chunks it loads for the pack and applies it in the same
// pass; the backward finishes the pack's grad_alpha row sums and turns them
// into the gate's grad_H / grad_C terms, added to the pack's before the one
// store, and its gl (for the parameter gradients).
// ===========================================================================
struct PackGateArgs {
  int64_t n;
  int D, K, interaction, weighting, mode;
  const float* H;
  const float* C;
  const float* P[kMaxGateHops];
  int64_t p_stride;
  const float* wt;    // gate weight [K, 2D]
  const float* bias;  // gate bias [K] (forward)
  float* alpha;       // [n, K]: written by the forward, read by the backward
  float* out;
  const float* grad_out;
  float* gH;
  float* gC;
  float* gP[kMaxGateHops];
  int64_t gp_stride;
  float* gl;  // [n, K] softmax-backward of the gate, for the parameter gradients
};

template <int LPR, int V, int W>
__device__ __forceinline__ void load_hc(const PackGateArgs& a, const Geo<LPR>& g, int64_t r, float (&h)[V][W],
                                        float (&c)[V][W]) {
  const int qd = a.D / W;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    const int q = g.q + v * LPR;
#pragma unroll
    for (int w = 0; w < W; ++w) h[v][w] = c[v][w] = 0.0f;
    if (q < qd) {
      Chunk<float, W>::load(a.H + r * a.D + q * W, h[v]);
      Chunk<float, W>::load(a.C + r * a.D + q * W, c[v]);
    }
  }
}

template <int LPR, int V, int W, int KT>
__global__ __launch_bounds__(kBlock) void pack_gate_fwd_kernel(PackGateArgs a) {
  constexpr int KC = gate_kc<KT>();
  const Geo<LPR> g;
  const int D = a.D, K = a.K, qd = D / W;
  const GateW<LPR, V, W, KT> gw(a.wt, D, g.q);
  const int64_t out_w = a.weighting == 0 ? 2LL * K * D : 2LL * D;
  const int64_t step = static_cast<int64_t>(gridDim.x) * Geo<LPR>::RPB;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * Geo<LPR>::RPB + g.rl; r < a.n; r += step) {
    float h[V][W], c[V][W];
    load_hc<LPR, V, W>(a, g, r, h, c);
    // alpha: softmax over k of <score, weight[k]> + bias[k]
    float al[KC];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      al[k] = 0.0f;
      if (KT > 0 || k < K) {
        float d = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int q = g.q + v * LPR;
          if (KT > 0 || q < qd) {
            float s1[W], s2[W], wa[W], wb[W];
            score_chunk<W>(h[v], c[v], a.mode, s1, s2);
            gw.get(k, v, wa, wb);
#pragma unroll
            for (int w = 0; w < W; ++w) d = fmaf(s1[w], wa[w], fmaf(s2[w], wb[w], d));
          }
        }
        al[k] = row_sum<LPR>(d) + a.bias[k];
        m = fmaxf(m, al[k]);
      }
    }
    float tot = 0.0f;
#pragma unroll
    for (int k = 0; k < KC; ++k)
      if (KT > 0 || k < K) {
        al[k] = expf(al[k] - m);
        tot += al[k];
      }
    const float itot = 1.0f / tot;
#pragma unroll
    for (int k = 0; k < KC; ++k)
      if (KT > 0 || k < K) {
        al[k] = al[k] * itot;
        if (g.q == (k % LPR)) a.alpha[r * K + k] = al[k];
      }
    // the pack with this row's alpha
    float dag[V][W], wag[V][W];
#pragma unroll
    for (int v = 0; v < V; ++v)
#pragma unroll
      for (int w = 0; w < W; ++w) dag[v][w] = wag[v][w] = 0.0f;
    float* orow = a.out + r * out_w;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      if (KT > 0 || k < K) {
        const float* pk = a.P[k] + r * a.p_stride;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int q = g.q + v * LPR;
          if (q < qd) {
            float th[W], tc[W], ow[W], od[W];
            Chunk<float, W>::load(pk + q * W, th);
            Chunk<float, W>::load(pk + D + q * W, tc);
#pragma unroll
            for (int w = 0; w < W; ++w) {
              const packk::DW e = packk::interact(h[v][w] * tc[w], c[v][w] * th[w], a.interaction);
              ow[w] = al[k] * e.Wv;
              od[w] = al[k] * e.Dv;
              dag[v][w] += od[w];
              wag[v][w] += ow[w];
            }
            if (a.weighting == 0) {
              Chunk<float, W>::store(orow + 2LL * k * D + q * W, ow);
              Chunk<float, W>::store(orow + 2LL * k * D + D + q * W, od);
            }
          }
        }
      }
    }
    if (a.weighting == 1)
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const int q = g.q + v * LPR;
        if (q < qd) {
          Chunk<float, W>::store(orow + q * W, dag[v]);
          Chunk<float, W>::store(orow + D + q * W, wag[v]);
        }
      }
  }
}

template <int LPR, int V, int W, int KT>
__global__ __launch_bounds__(kBlock) void pack_gate_bwd_kernel(PackGateArgs a) {
  constexpr int KC = gate_kc<KT>();
  const Geo<LPR> g;
  const int D = a.D, K = a.K, qd = D / W;
  const GateW<LPR, V, W, KT> gw(a.wt, D, g.q);
  const int64_t out_w = a.weighting == 0 ? 2LL * K * D : 2LL * D;
  const int64_t step = static_cast<int64_t>(gridDim.x) * Geo<LPR>::RPB;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * Geo<LPR>::RPB + g.rl; r < a.n; r += step) {
    float h[V][W], c[V][W], gh[V][W], gc[V][W], goD1[V][W], goW1[V][W];
    const float* grow = a.grad_out + r * out_w;
    load_hc<LPR, V, W>(a, g, r, h, c);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int q = g.q + v * LPR;
#pragma unroll
      for (int w = 0; w < W; ++w) gh[v][w] = gc[v][w] = goD1[v][w] = goW1[v][w] = 0.0f;
      if (a.weighting == 1 && q < qd) {
        Chunk<float, W>::load(grow + q * W, goD1[v]);
        Chunk<float, W>::load(grow + D + q * W, goW1[v]);
      }
    }
    // the pack's backward; ga[k] = grad_alpha[r, k] on every lane of the row
    float al[KC], ga[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      al[k] = ga[k] = 0.0f;
      if (KT > 0 || k < K) {
        al[k] = a.alpha[r * K + k];
        const float* pk = a.P[k] + r * a.p_stride;
        float* gpk = a.gP[k] + r * a.gp_stride;
        float gsum = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const int q = g.q + v * LPR;
          if (q < qd) {
            const int d0 = q * W;
            float th[W], tc[W], goW[W], goD[W], gpt[W], gpc[W];
            Chunk<float, W>::load(pk + d0, th);
            Chunk<float, W>::load(pk + D + d0, tc);
            if (a.weighting == 0) {
              Chunk<float, W>::load(grow + 2LL * k * D + d0, goW);
              Chunk<float, W>::load(grow + 2LL * k * D + D + d0, goD);
            } else {
#pragma unroll
              for (int w = 0; w < W; ++w) {
                goW[w] = goW1[v][w];
                goD[w] = goD1[v][w];
              }
            }
#pragma unroll
            for (int w = 0; w < W; ++w) {
              const packk::DW e = packk::interact(h[v][w] * tc[w], c[v][w] * th[w], a.interaction);
              const float gD = goD[w] * al[k];
              const float gW = goW[w] * al[k];
              const float gbhr = gD * e.dD_bhr + gW * e.dW_bhr;
              const float gbrh = gD * e.dD_brh + gW * e.dW_brh;
              gh[v][w] += gbhr * tc[w];
              gc[v][w] += gbrh * th[w];
              gpt[w] = gbrh * c[v][w];
              gpc[w] = gbhr * h[v][w];
              gsum += goW[w] * e.Wv + goD[w] * e.Dv;
            }
            Chunk<float, W>::store(gpk + d0, gpt);
            Chunk<float, W>::store(gpk + D + d0, gpc);
          }
        }
        ga[k] = row_sum<LPR>(gsum);
      }
    }
    // the gate's backward: gl = alpha (ga - <alpha, ga>), gs = sum_k gl weight[k]
    float dot = 0.0f;
#pragma unroll
    for (int k = 0; k < KC; ++k) dot += al[k] * ga[k];
    float gl[KC];
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      gl[k] = al[k] * (ga[k] - dot);
      if ((KT > 0 || k < K) && g.q == (k % LPR)) a.gl[r * K + k] = gl[k];
    }
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
            float wa[W], wb[W];
            gw.get(k, v, wa, wb);
#pragma unroll
            for (int w = 0; w < W; ++w) {
              g1[w] = fmaf(gl[k], wa[w], g1[w]);
              g2[w] = fmaf(gl[k], wb[w], g2[w]);
            }
          }
        }
#pragma unroll
        for (int w = 0; w < W; ++w) {
          if (a.mode == 0) {
            gh[v][w] += g1[w];
            gc[v][w] += g2[w];
          } else {
            const float d = h[v][w] - c[v][w];
            const float sg = d > 0.0f ? 1.0f : (d < 0.0f ? -1.0f : 0.0f);
            gh[v][w] += g1[w] + sg * g2[w];
            gc[v][w] += g1[w] - sg * g2[w];
          }
        }
        Chunk<float, W>::store(a.gH + r * D + q * W, gh[v]);
        Chunk<float, W>::store(a.gC + r * D + q * W, gc[v]);
      }
    }
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

// grad_weight / grad_bias from gl (the workspace's first n*K floats, written
// by a rows kernel): row-block partials, then deterministic column sums.
int gate_param_grads(hipStream_t st, int64_t n, int D, int K, int mode, int W, const float* H, const float* C,
                     void* workspace, float* grad_weight, float* grad_bias, const char* who) {
  const int nb = colsum_blocks(n);
  const float* gl = static_cast<const float*>(workspace);
  float* part_w = static_cast<float*>(workspace) + n * K;
  float* part_b = part_w + static_cast<int64_t>(nb) * K * 2 * D;
  const int qs = 2 * D / W;
  const dim3 cgrid(nb, (qs + kBlock - 1) / kBlock);
  if (W == 4)
    with_hops(K, [&](auto KC) {
      hipLaunchKernelGGL((hop_gate_bwd_cols_kernel<4, decltype(KC)::value>), cgrid, dim3(kBlock), 0, st, n, D, K,
                         mode, H, C, gl, part_w, part_b, nb);
    });
  else
    hipLaunchKernelGGL((hop_gate_bwd_cols_kernel<1, 0>), cgrid, dim3(kBlock), 0, st, n, D, K, mode, H, C, gl,
                       part_w, part_b, nb);
  int rc = check_launch(who);
  if (rc) return rc;
  if ((rc = launch_colsum(st, part_w, nb, K * 2 * D, 1, grad_weight, nullptr, who))) return rc;
  return launch_colsum(st, part_b, nb, K, 1, grad_bias, nullptr, who);
}

}  // namespace gate

int64_t gate::node_gate_ws_bytes(int64_t n, int D, int K) { return 4LL * gate_ws_floats(n, D, K); }

// Backward of the node hop gate given grad_alpha (gate.h).
int gate::node_gate_bwd(hipStream_t st, int64_t n, int D, int K, int score_mode, const float* H, const float* C,
                        const float* weight, const float* alpha, const float* grad_alpha, float* grad_H,
                        float* grad_C, float* grad_weight, float* grad_bias, void* workspace,
                        int64_t workspace_bytes, bool accumulate, const char* who) {
  int rc = check_gate(who, n, D, K, score_mode);
  if (rc) return rc;
  if (workspace_bytes < 4LL * gate_ws_floats(n, D, K)) return set_error(kInvalid, "%s: workspace too small", who);
  if (n == 0) return zero_outputs(st, grad_weight, K * 2 * D, grad_bias, K, who);
  float* gl = static_cast<float*>(workspace);
  const int W = gate_width(D, {H, C, weight, grad_H, grad_C});
  rc = with_geo(D / W, [&](auto LC, auto VC) {
    constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
    const int grid = grid_for(n, Geo<L>::RPB);
    auto go = [&](auto AC) {
      constexpr bool A = decltype(AC)::value;
      if (W == 4)
        with_hops(K, [&](auto KC) {
          hipLaunchKernelGGL((hop_gate_bwd_rows_kernel<L, V, 4, decltype(KC)::value, A>), dim3(grid), dim3(kBlock), 0,
                             st, n, D, K, score_mode, H, C, weight, alpha, grad_alpha, gl, grad_H, grad_C);
        });
      else
        hipLaunchKernelGGL((hop_gate_bwd_rows_kernel<L, V, 1, 0, A>), dim3(grid), dim3(kBlock), 0, st, n, D, K,
                           score_mode, H, C, weight, alpha, grad_alpha, gl, grad_H, grad_C);
    };
    if (accumulate) go(std::true_type());
    else go(std::false_type());
    return check_launch(who);
  });
  if (rc < 0) return set_error(kInvalid, "%s: D=%d too wide (max %d)", who, D, 256 * W);
  if (rc) return rc;
  return gate_param_grads(st, n, D, K, score_mode, W, H, C, workspace, grad_weight, grad_bias, who);
}

namespace gate {

int check_pack_gate(const char* who, int64_t n, int D, int K, int interaction, int weighting, int mode) {
  int rc = check_gate(who, n, D, K, mode);
  if (rc) return rc;
  if (interaction < 0 || interaction > 2) return set_error(kInvalid, "%s: interaction_mode must be 0, 1 or 2", who);
  if (weighting < 0 || weighting > 1) return set_error(kInvalid, "%s: weighting_mode must be 0(old) or 1(new)", who);
  return kOk;
}

// 4-float chunks when D, the hop stride(s) and every pointer allow 16-byte access.
int pack_gate_width(const PackGateArgs& a, bool bwd) {
  if (a.D % 4 != 0 || a.p_stride % 4 != 0 || (bwd && a.gp_stride % 4 != 0)) return 1;
  const void* ptrs[] = {a.H, a.C, a.wt, bwd ? static_cast<const void*>(a.grad_out) : static_cast<const void*>(a.out),
                        bwd ? static_cast<const void*>(a.gH) : a.H, bwd ? static_cast<const void*>(a.gC) : a.C};
  for (const void* p : ptrs)
    if (!aligned16(p)) return 1;
  for (int k = 0; k < a.K; ++k)
    if (!aligned16(a.P[k]) || (bwd && !aligned16(a.gP[k]))) return 1;
  return 4;
}

template <bool BWD>
int launch_pack_gate(hipStream_t st, const PackGateArgs& a, const char* who) {
  const int W = pack_gate_width(a, BWD);
  const int rc = with_geo(a.D / W, [&](auto LC, auto VC) {
    constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
    const int grid = grid_for(a.n, Geo<L>::RPB);
    if (W == 4)
      with_hops(a.K, [&](auto KC) {
        constexpr int KT = decltype(KC)::value;
        if constexpr (BWD)
          hipLaunchKernelGGL((pack_gate_bwd_kernel<L, V, 4, KT>), dim3(grid), dim3(kBlock), 0, st, a);
        else
          hipLaunchKernelGGL((pack_gate_fwd_kernel<L, V, 4, KT>), dim3(grid), dim3(kBlock), 0, st, a);
      });
    else if constexpr (BWD)
      hipLaunchKernelGGL((pack_gate_bwd_kernel<L, V, 1, 0>), dim3(grid), dim3(kBlock), 0, st, a);
    else
      hipLaunchKernelGGL((pack_gate_fwd_kernel<L, V, 1, 0>), dim3(grid), dim3(kBlock), 0, st, a);
    return check_launch(who);
  });
  if (rc < 0) return set_error(kInvalid, "%s: D=%d too wide (max %d)", who, a.D, 256 * W);
  return rc;
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
  return cign::gate::node_gate_bwd(static_cast<hipStream_t>(stream), n, D, K, score_mode, H, C, weight, alpha,
                                   grad_alpha, grad_H, grad_C, grad_weight, grad_bias, workspace, workspace_bytes,
                                   false, "cign_hop_gate_bwd");
}

int cign_pack_gate_fwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t weighting,
                       int32_t score_mode, const float* H, const float* C, const float* const* props,
                       int64_t prop_stride, const float* gate_weight, const float* gate_bias, float* alpha,
                       float* out) {
  int rc = check_pack_gate("cign_pack_gate_fwd", n, D, K, interaction, weighting, score_mode);
  if (rc) return rc;
  if (!props) return set_error(kInvalid, "cign_pack_gate_fwd: null hop pointer array");
  if (n == 0) return kOk;
  PackGateArgs a = {};
  a.n = n; a.D = D; a.K = K; a.interaction = interaction; a.weighting = weighting; a.mode = score_mode;
  a.H = H; a.C = C; a.p_stride = prop_stride; a.wt = gate_weight; a.bias = gate_bias; a.alpha = alpha; a.out = out;
  for (int k = 0; k < K; ++k) a.P[k] = props[k];
  return launch_pack_gate<false>(static_cast<hipStream_t>(stream), a, "cign_pack_gate_fwd");
}

int cign_pack_gate_bwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t weighting,
                       int32_t score_mode, const float* grad_out, const float* H, const float* C,
                       const float* const* props, int64_t prop_stride, const float* alpha, const float* gate_weight,
                       float* grad_H, float* grad_C, float* const* grad_props, int64_t grad_prop_stride,
                       float* grad_gate_weight, float* grad_gate_bias, void* workspace, int64_t workspace_bytes) {
  int rc = check_pack_gate("cign_pack_gate_bwd", n, D, K, interaction, weighting, score_mode);
  if (rc) return rc;
  if (!props || !grad_props) return set_error(kInvalid, "cign_pack_gate_bwd: null hop pointer array");
  if (workspace_bytes < 4LL * gate_ws_floats(n, D, K))
    return set_error(kInvalid, "cign_pack_gate_bwd: workspace too small");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n == 0) return zero_outputs(st, grad_gate_weight, K * 2 * D, grad_gate_bias, K, "cign_pack_gate_bwd");
  PackGateArgs a = {};
  a.n = n; a.D = D; a.K = K; a.interaction = interaction; a.weighting = weighting; a.mode = score_mode;
  a.H = H; a.C = C; a.p_stride = prop_stride; a.wt = gate_weight; a.alpha = const_cast<float*>(alpha);
  a.grad_out = grad_out; a.gH = grad_H; a.gC = grad_C; a.gp_stride = grad_prop_stride;
  a.gl = static_cast<float*>(workspace);
  for (int k = 0; k < K; ++k) {
    a.P[k] = props[k];
    a.gP[k] = grad_props[k];
  }
  if ((rc = launch_pack_gate<true>(st, a, "cign_pack_gate_bwd"))) return rc;
  const int W = gate_width(D, {H, C});
  return gate_param_grads(st, n, D, K, score_mode, W, H, C, workspace, grad_gate_weight, grad_gate_bias,
                          "cign_pack_gate_bwd");
}

}  // extern "C"
