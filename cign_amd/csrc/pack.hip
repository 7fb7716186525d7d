// Fused Clifford blade packing: the H/C interaction with the K propagated
// hops and the alpha weighting, forward and backward, and its C-ABI.
//
// For hop k, T_H = P_k[:, :D], T_C = P_k[:, D:], bhr = H*T_C, brh = C*T_H:
//   interaction 0 (old)       D = SiLU(bhr),            W = bhr - brh
//   interaction 1 (new)       D = SiLU((bhr + brh)/2),  W = (bhr - brh)/2
//   interaction 2 (new, tanh) D = SiLU((bhr + brh)/2),  W = tanh((bhr - brh)/2)
//   weighting 0 (old)  out [N, K*2D]: out[n, k*2D + d] = a_k W, out[n, k*2D + D + d] = a_k D
//   weighting 1 (new)  out [N, 2D]  : [sum_k a_k D | sum_k a_k W]   (D first)
// References: fused_clifford_pack_ext/fused_clifford_pack_cuda.cu:22-219 (old,
// K=3), fused_clifford_pack.py:88-139 (old, generic K), generic_engine/
// fused_clifford_cign_pack_ext/fused_clifford_switch_pack_cuda.cu:22-521
// (switch pack), generic_engine/fused_clifford_switch_pack_ext/...:48,51
// (tanh), generic_engine/fused_clifford_cign_generic.py:58-109 (new, generic K).
//
// The propagated tensors are addressed through K row pointers with a common
// row stride, which covers both K separate [N,2D] tensors (stride 2D) and one
// stacked [N,K,2D] tensor (pointer k = base + k*2D, stride 2KD).
// Forward: one thread per (node, 16-byte chunk of D), all K hops in registers.
// Backward: a row's chunks on one lane group (rowops.h) so grad_alpha is a
// butterfly; grad_H / grad_C accumulate over hops in registers (no atomics).
#include "clifford.h"

namespace cign {
namespace packk {
using namespace rowops;

constexpr int kMaxHops = 16;

struct PackArgs {
  int64_t n;
  int D, K, interaction, weighting;
  const float* H;
  const float* C;
  const float* alpha;  // [n, K]
  const float* P[kMaxHops];
  int64_t p_stride;
  // forward
  float* out;
  // backward
  const float* grad_out;
  float* gH;
  float* gC;
  float* gP[kMaxHops];
  int64_t gp_stride;
  float* gA;
};

template <int W>
__global__ __launch_bounds__(kBlock) void pack_fwd_kernel(PackArgs a) {
  const int D = a.D, K = a.K;
  const int qd = D / W;
  const int64_t total = a.n * qd;
  const int64_t out_w = a.weighting == 0 ? 2LL * K * D : 2LL * D;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t r = i / qd;
    const int d0 = static_cast<int>(i - r * qd) * W;
    float h[W], c[W], dag[W], wag[W];
    Chunk<float, W>::load(a.H + r * D + d0, h);
    Chunk<float, W>::load(a.C + r * D + d0, c);
#pragma unroll
    for (int w = 0; w < W; ++w) dag[w] = wag[w] = 0.0f;
    float* orow = a.out + r * out_w;
    for (int k = 0; k < K; ++k) {
      const float* pk = a.P[k] + r * a.p_stride;
      float th[W], tc[W], ow[W], od[W];
      Chunk<float, W>::load(pk + d0, th);
      Chunk<float, W>::load(pk + D + d0, tc);
      const float ak = a.alpha[r * K + k];
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const DW v = interact(h[w] * tc[w], c[w] * th[w], a.interaction);
        ow[w] = ak * v.Wv;
        od[w] = ak * v.Dv;
        dag[w] += od[w];
        wag[w] += ow[w];
      }
      if (a.weighting == 0) {
        Chunk<float, W>::store(orow + 2LL * k * D + d0, ow);
        Chunk<float, W>::store(orow + 2LL * k * D + D + d0, od);
      }
    }
    if (a.weighting == 1) {
      Chunk<float, W>::store(orow + d0, dag);
      Chunk<float, W>::store(orow + D + d0, wag);
    }
  }
}

template <int LPR, int V, int W>
__global__ __launch_bounds__(kBlock) void pack_bwd_kernel(PackArgs a) {
  const Geo<LPR> g;
  const int D = a.D, K = a.K;
  const int qd = D / W;
  const int64_t out_w = a.weighting == 0 ? 2LL * K * D : 2LL * D;
  const int64_t step = static_cast<int64_t>(gridDim.x) * Geo<LPR>::RPB;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * Geo<LPR>::RPB + g.rl; r < a.n; r += step) {
    float h[V][W], c[V][W], gh[V][W], gc[V][W], goD1[V][W], goW1[V][W];
    const float* grow = a.grad_out + r * out_w;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int q = g.q + v * LPR;
#pragma unroll
      for (int w = 0; w < W; ++w) h[v][w] = c[v][w] = gh[v][w] = gc[v][w] = goD1[v][w] = goW1[v][w] = 0.0f;
      if (q < qd) {
        Chunk<float, W>::load(a.H + r * D + q * W, h[v]);
        Chunk<float, W>::load(a.C + r * D + q * W, c[v]);
        if (a.weighting == 1) {
          Chunk<float, W>::load(grow + q * W, goD1[v]);
          Chunk<float, W>::load(grow + D + q * W, goW1[v]);
        }
      }
    }
    for (int k = 0; k < K; ++k) {
      const float ak = a.alpha[r * K + k];
      const float* pk = a.P[k] + r * a.p_stride;
      float* gpk = a.gP[k] + r * a.gp_stride;
      float ga = 0.0f;
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
            const DW s = interact(h[v][w] * tc[w], c[v][w] * th[w], a.interaction);
            const float gD = goD[w] * ak;
            const float gW = goW[w] * ak;
            const float gbhr = gD * s.dD_bhr + gW * s.dW_bhr;
            const float gbrh = gD * s.dD_brh + gW * s.dW_brh;
            gh[v][w] += gbhr * tc[w];
            gc[v][w] += gbrh * th[w];
            gpt[w] = gbrh * c[v][w];
            gpc[w] = gbhr * h[v][w];
            ga += goW[w] * s.Wv + goD[w] * s.Dv;
          }
          Chunk<float, W>::store(gpk + d0, gpt);
          Chunk<float, W>::store(gpk + D + d0, gpc);
        }
      }
      ga = row_sum<LPR>(ga);
      if (g.q == 0) a.gA[r * K + k] = ga;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int q = g.q + v * LPR;
      if (q < qd) {
        Chunk<float, W>::store(a.gH + r * D + q * W, gh[v]);
        Chunk<float, W>::store(a.gC + r * D + q * W, gc[v]);
      }
    }
  }
}

int check_pack(const char* who, int64_t n, int D, int K, int interaction, int weighting) {
  if (n < 0 || D < 1) return set_error(kInvalid, "%s: bad shape n=%lld D=%d", who, static_cast<long long>(n), D);
  if (K < 1 || K > kMaxHops) return set_error(kInvalid, "%s: hop count %d outside [1, %d]", who, K, kMaxHops);
  if (interaction < 0 || interaction > 2) return set_error(kInvalid, "%s: interaction_mode must be 0, 1 or 2", who);
  if (weighting < 0 || weighting > 1) return set_error(kInvalid, "%s: weighting_mode must be 0(old) or 1(new)", who);
  return kOk;
}

// 4-float chunks when D and every row pointer / stride allow 16-byte access.
int pack_width(const PackArgs& a, bool bwd) {
  if (a.D % 4 != 0 || a.p_stride % 4 != 0) return 1;
  const void* ptrs[] = {a.H, a.C, bwd ? static_cast<const void*>(a.grad_out) : static_cast<const void*>(a.out),
                        bwd ? static_cast<const void*>(a.gH) : a.H, bwd ? static_cast<const void*>(a.gC) : a.C};
  for (const void* p : ptrs)
    if (!aligned16(p)) return 1;
  for (int k = 0; k < a.K; ++k) {
    if (!aligned16(a.P[k])) return 1;
    if (bwd && (!aligned16(a.gP[k]) || a.gp_stride % 4 != 0)) return 1;
  }
  return 4;
}

}  // namespace packk
}  // namespace cign

using namespace cign;
using namespace cign::rowops;
using namespace cign::packk;

extern "C" {

int cign_pack_fwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t weighting,
                  const float* H, const float* C, const float* const* props, int64_t prop_stride, const float* alpha,
                  float* out) {
  int rc = check_pack("cign_pack_fwd", n, D, K, interaction, weighting);
  if (rc) return rc;
  if (!props) return set_error(kInvalid, "cign_pack_fwd: null hop pointer array");
  if (n == 0) return kOk;
  PackArgs a = {};
  a.n = n; a.D = D; a.K = K; a.interaction = interaction; a.weighting = weighting;
  a.H = H; a.C = C; a.alpha = alpha; a.p_stride = prop_stride; a.out = out;
  for (int k = 0; k < K; ++k) a.P[k] = props[k];
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int W = pack_width(a, false);
  const int grid = grid_for(n * (D / W), kBlock);
  if (W == 4)
    hipLaunchKernelGGL((pack_fwd_kernel<4>), dim3(grid), dim3(kBlock), 0, st, a);
  else
    hipLaunchKernelGGL((pack_fwd_kernel<1>), dim3(grid), dim3(kBlock), 0, st, a);
  return check_launch("cign_pack_fwd");
}

int cign_pack_bwd(void* stream, int64_t n, int32_t D, int32_t K, int32_t interaction, int32_t weighting,
                  const float* grad_out, const float* H, const float* C, const float* const* props,
                  int64_t prop_stride, const float* alpha, float* grad_H, float* grad_C, float* const* grad_props,
                  int64_t grad_prop_stride, float* grad_alpha) {
  int rc = check_pack("cign_pack_bwd", n, D, K, interaction, weighting);
  if (rc) return rc;
  if (!props || !grad_props) return set_error(kInvalid, "cign_pack_bwd: null hop pointer array");
  if (n == 0) return kOk;
  PackArgs a = {};
  a.n = n; a.D = D; a.K = K; a.interaction = interaction; a.weighting = weighting;
  a.H = H; a.C = C; a.alpha = alpha; a.p_stride = prop_stride; a.grad_out = grad_out;
  a.gH = grad_H; a.gC = grad_C; a.gA = grad_alpha; a.gp_stride = grad_prop_stride;
  for (int k = 0; k < K; ++k) {
    a.P[k] = props[k];
    a.gP[k] = grad_props[k];
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int W = pack_width(a, true);
  rc = with_geo(D / W, [&](auto LC, auto VC) {
    constexpr int L = decltype(LC)::value, V = decltype(VC)::value;
    const int grid = grid_for(n, Geo<L>::RPB);
    if (W == 4)
      hipLaunchKernelGGL((pack_bwd_kernel<L, V, 4>), dim3(grid), dim3(kBlock), 0, st, a);
    else
      hipLaunchKernelGGL((pack_bwd_kernel<L, V, 1>), dim3(grid), dim3(kBlock), 0, st, a);
    return check_launch("cign_pack_bwd");
  });
  if (rc < 0) return set_error(kInvalid, "cign_pack_bwd: D=%d too wide (max %d)", D, 256 * W);
  return rc;
}

}  // extern "C"
