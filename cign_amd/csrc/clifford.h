// The H/C interaction of the Clifford packs, per element, with its partial
// derivatives (shared by the pack kernels and the gated pack kernels):
//   mode 0 (old)       D = SiLU(bhr),            W = bhr - brh
//   mode 1 (new)       D = SiLU((bhr + brh)/2),  W = (bhr - brh)/2
//   mode 2 (new, tanh) D = SiLU((bhr + brh)/2),  W = tanh((bhr - brh)/2)
// with bhr = H*T_C, brh = C*T_H.
#pragma once

#include "rowops.h"

namespace cign {
namespace packk {
using namespace rowops;

struct DW {
  float Dv, Wv, dD_bhr, dD_brh, dW_bhr, dW_brh;
};

__device__ __forceinline__ DW interact(float bhr, float brh, int mode) {
  DW r;
  if (mode == 0) {
    r.Dv = silu(bhr);
    r.Wv = bhr - brh;
    r.dD_bhr = silu_grad(bhr);
    r.dD_brh = 0.0f;
    r.dW_bhr = 1.0f;
    r.dW_brh = -1.0f;
  } else {
    const float sym = 0.5f * (bhr + brh);
    const float anti = 0.5f * (bhr - brh);
    r.Dv = silu(sym);
    const float ds = silu_grad(sym);
    float dw = 1.0f;
    if (mode == 2) {
      r.Wv = tanhf(anti);
      dw = 1.0f - r.Wv * r.Wv;
    } else {
      r.Wv = anti;
    }
    r.dD_bhr = 0.5f * ds;
    r.dD_brh = 0.5f * ds;
    r.dW_bhr = 0.5f * dw;
    r.dW_brh = -0.5f * dw;
  }
  return r;
}

}  // namespace packk
}  // namespace cign
