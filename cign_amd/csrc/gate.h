// Internal interface of gate.hip for the other translation units of the
// library (not part of the C-ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace cign {
namespace gate {

// Backward of the node hop gate (cign_hop_gate_bwd) given grad_alpha [n,K]:
// grad_H and grad_C are written, or added to when `accumulate`; grad_weight
// [K,2D] and grad_bias [K] are written. Workspace: cign_hop_gate_bwd_workspace_bytes.
// Workspace bytes of node_gate_bwd (cign_hop_gate_bwd_workspace_bytes).
int64_t node_gate_ws_bytes(int64_t n, int D, int K);

int node_gate_bwd(hipStream_t st, int64_t n, int D, int K, int score_mode, const float* H, const float* C,
                  const float* weight, const float* alpha, const float* grad_alpha, float* grad_H, float* grad_C,
                  float* grad_weight, float* grad_bias, void* workspace, int64_t workspace_bytes, bool accumulate,
                  const char* who);

}  // namespace gate
}  // namespace cign
