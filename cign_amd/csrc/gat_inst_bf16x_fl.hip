// Explicit instantiation of the narrow-row feature-layout collapsed-GAT kernels
// (one chunk per lane) for bf16 features with fp32 outputs and gradients.
#include "gat_fl.h"

CIGN_GAT_FL_INSTANTIATE(::cign::bf16x)
