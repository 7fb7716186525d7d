// Explicit instantiation of the wide-row feature-layout collapsed-GAT kernels
// (several chunks per lane) for bf16 features with fp32 outputs and gradients.
#include "gat_fl.h"

CIGN_GAT_FLW_INSTANTIATE(::cign::bf16x)
