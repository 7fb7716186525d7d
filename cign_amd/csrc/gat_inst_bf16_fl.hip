// Explicit instantiation of the feature-layout collapsed-GAT forward for bf16.
#include "gat_kernels.h"

CIGN_GAT_FL_INSTANTIATE(::cign::bf16)
