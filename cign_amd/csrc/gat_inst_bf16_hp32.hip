// Explicit instantiation of the collapsed-GAT kernels for bf16, 32 head lanes.
#include "gat_kernels.h"

CIGN_GAT_INSTANTIATE(::cign::bf16, 32)
