// Explicit instantiation of the collapsed-GAT kernels for bf16, 8 head lanes.
#include "gat_kernels.h"

CIGN_GAT_INSTANTIATE(::cign::bf16, 8)
