// Explicit instantiation of the feature-layout collapsed-GAT kernels for bf16.
#include "gat_fl.h"

CIGN_GAT_FL_INSTANTIATE(::cign::bf16)
