// Explicit instantiation of the narrow feature-layout collapsed-GAT kernels
// for bf16 features taken four values per lane (small graphs).
#include "gat_fl.h"

CIGN_GAT_FL_INSTANTIATE(::cign::bf16h)
