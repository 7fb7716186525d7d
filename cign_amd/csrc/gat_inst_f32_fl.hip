// Explicit instantiation of the feature-layout collapsed-GAT forward for float.
#include "gat_kernels.h"

CIGN_GAT_FL_INSTANTIATE(float)
