// Explicit instantiation of the collapsed-GAT kernels for float, 8 head lanes.
#include "gat_kernels.h"

CIGN_GAT_INSTANTIATE(float, 8)
