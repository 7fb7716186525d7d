// Explicit instantiation of the collapsed-GAT kernels for float, 4 head lanes.
#include "gat_kernels.h"

CIGN_GAT_INSTANTIATE(float, 4)
