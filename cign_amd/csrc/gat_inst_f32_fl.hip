// Explicit instantiation of the feature-layout collapsed-GAT kernels for float.
#include "gat_fl.h"

CIGN_GAT_FL_INSTANTIATE(float)
