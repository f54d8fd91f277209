// Decode matrix-vector kernels for BF16 weights (matvec.h).
#include "matvec.h"

TINYOAI_MATVEC_DEFINE(FMT_BF16)
TINYOAI_MATVEC_DEFINE_FUSED(FMT_BF16)
