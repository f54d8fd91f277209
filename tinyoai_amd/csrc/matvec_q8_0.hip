// Decode matrix-vector kernels for Q8_0 weights (matvec.h).
#include "matvec.h"

TINYOAI_MATVEC_DEFINE(FMT_Q8_0)
TINYOAI_MATVEC_DEFINE_FUSED(FMT_Q8_0)
