// Decode matrix-vector kernels for Q4_K weights (matvec.h).
#include "matvec.h"

TINYOAI_MATVEC_DEFINE(FMT_Q4_K)
