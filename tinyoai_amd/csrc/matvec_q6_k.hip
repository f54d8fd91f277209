// Decode matrix-vector kernels for Q6_K weights (matvec.h).
#include "matvec.h"

TINYOAI_MATVEC_DEFINE(FMT_Q6_K)
