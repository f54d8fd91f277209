// Decode matrix-vector kernels for Q5_K weights (matvec.h).
#include "matvec.h"

TINYOAI_MATVEC_DEFINE(FMT_Q5_K)
