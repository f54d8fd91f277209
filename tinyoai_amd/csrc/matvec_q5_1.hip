// Decode matrix-vector kernels for Q5_1 weights (matvec.h).
#include "matvec.h"

TINYOAI_MATVEC_DEFINE(FMT_Q5_1)
