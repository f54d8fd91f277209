// Decode matrix-vector kernels for F16 weights (matvec.h).
#include "matvec.h"

TINYOAI_MATVEC_DEFINE(FMT_F16)
