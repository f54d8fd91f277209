// Decode matrix-vector kernels for F32 weights (matvec.h).
#include "matvec.h"

TINYOAI_MATVEC_DEFINE(FMT_F32)
