// GEMM kernel instances for epilogue 2 (one file per epilogue so they compile in parallel).
#include "gemm.h"

HI_GEMM_DEFINE_RUN(2)
