// GEMV kernel instances for epilogue 2 (one file per epilogue so they compile in parallel).
#include "gemv.h"

HI_GEMV_DEFINE_RUN(2)
