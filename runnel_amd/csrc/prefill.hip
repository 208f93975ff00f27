// Prefill kernels (expert-sorted grouped dequant-GEMM) live here.
#include "common.h"
#include "kernels.h"
