// The 128x128 lock-step variants' kernels (kSmall, and kSmall64 at BK = 64:
// bf16/f16 operands, with and without reductions).  One variant per translation unit so that the library's kernels
// compile in parallel.
#include "gemm_epilogue_kernel.h"

FUSEML_GEMM_INSTANTIATE(fuseml_gemm::kSmall)
FUSEML_GEMM_INSTANTIATE(fuseml_gemm::kSmall64)
