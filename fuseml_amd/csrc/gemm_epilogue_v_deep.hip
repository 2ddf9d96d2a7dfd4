// The deep tile variant's kernels (kDeep: bf16/f16 operands, with and without
// reductions).  One variant per translation unit so that the library's kernels
// compile in parallel.
#include "gemm_epilogue_kernel.h"

FUSEML_GEMM_INSTANTIATE(fuseml_gemm::kDeep)
