// The 256x128 ping-pong variant's kernels (kLarge128: bf16/f16 operands, with
// and without reductions).  One variant per translation unit so that the
// library's kernels compile in parallel.
#include "gemm_epilogue_kernel.h"

FUSEML_GEMM_INSTANTIATE(fuseml_gemm::kLarge128)
