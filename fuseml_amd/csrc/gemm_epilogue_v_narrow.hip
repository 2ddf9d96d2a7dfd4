// The narrow tile variants' kernels (kNarrow64, kNarrow32: bf16/f16 operands,
// with and without reductions).  One translation unit per tile family so that
// the library's kernels compile in parallel.
#include "gemm_epilogue_kernel.h"

FUSEML_GEMM_INSTANTIATE(fuseml_gemm::kNarrow64)
FUSEML_GEMM_INSTANTIATE(fuseml_gemm::kNarrow32)
