// Fixed-chain kernels of the deep3 tile variant (bf16 operands), part 2: the
// chains with an LDS-staged 2-D operand (bias + residual, and the
// bias, ReLU, gate product, sigmoid, row-add chain).
#include "gemm_epilogue_kernel.h"

FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, false, fuseml_gemm::kChainBiasTile)
FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, false, fuseml_gemm::kChainActHeavy)
