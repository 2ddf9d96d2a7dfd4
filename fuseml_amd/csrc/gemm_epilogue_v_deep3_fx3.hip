// Fixed-chain kernels of the deep3 tile variant (bf16 operands), part 3: the
// short chains (none, bias, bias + ReLU, ReLU) and ReLU followed by fused
// reductions.
#include "gemm_epilogue_kernel.h"

FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, false, fuseml_gemm::kChainNone)
FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, false, fuseml_gemm::kChainBias)
FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, false, fuseml_gemm::kChainBiasRelu)
FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, false, fuseml_gemm::kChainRelu)
FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, true, fuseml_gemm::kChainRelu)
