// Fixed-chain kernels of the deep3 tile variant (bf16 operands), part 1: the
// chains of the activation GEMMs (bias + GELU, erf and tanh forms).  Fixed
// chains are split over several translation units so that they compile in
// parallel with the generic kernels.
#include "gemm_epilogue_kernel.h"

FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, false, fuseml_gemm::kChainBiasGeluErf)
FUSEML_GEMM_INSTANTIATE_ONE(fuseml_gemm::kDeep3, __bf16, false, fuseml_gemm::kChainBiasGeluTanh)
