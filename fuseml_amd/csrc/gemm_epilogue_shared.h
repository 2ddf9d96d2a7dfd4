// gemm_epilogue_shared.h — what the host side of the GEMM+epilogue kernels
// (gemm_epilogue.hip) and the kernel template (gemm_epilogue_kernel.h) both
// need: the host-derived operand flags, the tile variants, and the kernel's
// declaration.  The kernels are instantiated one variant per translation
// unit (gemm_epilogue_v_*.hip), so the library builds in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "fuseml_hip.h"

namespace fuseml_gemm {

// Host-derived flags kept in the `reserved` field of operands and outputs.
constexpr int kFlagVec4 = 1;   // unit stride along N, rows 4-element aligned: 8/16-byte vectors
constexpr int kFlagStage = 2;  // 16-bit, rows 8-element aligned, 16-byte base: LDS-staged tile
constexpr int kFlagAux = 4;    // row ([N]) or column ([M]) vector staged as fp32 in LDS slot (bits 8-9)
constexpr int kAuxSlots = 4;   // vector operands staged per launch

struct TileConfig {
  int bm, bn, bk, stages, wm, wn;
  int sched;  // K-loop schedule (kernel template parameter SCHED)
  constexpr int lds_bytes() const {
    return stages * (bm + bn) * bk * 2 + kAuxSlots * (bm > bn ? bm : bn) * 4;
  }
};

constexpr TileConfig kLarge = {256, 256, 32, 4, 2, 4, 1};  // 8 waves ping-pong, 132 KB LDS, 1 WG/CU
constexpr TileConfig kDeep = {256, 256, 64, 2, 2, 2, 3};   // 4 waves (1/SIMD), BK=64 x 2 stages, 132 KB LDS
constexpr TileConfig kSmall = {128, 128, 32, 4, 2, 2, 0};  // 4 waves lock-step, 66 KB LDS, 2 WG/CU
constexpr TileConfig kDeep3 = {256, 256, 64, 2, 2, 2, 6};  // as kDeep, whole-stage fragments; K % 64 == 0
constexpr TileConfig kNarrow64 = {64, 128, 64, 3, 2, 2, 0};  // 4 waves lock-step (wave tile 32x64), 74 KB LDS, 2 WG/CU
constexpr TileConfig kNarrow32 = {32, 128, 64, 3, 1, 4, 0};  // 4 waves lock-step (wave tile 32x32), 62 KB LDS, 2 WG/CU
constexpr TileConfig kLarge128 = {256, 128, 32, 4, 4, 2, 1};  // 8 waves ping-pong (wave tile 64x64), 100 KB LDS, 1 WG/CU
constexpr TileConfig kSmall64 = {128, 128, 64, 4, 2, 2, 0};  // kSmall at BK = 64: 130 KB LDS, 1 WG/CU

// Epilogue chains compiled into kernels of their own (template parameter CH
// of the kernel).  kChainGeneric runs the descriptor's op list through the
// runtime op loop; every other value is one fixed op sequence, matched on the
// host (operand kinds included) and compiled as straight-line code with no
// per-op dispatch.  "row" is a [N] vector operand in an LDS slot, "tile" the
// LDS-staged bf16 2-D operand; ADD keeps its alpha from the descriptor.
enum FixedChain : int {
  kChainGeneric = 0,
  kChainNone = 1,          // (no ops)
  kChainBias = 2,          // add(row)
  kChainBiasGeluErf = 3,   // add(row), gelu(approximate='none')
  kChainBiasGeluTanh = 4,  // add(row), gelu(approximate='tanh')
  kChainBiasRelu = 5,      // add(row), relu
  kChainBiasTile = 6,      // add(row), add(tile)           (bias + residual)
  kChainActHeavy = 7,      // add(row), relu, mul(tile), sigmoid, add(row)
  kChainRelu = 8,          // relu                          (also with reductions)
  kNumChains = 9,
};

// The kernel (defined in gemm_epilogue_kernel.h).  SCHED selects the K-loop
// schedule, T the GEMM operand type (__bf16 or _Float16), RED whether the
// launch has reductions, CH the epilogue chain (FixedChain).
template <int BM, int BN, int BK, int S, int WM, int WN, int SCHED, typename T, bool RED, int CH>
__global__ void gemm_epilogue_kernel(const fuseml_gemm_desc d_arg);

}  // namespace fuseml_gemm
