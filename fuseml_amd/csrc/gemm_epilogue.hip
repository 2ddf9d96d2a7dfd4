// gemm_epilogue.hip — host side of the gfx950 fused GEMM+epilogue kernel
// family: validation, variant choice, launch, and the C ABI.  The kernel
// template is gemm_epilogue_kernel.h, instantiated one tile variant per
// translation unit (gemm_epilogue_v_*.hip).
//
// What one launch computes (one fusion group):
//   acc = A[M,K] @ B[K,N] in fp32 on bf16/f16 MFMA (v_mfma_f32_32x32x16_*),
//   v   = epilogue op chain applied to acc in registers,
//   out = cast(v) stored once, plus optional escape stores and fused row/column
//         sum/amax/mean reductions.
// This replaces the generated Triton kernel of the reference
// (fuseml/codegen/kernel_generator.py: K-loop 1454-1542, bias 881-901,
// epilogue emitters 1599-1903, store 1544-1593, reductions 1909-2018) and the
// cuBLASLt epilogue extension (fuseml/codegen/cublas_epilogue.py:355-557).
//
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "fuseml_hip.h"
#include "gemm_epilogue_shared.h"

using namespace fuseml_gemm;

namespace {

thread_local char g_last_error[512];

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

// Initialise reduction buffers: sum/mean to 0, amax to -inf.
__global__ void reduce_fill_kernel(float* sum, float* amax, float* mean, int len) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= len) return;
  if (sum) sum[i] = 0.0f;
  if (amax) amax[i] = -INFINITY;
  if (mean) mean[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// Host side: validation, variant table, launch
// ---------------------------------------------------------------------------

constexpr int64_t kMaxBytes = (int64_t)1 << 31;
constexpr int64_t kTileSpan = 256;  // largest tile edge of any variant

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Pinned variant: 0 automatic, else 1 + index into {large, deep, deep3, small,
// deep3-generic, narrow64, narrow32, large128, small64} (deep3-generic: deep3
// with the generic op loop even where a fixed chain matches).  Initialised once per process from FUSEML_HIP_TILE, changed
// only through fuseml_gemm_epilogue_force_variant.
constexpr const char* kVariantNames[] = {"large", "deep", "deep3", "small", "deep3-generic", "narrow64", "narrow32",
                                         "large128", "small64"};
constexpr int kNumVariantNames = 9;
constexpr int kForcedDeep3Generic = 5;
std::atomic<int> g_forced_variant{-1};  // -1: environment not read yet

int variant_code(const char* name) {
  if (name == nullptr || name[0] == '\0' || !strcmp(name, "auto")) return 0;
  for (int i = 0; i < kNumVariantNames; ++i)
    if (!strcmp(name, kVariantNames[i])) return i + 1;
  return -1;
}

int forced_variant() {
  int v = g_forced_variant.load(std::memory_order_relaxed);
  if (v < 0) {
    const int e = variant_code(getenv("FUSEML_HIP_TILE"));
    int expected = -1;
    g_forced_variant.compare_exchange_strong(expected, e < 0 ? 0 : e, std::memory_order_relaxed);
    v = g_forced_variant.load(std::memory_order_relaxed);
  }
  return v;
}

int match_fixed_chain(const fuseml_gemm_desc& d);

// Below one round of 256x256 tiles: the 128x128, 64x128 or 32x128 lock-step
// tile (4 waves, two workgroups per CU) or the 256x128 ping-pong tile (8
// waves, one per CU), whichever gives its busiest CU the least K-loop work:
// ceil(tiles / CUs) x (BM + BN) operand rows per unit of K, weighted by how
// fast a CU moves them: 5 for the lock-step tiles with two workgroups on some
// CU, 8 with at most one (one wave per SIMD hides less of the LDS DMA's
// latency and none of the epilogue; 7 for K > 2048), 6 for the ping-pong
// tile; the first of the list on a tie.  Also for M <= 128 at any N, where a
// 256-row tile is at least half padding.  Each CU moves its tiles' A and W
// rows through the LDS DMA at a roughly fixed rate (37-48 GB/s measured,
// whatever the tile), so below two 128x128 tiles per CU a narrower tile
// spreads the same K over more CUs or more waves.  Measured
// (bias + GELU or bias + residual, M x N x K, us): 128x1024x256 9.6 -> 5.9 and
// 1024x1024x1024 16.8 -> 9.9 on 32x128 tiles; 2048x1024x4096 44.7 -> 31.7,
// 2048x2048x1024 20.0 -> 17.7 and 8192x512x2048 31.5 -> 28.8 on 64x128 tiles;
// 2048x4096x1024 33.0 -> 29.0 and 4096x2048x1024 31.8 -> 29.5 on 256x128
// ping-pong tiles (64x128 tiles there: 35.0 and 33.2); 128x32768x4096 stays on
// 128x128 tiles (58.2; 64x128 63.8); 64x65536x4096 138.7 -> 125,
// 16x65536x1024 36.0 -> 23.0, 128x65536x1024 38.7 -> 31.9 and 128x65536x4096
// 151.9 -> 136.1 on lock-step tiles instead of 256x256 ones.
TileConfig choose_partial_round(const fuseml_gemm_desc& d, int cus) {
  struct Cand {
    const TileConfig* c;
    int w_one, w_two;  // weight with at most one / with two workgroups on a CU
  };
  // One lock-step workgroup per CU costs less beside a long K loop, where the
  // pipeline runs in its steady state longer than the epilogue takes.
  const int one = d.K > 2048 ? 7 : 8;
  const Cand cand[4] = {{&kSmall, one, 5}, {&kNarrow64, one, 5}, {&kNarrow32, one, 5}, {&kLarge128, 6, 6}};
  const TileConfig* best = cand[0].c;
  int64_t best_work = 0;
  for (const Cand& k : cand) {
    const int64_t tiles = cdiv(d.M, k.c->bm) * cdiv(d.N, k.c->bn);
    const int64_t work = cdiv(tiles, cus) * (k.c->bm + k.c->bn) * (tiles <= cus ? k.w_one : k.w_two);
    if (k.c == cand[0].c || work < best_work) {
      best = k.c;
      best_work = work;
    }
  }
  return *best;
}

// `cus`: the device's CU count (the 256-wide variants run one workgroup per CU).
// `d` has its flags derived (derive_flags).
TileConfig choose_config(const fuseml_gemm_desc& d, int cus) {
  // A pinned variant (tuning sweeps and the per-variant parity tests; deep3
  // falls back to deep when K % 64 != 0).
  switch (forced_variant()) {
    case 1: return kLarge;
    case 2: return kDeep;
    case 3: return d.K % 64 == 0 ? kDeep3 : kDeep;
    case 4: return kSmall;
    case kForcedDeep3Generic: return d.K % 64 == 0 ? kDeep3 : kDeep;
    case 6: return kNarrow64;
    case 7: return kNarrow32;
    case 8: return kLarge128;
    case 9: return kSmall64;
    default: break;
  }
  // A 256x256 tile keeps the LDS traffic per MFMA low enough for the MFMA pipe
  // to stay busy; below one full wave of 256-tile work the 128x128 variant
  // fills more CUs.  Of the 256x256 schedules, the one-wave-per-SIMD ones have
  // the faster K loop but the slower epilogue (no second wave on a SIMD to
  // overlap its latencies).  The whole-stage one wins from K = 2048 with at
  // least one full round of tiles (C4 2%, C5 4-10%, C2's second GEMM at K =
  // 4096 and 256 tiles 3%) or from K = 8192.  At K = 1024 its generic op loop
  // loses 12-16% on bias+GELU and C3's chain, but with a fixed-chain epilogue
  // it wins on every fixed chain (3-7% on 256 to 1024 tiles; none, bias, ReLU,
  // bias+ReLU, GELU(tanh), bias+residual, the act-heavy chain) except
  // bias+GELU(erf), which ties or loses up to 1.5%.  With K % 64 != 0 the
  // two-stage one takes over from K = 8192.
  // Below one round of 256x256 tiles (2 x large_tiles <= cus) the smaller
  // tiles (choose_partial_round): at 128 large tiles on 256 CUs the 128x128
  // one was 7-17% faster than 256x256 (bias+GELU at K = 512-1024), from 144
  // on the 256x256 ones are.
  // Decode-sized M against a wide weight (a 128-column tile per CU or more):
  // the GEMM streams the weight from HBM, so one row of tiles (the smallest
  // BM >= M: the weight read once) in K stages of 64 (128 contiguous bytes of
  // each weight row per stage where 32 fetch 64).  128x65536x8192 251.9 ->
  // 215.8 us and 128x32768x4096 59.6 -> 53.6 on the 128x128 tile at BK = 64
  // instead of 32 (eager 219.9 and 57.3); 64 and 16 rows: 113.0 and 41.8 on
  // 64x128 and 32x128 tiles (eager 134.2, 44.4).
  if (d.M <= 128 && cdiv(d.N, 128) >= cus) return d.M <= 32 ? kNarrow32 : d.M <= 64 ? kNarrow64 : kSmall64;
  const int64_t large_tiles = cdiv(d.M, 256) * cdiv(d.N, 256);
  if (2 * large_tiles <= cus || d.M <= 128) return choose_partial_round(d, cus);
  if (d.K % 64 == 0 && (d.K >= 8192 || (d.K >= 2048 && large_tiles >= cus))) return kDeep3;
  if (d.K % 64 == 0 && d.K >= 1024 && large_tiles >= cus) {
    const int ch = match_fixed_chain(d);
    if (ch != kChainGeneric && ch != kChainBiasGeluErf) return kDeep3;
  }
  return d.K >= 8192 ? kDeep : kLarge;
}

bool check_output(const fuseml_output& o, const fuseml_gemm_desc& d, const char* what) {
  if (o.ptr == nullptr) return true;
  if (o.dtype < FUSEML_BF16 || o.dtype > FUSEML_F32) {
    set_error("%s: unknown dtype %d", what, o.dtype);
    return false;
  }
  if (o.ld < d.N) {
    set_error("%s: row stride %lld < N %lld", what, (long long)o.ld, (long long)d.N);
    return false;
  }
  return true;
}

int validate(const fuseml_gemm_desc* dp) {
  if (dp == nullptr) {
    set_error("null descriptor");
    return FUSEML_EINVAL;
  }
  const fuseml_gemm_desc& d = *dp;
  if (d.M <= 0 || d.N <= 0 || d.K < 0) {
    set_error("bad problem size M=%lld N=%lld K=%lld", (long long)d.M, (long long)d.N,
              (long long)d.K);
    return FUSEML_EINVAL;
  }
  if (d.M >= ((int64_t)1 << 30) || d.N >= ((int64_t)1 << 30) || d.K >= ((int64_t)1 << 30)) {
    set_error("problem dimension exceeds 2^30");
    return FUSEML_EUNSUPPORTED;
  }
  if (d.ab_dtype != FUSEML_BF16 && d.ab_dtype != FUSEML_F16) {
    set_error("GEMM operand dtype %d has no MFMA variant (bf16/f16 only)", d.ab_dtype);
    return FUSEML_EUNSUPPORTED;
  }
  if (d.K > 0 && (d.a == nullptr || d.b == nullptr)) {
    set_error("null GEMM operand");
    return FUSEML_EINVAL;
  }
  if (d.K > 0 && (d.K % 8 != 0 || d.lda % 8 != 0 || d.ldb % 8 != 0 || ((uintptr_t)d.a & 15) ||
      ((uintptr_t)d.b & 15))) {
    set_error("GEMM operands need K, lda, ldb multiples of 8 and 16-byte aligned bases "
              "(K=%lld lda=%lld ldb=%lld)",
              (long long)d.K, (long long)d.lda, (long long)d.ldb);
    return FUSEML_EUNSUPPORTED;
  }
  if (d.K > 0 && (d.lda < d.K || d.ldb < d.K)) {
    set_error("row stride smaller than K");
    return FUSEML_EINVAL;
  }
  // Buffer resources are based at each tile's origin: the rows one tile reads
  // must span less than 2 GiB (the whole operand may be larger).
  const int64_t tm = d.M < kTileSpan ? d.M : kTileSpan, tn = d.N < kTileSpan ? d.N : kTileSpan;
  if (d.K > 0 && (((tm - 1) * d.lda + d.K) * 2 >= kMaxBytes || ((tn - 1) * d.ldb + d.K) * 2 >= kMaxBytes)) {
    set_error("GEMM operand rows of one tile span 2 GiB or more (lda=%lld ldb=%lld)", (long long)d.lda,
              (long long)d.ldb);
    return FUSEML_EUNSUPPORTED;
  }
  if (d.n_ops < 0 || d.n_ops > FUSEML_MAX_OPS || d.n_operands < 0 ||
      d.n_operands > FUSEML_MAX_OPERANDS || d.n_extra < 0 || d.n_extra > FUSEML_MAX_EXTRA_OUT) {
    set_error("op/operand/extra counts out of range");
    return FUSEML_EINVAL;
  }
  for (int i = 0; i < d.n_operands; ++i) {
    const fuseml_operand& op = d.operands[i];
    if (op.ptr == nullptr || op.dtype < FUSEML_BF16 || op.dtype > FUSEML_F32 || op.stride_m < 0 ||
        op.stride_n < 0 || op.extent <= 0) {
      set_error("operand %d malformed", i);
      return FUSEML_EINVAL;
    }
    const int64_t need = (d.M - 1) * op.stride_m + (d.N - 1) * op.stride_n + 1;
    if (op.extent < need) {
      set_error("operand %d extent %lld < reachable %lld", i, (long long)op.extent,
                (long long)need);
      return FUSEML_EINVAL;
    }
    if (((tm - 1) * op.stride_m + (tn - 1) * op.stride_n + 1) * (op.dtype == FUSEML_F32 ? 4 : 2) >= kMaxBytes) {
      set_error("operand %d: one tile's elements span 2 GiB or more", i);
      return FUSEML_EUNSUPPORTED;
    }
  }
  for (int i = 0; i < d.n_ops; ++i) {
    const fuseml_epi_op& o = d.ops[i];
    if (o.kind < FUSEML_OP_ADD || o.kind > FUSEML_OP_MUL_SELF) {
      set_error("op %d: unknown kind %d", i, o.kind);
      return FUSEML_EINVAL;
    }
    if ((o.kind == FUSEML_OP_ADD || o.kind == FUSEML_OP_MUL) &&
        (o.operand < 0 || o.operand >= d.n_operands)) {
      set_error("op %d: operand index %d out of range", i, o.operand);
      return FUSEML_EINVAL;
    }
    if (o.kind == FUSEML_OP_STORE &&
        (o.operand < 0 || o.operand >= d.n_extra || d.extra[o.operand].ptr == nullptr)) {
      set_error("op %d: extra output %d missing", i, o.operand);
      return FUSEML_EINVAL;
    }
  }
  if (!check_output(d.out, d, "out")) return FUSEML_EINVAL;
  for (int i = 0; i < d.n_extra; ++i)
    if (!check_output(d.extra[i], d, "extra")) return FUSEML_EINVAL;
  if (d.reduce_mask & ~7u) {
    set_error("unknown reduction bits 0x%x", d.reduce_mask);
    return FUSEML_EINVAL;
  }
  if (d.reduce_mask) {
    if (d.reduce_axis != 0 && d.reduce_axis != 1) {
      set_error("reduce_axis must be 0 or 1");
      return FUSEML_EINVAL;
    }
    for (int b = 0; b < 3; ++b)
      if ((d.reduce_mask & (1u << b)) && d.reduce_out[b] == nullptr) {
        set_error("reduction output %d missing", b);
        return FUSEML_EINVAL;
      }
  }
  if (d.out.ptr == nullptr && d.reduce_mask == 0 && d.n_extra == 0) {
    set_error("descriptor produces no output");
    return FUSEML_EINVAL;
  }
  return FUSEML_OK;
}

// A chain that has no main output and ends in an escape store writes that
// store as the main output: through the LDS staging tile as whole rows, not
// from the accumulator layout (32 rows per store instruction).  The values and
// the reductions after the chain are unchanged.
void fold_final_store(fuseml_gemm_desc& d) {
  if (d.out.ptr != nullptr || d.n_ops == 0) return;
  const fuseml_epi_op& last = d.ops[d.n_ops - 1];
  if (last.kind != FUSEML_OP_STORE) return;
  d.out = d.extra[last.operand];
  d.n_ops -= 1;
}

// Fill in the host-derived access-path flags (kept in the `reserved` fields).
void derive_flags(fuseml_gemm_desc& d) {
  for (int i = 0; i < d.n_operands; ++i) {
    fuseml_operand& op = d.operands[i];
    const int eb = op.dtype == FUSEML_F32 ? 4 : 2;
    const bool vec = op.stride_n == 1 && (op.stride_m % 4 == 0) && (d.N % 4 == 0) &&
                     ((uintptr_t)op.ptr % (4 * eb) == 0);
    // Column reductions write their partials over the staging tile while other
    // waves are still in the op chain, so they rule out a staged operand.
    const bool stage = eb == 2 && op.stride_n == 1 && op.stride_m != 0 && (op.stride_m % 8 == 0) &&
                       (d.N % 8 == 0) && ((uintptr_t)op.ptr % 16 == 0) &&
                       !(d.reduce_mask != 0 && d.reduce_axis == 0);
    op.reserved = (vec ? kFlagVec4 : 0) | (stage ? kFlagStage : 0);
  }
  // Vector operands of ADD/MUL ops get LDS slots, in first-use order.
  int slots = 0;
  for (int o = 0; o < d.n_ops && slots < kAuxSlots; ++o) {
    const int k = d.ops[o].kind;
    if (k != FUSEML_OP_ADD && k != FUSEML_OP_MUL) continue;
    fuseml_operand& op = d.operands[d.ops[o].operand];
    if ((op.reserved & kFlagAux) || (op.stride_m != 0 && op.stride_n != 0)) continue;
    op.reserved = (op.reserved & ~kFlagStage) | kFlagAux | (slots << 8);
    ++slots;
  }
  auto out_flags = [&](fuseml_output& o) {
    const int eb = o.dtype == FUSEML_F32 ? 4 : 2;
    const bool vec = o.ptr != nullptr && o.ld % 4 == 0 && d.N % 4 == 0 && (uintptr_t)o.ptr % (4 * eb) == 0;
    const bool stage = o.ptr != nullptr && eb == 2 && o.ld % 8 == 0 && d.N % 8 == 0 &&
                       (uintptr_t)o.ptr % 16 == 0;
    o.reserved = (vec ? kFlagVec4 : 0) | (stage ? kFlagStage : 0);
  };
  out_flags(d.out);
  for (int i = 0; i < d.n_extra; ++i) out_flags(d.extra[i]);
}

// The fixed chain (FixedChain) that expresses the descriptor's epilogue, or
// kChainGeneric.  Called after derive_flags: a "row" operand is a [N] vector
// holding an LDS slot, a "tile" operand the LDS-staged bf16 2-D operand.
// Fixed chains are built for bf16 GEMM operands, no escape stores, and no
// reductions except after a lone relu (the ReLU + row/column reductions
// group).
int match_fixed_chain(const fuseml_gemm_desc& d) {
  if (d.ab_dtype != FUSEML_BF16 || d.n_extra != 0) return kChainGeneric;
  auto is = [&](int o, int kind) { return o < d.n_ops && d.ops[o].kind == kind; };
  auto row = [&](int o) {
    if (!is(o, FUSEML_OP_ADD)) return false;
    const fuseml_operand& op = d.operands[d.ops[o].operand];
    return (op.reserved & kFlagAux) != 0 && op.stride_m == 0;
  };
  auto tile = [&](int o, int kind) {
    if (!is(o, kind)) return false;
    const fuseml_operand& op = d.operands[d.ops[o].operand];
    return (op.reserved & kFlagStage) != 0 && op.dtype == FUSEML_BF16;
  };
  int ch = kChainGeneric;
  switch (d.n_ops) {
    case 0: ch = kChainNone; break;
    case 1:
      if (row(0)) ch = kChainBias;
      else if (is(0, FUSEML_OP_RELU)) ch = kChainRelu;
      break;
    case 2:
      if (row(0) && is(1, FUSEML_OP_GELU_ERF)) ch = kChainBiasGeluErf;
      else if (row(0) && is(1, FUSEML_OP_GELU_TANH)) ch = kChainBiasGeluTanh;
      else if (row(0) && is(1, FUSEML_OP_RELU)) ch = kChainBiasRelu;
      else if (row(0) && tile(1, FUSEML_OP_ADD)) ch = kChainBiasTile;
      break;
    case 5:
      if (row(0) && is(1, FUSEML_OP_RELU) && tile(2, FUSEML_OP_MUL) && is(3, FUSEML_OP_SIGMOID) && row(4))
        ch = kChainActHeavy;
      break;
    default: break;
  }
  if (d.reduce_mask != 0 && ch != kChainRelu) return kChainGeneric;
  return ch;
}

// `max_wg` caps the grid (0: one workgroup per tile); the kernel loops over the
// remaining tiles.
template <const TileConfig& C>
hipError_t launch_variant(const fuseml_gemm_desc& d, hipStream_t stream, int max_wg) {
  int64_t tiles = cdiv(d.M, C.bm) * cdiv(d.N, C.bn);
  if (max_wg > 0 && tiles > max_wg) tiles = max_wg;
  const dim3 grid((unsigned)tiles), block(C.wm * C.wn * 64);
  const bool red = d.reduce_mask != 0;
  constexpr int G = kChainGeneric;
  if (d.ab_dtype == FUSEML_BF16 && !red)
    hipLaunchKernelGGL((gemm_epilogue_kernel<C.bm, C.bn, C.bk, C.stages, C.wm, C.wn, C.sched, __bf16, false, G>),
                       grid, block, 0, stream, d);
  else if (d.ab_dtype == FUSEML_BF16)
    hipLaunchKernelGGL((gemm_epilogue_kernel<C.bm, C.bn, C.bk, C.stages, C.wm, C.wn, C.sched, __bf16, true, G>),
                       grid, block, 0, stream, d);
  else if (!red)
    hipLaunchKernelGGL((gemm_epilogue_kernel<C.bm, C.bn, C.bk, C.stages, C.wm, C.wn, C.sched, _Float16, false, G>),
                       grid, block, 0, stream, d);
  else
    hipLaunchKernelGGL((gemm_epilogue_kernel<C.bm, C.bn, C.bk, C.stages, C.wm, C.wn, C.sched, _Float16, true, G>),
                       grid, block, 0, stream, d);
  return hipGetLastError();
}

// A fixed-chain kernel of variant C (bf16 operands; reductions only with
// kChainRelu, as match_fixed_chain guarantees).
template <const TileConfig& C, int CH>
void launch_fixed_one(const fuseml_gemm_desc& d, hipStream_t stream, dim3 grid, dim3 block) {
  if constexpr (CH == kChainRelu) {
    if (d.reduce_mask != 0) {
      hipLaunchKernelGGL((gemm_epilogue_kernel<C.bm, C.bn, C.bk, C.stages, C.wm, C.wn, C.sched, __bf16, true, CH>),
                         grid, block, 0, stream, d);
      return;
    }
  }
  hipLaunchKernelGGL((gemm_epilogue_kernel<C.bm, C.bn, C.bk, C.stages, C.wm, C.wn, C.sched, __bf16, false, CH>),
                     grid, block, 0, stream, d);
}

template <const TileConfig& C>
hipError_t launch_fixed(const fuseml_gemm_desc& d, int ch, hipStream_t stream, int max_wg) {
  int64_t tiles = cdiv(d.M, C.bm) * cdiv(d.N, C.bn);
  if (max_wg > 0 && tiles > max_wg) tiles = max_wg;
  const dim3 grid((unsigned)tiles), block(C.wm * C.wn * 64);
  switch (ch) {
    case kChainNone: launch_fixed_one<C, kChainNone>(d, stream, grid, block); break;
    case kChainBias: launch_fixed_one<C, kChainBias>(d, stream, grid, block); break;
    case kChainBiasGeluErf: launch_fixed_one<C, kChainBiasGeluErf>(d, stream, grid, block); break;
    case kChainBiasGeluTanh: launch_fixed_one<C, kChainBiasGeluTanh>(d, stream, grid, block); break;
    case kChainBiasRelu: launch_fixed_one<C, kChainBiasRelu>(d, stream, grid, block); break;
    case kChainBiasTile: launch_fixed_one<C, kChainBiasTile>(d, stream, grid, block); break;
    case kChainActHeavy: launch_fixed_one<C, kChainActHeavy>(d, stream, grid, block); break;
    case kChainRelu: launch_fixed_one<C, kChainRelu>(d, stream, grid, block); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The fixed chain a launch of `d` (flags derived) on variant `c` runs, or
// kChainGeneric: fixed chains are built for the one-wave whole-stage variant.
int launch_chain(const fuseml_gemm_desc& d, const TileConfig& c) {
  if (c.sched != kDeep3.sched || forced_variant() == kForcedDeep3Generic) return kChainGeneric;
  return match_fixed_chain(d);
}

// Per-device check and CU count, queried once per device: the CU count for a
// gfx950 device, else FUSEML_EDEVICE or FUSEML_EHIP (negative; the error is set).
constexpr int kMaxDevices = 64;
std::atomic<int> g_device_cus[kMaxDevices];

int device_cus(int dev) {
  if (dev >= 0 && dev < kMaxDevices) {
    const int known = g_device_cus[dev].load(std::memory_order_relaxed);
    if (known > 0) return known;
  }
  char arch[64];
  if (fuseml_device_arch(dev, arch, sizeof(arch)) != FUSEML_OK) return FUSEML_EHIP;
  if (strncmp(arch, "gfx950", 6) != 0) {
    set_error("device %d is %s; kernels are built for gfx950 only", dev, arch);
    return FUSEML_EDEVICE;
  }
  int cus = 0;
  const hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess || cus <= 0) {
    set_error("hipDeviceGetAttribute(MultiprocessorCount): %s", hipGetErrorString(e));
    return FUSEML_EHIP;
  }
  if (dev >= 0 && dev < kMaxDevices) g_device_cus[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

}  // namespace

namespace fuseml_detail {
// Error text for the other translation units of the library (mlp_block.hip).
void set_error_text(const char* msg) {
  strncpy(g_last_error, msg, sizeof(g_last_error) - 1);
  g_last_error[sizeof(g_last_error) - 1] = '\0';
}
}  // namespace fuseml_detail

extern "C" {

const char* fuseml_last_error(void) { return g_last_error; }

int fuseml_abi_version(void) { return FUSEML_ABI_VERSION; }

size_t fuseml_desc_size(void) { return sizeof(fuseml_gemm_desc); }

size_t fuseml_mlp_desc_size(void) { return sizeof(fuseml_mlp_desc); }

int fuseml_gemm_epilogue_supported(const fuseml_gemm_desc* desc) {
  g_last_error[0] = '\0';
  return validate(desc) == FUSEML_OK ? 1 : 0;
}

int fuseml_gemm_epilogue_config(const fuseml_gemm_desc* desc, int32_t cfg[4]) {
  g_last_error[0] = '\0';
  const int rc = validate(desc);
  if (rc != FUSEML_OK) return rc;
  // The CU count of the current device if it is known, else MI355X's.
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices) {
    const int known = g_device_cus[dev].load(std::memory_order_relaxed);
    if (known > 0) cus = known;
  }
  fuseml_gemm_desc d = *desc;
  fold_final_store(d);
  derive_flags(d);
  const TileConfig c = choose_config(d, cus);
  cfg[0] = c.bm;
  cfg[1] = c.bn;
  cfg[2] = c.wm * c.wn;
  cfg[3] = c.lds_bytes();
  return FUSEML_OK;
}

int fuseml_gemm_epilogue_chain(const fuseml_gemm_desc* desc) {
  g_last_error[0] = '\0';
  const int rc = validate(desc);
  if (rc != FUSEML_OK) return rc;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices) {
    const int known = g_device_cus[dev].load(std::memory_order_relaxed);
    if (known > 0) cus = known;
  }
  fuseml_gemm_desc d = *desc;
  fold_final_store(d);
  derive_flags(d);
  return launch_chain(d, choose_config(d, cus));
}

int fuseml_gemm_epilogue_force_variant(const char* name) {
  g_last_error[0] = '\0';
  const int v = variant_code(name);
  if (v < 0) {
    set_error("unknown variant '%s' (large, deep, deep3, small, deep3-generic, narrow64, narrow32, large128, small64 "
              "or auto)", name);
    return FUSEML_EINVAL;
  }
  forced_variant();  // the environment is read first, so it cannot override this later
  g_forced_variant.store(v, std::memory_order_relaxed);
  return FUSEML_OK;
}

int fuseml_device_arch(int device, char* buf, int buflen) {
  hipDeviceProp_t prop;
  const hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) {
    set_error("hipGetDeviceProperties: %s", hipGetErrorString(e));
    return FUSEML_EHIP;
  }
  if (buf != nullptr && buflen > 0) {
    strncpy(buf, prop.gcnArchName, (size_t)buflen - 1);
    buf[buflen - 1] = '\0';
  }
  return FUSEML_OK;
}

int fuseml_gemm_epilogue(const fuseml_gemm_desc* desc, void* stream_ptr) {
  g_last_error[0] = '\0';
  int rc = validate(desc);
  if (rc != FUSEML_OK) return rc;
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_ptr);

  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("hipGetDevice: %s", hipGetErrorString(e));
    return FUSEML_EHIP;
  }
  const int cus = device_cus(dev);
  if (cus <= 0) return cus < 0 ? cus : FUSEML_EHIP;

  fuseml_gemm_desc d = *desc;
  fold_final_store(d);
  derive_flags(d);

  if (d.reduce_mask) {
    const int len = (int)(d.reduce_axis == 1 ? d.M : d.N);
    float* sum = (d.reduce_mask & FUSEML_RED_SUM) ? d.reduce_out[0] : nullptr;
    float* amax = (d.reduce_mask & FUSEML_RED_AMAX) ? d.reduce_out[1] : nullptr;
    float* mean = (d.reduce_mask & FUSEML_RED_MEAN) ? d.reduce_out[2] : nullptr;
    hipLaunchKernelGGL(reduce_fill_kernel, dim3((unsigned)cdiv(len, 256)), dim3(256), 0, stream,
                       sum, amax, mean, len);
    e = hipGetLastError();
    if (e != hipSuccess) {
      set_error("reduce_fill launch: %s", hipGetErrorString(e));
      return FUSEML_EHIP;
    }
  }

  const TileConfig c = choose_config(d, cus);
  const int ch = launch_chain(d, c);
  if (ch != kChainGeneric)
    e = launch_fixed<kDeep3>(d, ch, stream, cus);
  else if (c.sched == kDeep.sched)
    e = launch_variant<kDeep>(d, stream, cus);
  else if (c.sched == kLarge.sched && c.bn == kLarge128.bn)
    e = launch_variant<kLarge128>(d, stream, cus);
  else if (c.sched == kLarge.sched)
    e = launch_variant<kLarge>(d, stream, cus);
  else if (c.sched == kDeep3.sched)
    e = launch_variant<kDeep3>(d, stream, cus);
  else if (c.bm == kSmall64.bm && c.bk == kSmall64.bk)
    e = launch_variant<kSmall64>(d, stream, 0);
  else if (c.bm == kNarrow64.bm)
    e = launch_variant<kNarrow64>(d, stream, 0);
  else if (c.bm == kNarrow32.bm)
    e = launch_variant<kNarrow32>(d, stream, 0);
  else
    e = launch_variant<kSmall>(d, stream, 0);
  if (e != hipSuccess) {
    set_error("gemm_epilogue launch: %s", hipGetErrorString(e));
    return FUSEML_EHIP;
  }
  return FUSEML_OK;
}

}  // extern "C"