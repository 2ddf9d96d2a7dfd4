// gemm_epilogue_kernel.h — the gfx950 fused GEMM+epilogue kernel template.
// Included only by the per-variant instantiation units (gemm_epilogue_v_*.hip);
// the host side (validation, variant choice, launch, C ABI) is gemm_epilogue.hip.
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
// Kernel structure (per workgroup: one BM x BN output tile at a time):
//   * Both operands are K-contiguous in HBM (A = x[M,K]; B = t(W), i.e. W[N,K]).
//     A K-stage holds BK columns of the tile's A rows and W rows in LDS, rows of
//     2*BK bytes with the 16-byte chunk index XOR-swizzled so that the MFMA
//     fragment reads (ds_read_b128) are free of bank conflicts.
//   * Stages are filled by the global -> LDS DMA (buffer_load_dwordx4 ... lds):
//     no staging registers, and an out-of-range offset returns zeros, which masks
//     the M/N/K edges with no branches.
//   * Four K-loop schedules (template parameter SCHED), one per tile variant:
//     256x256 ping-pong (8 waves, two groups alternating memory and compute
//     phases, BK=32, 4 stages), 256x256 one wave per SIMD (4 waves, 128x128
//     accumulators in AGPRs, BK=64, 2 stages) in two forms (one k-step of
//     fragments read ahead, or a whole stage of fragments read during its
//     first k-step so that the next stage's DMA spreads over the other three),
//     and 128x128 lock-step.
//   * MFMA roles are swapped (MFMA "A" = rows of W, MFMA "B" = rows of x) so that
//     each lane's accumulator holds one output row m and runs of 4 consecutive
//     columns n; a row reduction needs a single cross-half-wave exchange.
//   * Epilogue: the op chain from the kernel-argument descriptor, one column
//     block at a time in a runtime loop (one copy of the op code).  Vector
//     operands come from fp32 LDS slots, the first 2-D operand from an LDS
//     staging tile (fetched by the DMA during the K loop's last stages in the
//     256-wide variants), and the output is staged in LDS and stored as whole
//     rows.
//   * The 256-wide variants launch at most one workgroup per CU, each running
//     tiles b, b + grid, ... in turn.  The tile map is XCD-aware: the hardware
//     deals workgroups to the 8 XCDs round-robin, so each XCD is given a
//     contiguous range of each round's logical tiles, ordered in GROUP_M-row
//     column strips for L2 reuse.
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "amax_order.h"
#include "fuseml_hip.h"
#include "gelu_phi.h"
#include "gemm_epilogue_shared.h"

namespace fuseml_gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));

constexpr int kGroupM = 8;              // tile-row strip height of the tile order
constexpr uint32_t kOOB = 0x80000000u;  // buffer offset that always reads zero
constexpr int kRsrcWord3 = 0x00020000;  // buffer descriptor word 3 for gfx9 (32-bit data)
constexpr float kFp16Max = 65504.0f;

// The kernel reads its descriptor in place from the kernel-argument segment
// (constant address space, scalar loads) instead of through the by-value
// parameter, whose address the compiler would otherwise copy to scratch.
typedef const __attribute__((address_space(4))) fuseml_gemm_desc KDesc;


// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

// Buffer resource over [p, p + bytes).  Every caller passes wave-uniform
// values; readfirstlane states that to the compiler, which otherwise may build
// the descriptor in VGPRs and wrap each buffer access in a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* q = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(q, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), kRsrcWord3);
}

// Buffer resource over [p + skip, p + total): the caller's offsets are relative
// to p + skip, so only the span one tile touches must fit the 32-bit offsets
// (the host checks that), not the whole operand.  The record count is clamped
// to 2^31 - 1; an offset at or past it reads zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_at(const void* p, int64_t skip, int64_t total) {
  const int64_t rest = total - skip;
  const uint32_t bytes = rest <= 0 ? 0u : (rest >= 0x7fffffffLL ? 0x7fffffffu : (uint32_t)rest);
  return make_rsrc(static_cast<const char*>(p) + skip, bytes);
}

template <typename T>
__device__ __forceinline__ f32x16_t mfma32(i32x4_t a, i32x4_t b, f32x16_t c);

template <>
__device__ __forceinline__ f32x16_t mfma32<__bf16>(i32x4_t a, i32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                  __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x16_t mfma32<_Float16>(i32x4_t a, i32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                 __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ float elem_to_f32(uint32_t bits, int dtype) {
  if (dtype == FUSEML_BF16) return bf16_bits_to_f32(bits & 0xffffu);
  if (dtype == FUSEML_F16) return f16_bits_to_f32(bits & 0xffffu);
  return __uint_as_float(bits);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  __bf16 h = (__bf16)x;  // round-to-nearest-even (v_cvt_pk_bf16_f32)
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// IEEE 754-2019 maximum / minimum: NaN if either operand is NaN (torch.amax
// and torch.clamp semantics; fmaxf / fminf return the other operand).  One
// v_maximum3_f32 / v_minimum3_f32 each on gfx950.
__device__ __forceinline__ float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float min_nan(float a, float b) { return __builtin_elementwise_minimum(a, b); }

__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
  // Saturate to the finite fp16 range before narrowing
  // (fuseml/codegen/kernel_generator.py:1575-1581); NaN stays NaN.
  x = min_nan(max_nan(x, -kFp16Max), kFp16Max);
  _Float16 h = (_Float16)x;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Two values to packed 16-bit (a in the low half) with one v_cvt_pk_* each;
// the same rounding (and fp16 saturation) as the scalar conversions above.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  a = min_nan(max_nan(a, -kFp16Max), kFp16Max);
  b = min_nan(max_nan(b, -kFp16Max), kFp16Max);
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}

__device__ __forceinline__ int dtype_bytes(int dtype) { return dtype == FUSEML_F32 ? 4 : 2; }

// Load the 4 operand values at (m, n..n+3) of the tile at (m0, n0).  `ok` says
// the whole run of four is inside [0,M) x [0,N); an invalid run reads zeros
// through the buffer bound.  Offsets are relative to the tile origin.
template <typename Op>
__device__ __forceinline__ void load_operand4(const Op& op, int m0, int n0, int m, int n, bool ok, float v[4]) {
  const int dt = op.dtype;
  const int eb = dtype_bytes(dt);
  const __amdgpu_buffer_rsrc_t r =
      make_rsrc_at(op.ptr, ((int64_t)m0 * op.stride_m + (int64_t)n0 * op.stride_n) * eb, op.extent * eb);
  const int64_t base = (int64_t)(m - m0) * op.stride_m + (int64_t)(n - n0) * op.stride_n;
  if (op.reserved & kFlagVec4) {
    // Unit stride along N and 4-element aligned rows: one vector load.
    const uint32_t off = ok ? (uint32_t)(base * eb) : kOOB;
    if (dt == FUSEML_F32) {
      i32x4_t x = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
      v[0] = __int_as_float(x.x); v[1] = __int_as_float(x.y);
      v[2] = __int_as_float(x.z); v[3] = __int_as_float(x.w);
    } else {
      i32x2_t x = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
      v[0] = elem_to_f32((uint32_t)x.x & 0xffffu, dt);
      v[1] = elem_to_f32((uint32_t)x.x >> 16, dt);
      v[2] = elem_to_f32((uint32_t)x.y & 0xffffu, dt);
      v[3] = elem_to_f32((uint32_t)x.y >> 16, dt);
    }
    return;
  }
  if (op.stride_n == 0) {
    const uint32_t off = ok ? (uint32_t)(base * eb) : kOOB;
    uint32_t bits = (eb == 4) ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0)
                              : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    const float x = elem_to_f32(bits, dt);
    v[0] = v[1] = v[2] = v[3] = x;
    return;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t off = ok ? (uint32_t)((base + (int64_t)e * op.stride_n) * eb) : kOOB;
    uint32_t bits = (eb == 4) ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0)
                              : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    v[e] = elem_to_f32(bits, dt);
  }
}

// Store 4 values to (m, n..n+3) of a row-major output; vector store when the
// output rows are 4-element aligned (o.reserved set by the host).
template <typename Out>
__device__ __forceinline__ void store_out4(const Out& o, int m, int n, int M, int N, const float v[4]) {
  if (m >= M || n >= N) return;
  const int64_t base = (int64_t)m * o.ld + n;
  if (o.dtype == FUSEML_F32) {
    float* p = reinterpret_cast<float*>(o.ptr) + base;
    if (o.reserved & kFlagVec4) {
      *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      for (int e = 0; e < 4 && n + e < N; ++e) p[e] = v[e];
    }
    return;
  }
  uint2 w;
  if (o.dtype == FUSEML_BF16)
    w = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
  else
    w = make_uint2(pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3]));
  uint16_t* p = reinterpret_cast<uint16_t*>(o.ptr) + base;
  if (o.reserved & kFlagVec4) {
    *reinterpret_cast<uint2*>(p) = w;
  } else {
    for (int e = 0; e < 4 && n + e < N; ++e) p[e] = (uint16_t)((e < 2 ? w.x : w.y) >> (16 * (e & 1)));
  }
}

// Float atomic max through integer atomics, dispatched on the sign bit
// (amax_order.h: -0.0 takes the unsigned-min path like every other value with
// the sign bit set; NaN is written as 0x7fc00000 and then always kept).
__device__ __forceinline__ void atomic_max_f32(float* p, float v) {
  uint32_t bits;
  if (fuseml_amax::atomic_for(__float_as_uint(v), &bits) == fuseml_amax::kSignedMax)
    atomicMax(reinterpret_cast<int*>(p), (int)bits);
  else
    atomicMin(reinterpret_cast<unsigned int*>(p), bits);
}


// Standard normal CDF for GELU (approximate='none'): the constrained fit of
// gelu_phi.h (|Phi error| <= 1.5e-5 in float32; beyond the clamp Phi is 1
// above and 2e-8 below, so GELU there is x or ~0).
using namespace fuseml_phi;

// LDS stage geometry for a K depth of BK 16-bit elements.  A stage row (one row
// of A or of W) is BK*2 bytes = BK/8 chunks of 16 bytes.  A ds_read_b128 is
// served 16 lanes at a time across 64 four-byte banks (256 bytes), which hold
// 256/(BK*2) consecutive rows; XOR-ing the chunk index with
// (row / rows_per_sweep) % chunks gives the 16 consecutive rows that one
// fragment read touches 16 distinct 16-byte bank groups (no conflicts).
template <int BK>
struct StageGeom {
  static constexpr int kRowBytes = BK * 2;
  static constexpr int kChunks = BK / 8;
  static constexpr int kRowsPerSweep = 256 / kRowBytes;
  static constexpr int kRowsPerDma = 1024 / kRowBytes;  // rows one wave-wide 16-byte DMA fills
  static_assert(kRowsPerSweep * kChunks == 16, "swizzle covers one 16-lane bank sweep");
  __device__ static __forceinline__ int swizzle(int row) { return (row / kRowsPerSweep) & (kChunks - 1); }
};

// s_waitcnt lgkmcnt(0) (LDS reads returned), other counters unconstrained.
__device__ __forceinline__ void wait_lgkmcnt0() {
  __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4));
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at maximum).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier that orders LDS accesses only: this wave's LDS operations
// complete, then s_barrier.  __syncthreads() adds a release fence, which also
// waits for every global load, store and LDS DMA this wave has in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  wait_lgkmcnt0();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).  Used
// wherever an accumulator array is indexed, so every index is a constant and
// the arrays stay in registers whatever the unroller decides.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// The activations over G independent elements, evaluated one step at a time
// across all of them, with a scheduling barrier between steps: a dependent
// instruction issues G instructions after its input instead of right behind it,
// which a lone wave on a SIMD (nothing else to issue while a dependent VALU op
// waits) needs to keep the VALU busy.
__device__ __forceinline__ void step_boundary() { __builtin_amdgcn_sched_barrier(0); }

// GELU (approximate='none'): x * Phi(x), with Phi(x) = 0.5 + xc * Q(xc^2),
// xc = clamp(x, +-3 sqrt 2), Q in Horner form.
template <int G>
__device__ __forceinline__ void gelu_erf_n(float* v) {
  float xc[G], t[G], q[G];
  static_for<0, G>([&](auto e) { xc[e] = __builtin_amdgcn_fmed3f(v[e], -kPhiClamp, kPhiClamp); });
  step_boundary();
  static_for<0, G>([&](auto e) { t[e] = xc[e] * xc[e]; });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(kPhiQ8, t[e], kPhiQ7); });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(q[e], t[e], kPhiQ6); });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(q[e], t[e], kPhiQ5); });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(q[e], t[e], kPhiQ4); });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(q[e], t[e], kPhiQ3); });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(q[e], t[e], kPhiQ2); });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(q[e], t[e], kPhiQ1); });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(q[e], t[e], kPhiQ0); });
  step_boundary();
  static_for<0, G>([&](auto e) { q[e] = fmaf(xc[e], q[e], 0.5f); });
  step_boundary();
  static_for<0, G>([&](auto e) { v[e] = v[e] * q[e]; });
}

// Logistic function from the hardware exp2 and reciprocal (about 1 ulp each):
// 1 / (1 + 2^(-x log2 e)).
template <int G>
__device__ __forceinline__ void sigmoid_n(float* v) {
  float d[G];
  static_for<0, G>([&](auto e) { d[e] = -1.4426950408889634f * v[e]; });
  step_boundary();
  static_for<0, G>([&](auto e) { d[e] = __builtin_amdgcn_exp2f(d[e]); });
  step_boundary();
  static_for<0, G>([&](auto e) { d[e] = 1.0f + d[e]; });
  step_boundary();
  static_for<0, G>([&](auto e) { v[e] = __builtin_amdgcn_rcpf(d[e]); });
}

// GELU, approximate='tanh': 0.5 x (1 + tanh(u)) with u = sqrt(2/pi)(x + 0.044715 x^3)
// (Hendrycks & Gimpel 2016).  Since 0.5 (1 + tanh(u)) = sigmoid(2u), this is
// x * sigmoid(2u), 2u = 2x * (sqrt(2/pi) + sqrt(2/pi) 0.044715 x^2).
template <int G>
__device__ __forceinline__ void gelu_tanh_n(float* v) {
  constexpr float kC = 0.79788456080286536f;  // sqrt(2/pi)
  float u[G];
  static_for<0, G>([&](auto e) { u[e] = v[e] * v[e]; });
  step_boundary();
  static_for<0, G>([&](auto e) { u[e] = fmaf(kC * 0.044715f, u[e], kC); });
  step_boundary();
  static_for<0, G>([&](auto e) { u[e] = (2.0f * v[e]) * u[e]; });
  step_boundary();
  sigmoid_n<G>(u);
  step_boundary();
  static_for<0, G>([&](auto e) { v[e] = v[e] * u[e]; });
}

// LDS staging tile of BN 16-bit columns per row.  The 32 rows that one
// ds_read_b64/ds_write_b64 of the accumulator layout touches must land in 32
// distinct bank pairs, and a whole-row pass of 16-byte chunk accesses must not
// conflict either.
//  * BN >= 256 (32 or more chunks per row): chunk c of row r sits at chunk
//    c ^ (r & 31).  Chunks stay whole, so the tile can be filled by the LDS DMA.
//  * BN = 128 (16 chunks): 8-byte units are XOR-swizzled by (r & 31) instead,
//    which swaps the two halves of a chunk on odd rows.
template <int BN>
constexpr bool kChunkSwizzle = BN >= 256;

// Byte address of 8-byte unit u (four 16-bit elements) of row r.
template <int BN>
__device__ __forceinline__ int stage_unit(int r, int u) {
  if constexpr (kChunkSwizzle<BN>)
    return r * (2 * BN) + ((((u >> 1) ^ (r & 31)) << 4) | ((u & 1) << 3));
  else
    return r * (2 * BN) + ((u ^ (r & 31)) << 3);
}

// Byte address of 16-byte chunk c of row r; read or written whole, its halves
// are swapped when stage_swapped(r).
template <int BN>
__device__ __forceinline__ int stage_chunk(int r, int c) {
  if constexpr (kChunkSwizzle<BN>)
    return r * (2 * BN) + ((c ^ (r & 31)) << 4);
  else
    return r * (2 * BN) + (((2 * c) ^ (r & 31)) & ~1) * 8;
}

template <int BN>
__device__ __forceinline__ bool stage_swapped(int r) {
  return !kChunkSwizzle<BN> && (r & 1);
}

__device__ __forceinline__ i32x4_t swap_halves(i32x4_t x) { return i32x4_t{x.z, x.w, x.x, x.y}; }

// ---------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------

// SCHED selects the K-loop schedule: 0 lock-step waves, 1 ping-pong (8 waves,
// two per SIMD), 3 one wave per SIMD (4 waves, 128x128 wave tiles, accumulators
// in AGPRs) with two deep stages (BK=64), the barrier before each stage's last
// k-step and each stage's DMA split over two k-steps, 6 the same tile with a
// whole stage of fragments in registers (described at its loop).  RED: the
// launch has reductions.  Only that instantiation carries the reductions' code
// (the row partials of interior tiles as an unmasked tree); without it, a
// staged output's block tail is the staging writes alone.  CH: the epilogue
// chain (FixedChain): kChainGeneric interprets the descriptor's ops; a fixed
// chain is the same arithmetic compiled as straight-line code (bitwise the
// same results), which at one wave per SIMD removes the op loop's per-op
// descriptor loads, dispatch and register copies from every column block.
template <int BM, int BN, int BK, int S, int WM, int WN, int SCHED, typename T, bool RED, int CH>
__global__ __launch_bounds__(WM* WN * 64) __attribute__((amdgpu_waves_per_eu(SCHED >= 3 ? 1 : 2)))
void gemm_epilogue_kernel(const fuseml_gemm_desc d_arg) {
  using G = StageGeom<BK>;
  constexpr int NW = WM * WN;  // waves per workgroup
  constexpr int NT = NW * 64;
  constexpr int TM = BM / WM;  // wave tile rows (m)
  constexpr int TN = BN / WN;  // wave tile cols (n)
  constexpr int NJ = TM / 32;  // 32x32 blocks along m (MFMA "B" operand)
  constexpr int NI = TN / 32;  // 32x32 blocks along n (MFMA "A" operand)
  constexpr int RB = G::kRowBytes;
  constexpr int A_BYTES = BM * RB;
  constexpr int STAGE = (BM + BN) * RB;
  constexpr int A_DMA = BM / (G::kRowsPerDma * NW);  // DMA instructions per wave per stage
  constexpr int B_DMA = BN / (G::kRowsPerDma * NW);
  constexpr int LPS = A_DMA + B_DMA;                 // vector-memory ops per thread per stage
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(A_DMA * G::kRowsPerDma * NW == BM && B_DMA * G::kRowsPerDma * NW == BN,
                "stage rows must split evenly over the waves");
  static_assert(S >= 2 && LPS * (S - 2) < 64, "pipeline depth");

  constexpr int AUXLEN = BM > BN ? BM : BN;  // floats per staged vector slot
  __shared__ __attribute__((aligned(1024))) char smem[S * STAGE + kAuxSlots * AUXLEN * 4];
  float* aux = reinterpret_cast<float*>(smem + S * STAGE);

  const KDesc& dk = *(const KDesc*)(__builtin_amdgcn_kernarg_segment_ptr());
  const int tiles_m = ((int)dk.M + BM - 1) / BM;
  const int tiles_n = ((int)dk.N + BN - 1) / BN;

  // Workgroup b runs tiles b, b + nwg, b + 2*nwg, ... (the 256-wide variants
  // launch at most one workgroup per CU, so a workgroup runs several tiles
  // back to back with no relaunch).  Round r is tiles [r*nwg, r*nwg + nwg).
  // XCD-aware order within a round: the hardware deals workgroups to the 8
  // XCDs round-robin (XCD = blockIdx % 8), so each XCD is given a contiguous
  // range of the round's logical tiles; consecutive logical tiles form
  // GROUP_M-row column strips, so the tiles an XCD runs at the same time share
  // A rows and B columns in its L2.
  const int nwg = gridDim.x;
  const int ntiles = tiles_m * tiles_n;
  for (int tile = blockIdx.x; tile < ntiles; tile += nwg) {
    const int round0 = tile - (int)blockIdx.x;
    const int in_round = min(nwg, ntiles - round0);
    int lid = tile;
    if ((in_round & 7) == 0) lid = round0 + ((int)blockIdx.x & 7) * (in_round >> 3) + ((int)blockIdx.x >> 3);
    // The previous tile's LDS reads are complete in every wave before this
    // tile's DMA overwrites the slots.  The waits run on every path into the
    // tile (on the first tile nothing is outstanding).  The generic op loop's
    // kernels of the one-wave schedules also wait for the previous tile's
    // global stores: without that wait, the compiler's wait insertion sees
    // them as possibly pending at this tile's K loop and puts an s_waitcnt
    // vmcnt(0) into the steady loop.  The other kernels leave the stores in
    // flight: their K loops' counted waits only get stricter for older
    // operations (vector-memory operations complete in issue order).
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkmcnt0();
    if constexpr (SCHED == 3 || (SCHED == 6 && CH == kChainGeneric)) wait_vmcnt<0>();
    __builtin_amdgcn_sched_barrier(0);
    if (tile != (int)blockIdx.x) {
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    }
    // The descriptor pointer and the thread index pass through empty asm each
    // tile, so nothing derived from them is hoisted out of the tile loop: held
    // across the K loop, the epilogue's address arithmetic would spill.
    const char* kargs = (const char*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(kargs));
    const KDesc& d = *(const KDesc*)kargs;
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN;
    const int wn = wave % WN;
    const int M = (int)d.M, N = (int)d.N, K = (int)d.K;
    const int strip = kGroupM * tiles_n;
    const int first_m = (lid / strip) * kGroupM;
    const int strip_h = min(tiles_m - first_m, kGroupM);
    const int pid_m = first_m + (lid % strip) % strip_h;
    const int pid_n = (lid % strip) / strip_h;
    const int m0 = pid_m * BM;
    const int n0 = pid_n * BN;

    // Operand buffer resources based at the tile's first row of A and of W, so
    // that only a tile's rows need 32-bit offsets (the host checks that span).
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc_at(d.a, (int64_t)m0 * d.lda * 2, ((int64_t)(M - 1) * d.lda + K) * 2);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc_at(d.b, (int64_t)n0 * d.ldb * 2, ((int64_t)(N - 1) * d.ldb + K) * 2);

    // Vector operands with an LDS slot (bias and the like): this thread's element
    // of each is loaded now, lands during the K loop, and is written to its slot
    // (as fp32) after it.  Every slot holds at most one element per thread.
    // Slot q's load goes straight into aux_bits[q] (q a compile-time index; the
    // operand holding the slot is found by a scalar search).  Loaded into a
    // temporary and moved to its slot's register by a runtime choice, the
    // move would wait for the load, i.e. for its full latency, right here.
    static_assert(AUXLEN <= NT, "one staged vector element per thread");
    uint32_t aux_bits[kAuxSlots];
    static_for<0, kAuxSlots>([&](auto q) {
      int oi = -1;
      for (int k = 0; k < d.n_operands; ++k) {
        const int fl = d.operands[k].reserved;
        if ((fl & kFlagAux) && ((fl >> 8) & (kAuxSlots - 1)) == q) {
          oi = k;
          break;
        }
      }
      if (oi < 0) {
        aux_bits[q] = 0;
        return;
      }
      const bool rowv = d.operands[oi].stride_m == 0;
      const int idx = (rowv ? n0 : m0) + tid;
      const bool ok = tid < (rowv ? BN : BM) && idx < (rowv ? N : M);
      const int64_t st = rowv ? d.operands[oi].stride_n : d.operands[oi].stride_m;
      const int eb = d.operands[oi].dtype == FUSEML_F32 ? 4 : 2;
      const __amdgpu_buffer_rsrc_t r = make_rsrc_at(d.operands[oi].ptr, (int64_t)(rowv ? n0 : m0) * st * eb,
                                                    d.operands[oi].extent * eb);
      const uint32_t off = ok ? (uint32_t)((int64_t)tid * st * eb) : kOOB;
      aux_bits[q] = (eb == 4) ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0)
                              : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
    });

    // The epilogue stages the first LDS-eligible 2-D operand of the chain in an
    // LDS tile [BM][BN] of 16-bit elements that reuses the pipeline's slots.
    int staged = -1;
    for (int o = 0; o < d.n_ops; ++o) {
      const int k = d.ops[o].kind;
      if ((k == FUSEML_OP_ADD || k == FUSEML_OP_MUL) && (d.operands[d.ops[o].operand].reserved & kFlagStage)) {
        staged = d.ops[o].operand;
        break;
      }
    }
    // With whole-chunk staging (BN >= 256) and a pipelined K loop the tile is
    // filled by the LDS DMA.  Pipeline slot s holds staging rows [s*RPS,
    // (s+1)*RPS), and a DMA of that slot's share of the operand goes to the
    // same LDS address as the stage DMA it replaces: once no further stage of K
    // is bound for a slot, the K loop's DMA issue points fetch the operand
    // instead (same count per wave, so the vmcnt bookkeeping is unchanged), and
    // the slot that holds the last stage is fetched after the loop.  Lane l of
    // a DMA writes physical chunk l % CPR of row l / CPR and fetches the logical
    // chunk that the staging swizzle places there.  A slot's DMAs go through a
    // buffer resource whose base is the slot's first operand row, so the lane
    // offsets do not depend on the slot.  Rows past M are not masked: they read
    // in-bounds operand data (the resource's range check) that no result uses.
    constexpr int SP = 2 * BN;        // staging row pitch in bytes
    constexpr int CPR = BN / 8;       // 16-byte chunks per staged row
    constexpr bool kOpDma = kChunkSwizzle<BN> && SCHED != 0;
    constexpr int RPD = 1024 / SP;    // staging rows one wave-wide DMA fills
    constexpr int RPS = STAGE / SP;   // staging rows per pipeline slot
    static_assert(!kOpDma || (STAGE % SP == 0 && RPS % 32 == 0 && RPS == RPD * NW * LPS),
                  "operand DMAs line up with the stage DMAs");
    const bool op_dma = kOpDma && staged >= 0;
    const void* op_ptr = d.a;
    int64_t op_bytes = 0;  // bytes of the operand from its row m0 on
    uint32_t op_o[kOpDma ? LPS : 1];  // chunk c's byte offset in its slot (kOOB: column past N)
    uint64_t op_row_bytes = 0;        // operand row pitch in bytes
    uint32_t op_osm = 0;
    if constexpr (kOpDma) {
      const int si = staged >= 0 ? staged : 0;
      const uint32_t osm = (uint32_t)d.operands[si].stride_m;
      op_osm = osm;
      op_row_bytes = (uint64_t)osm * 2u;
      // Based at the tile's first row: offsets cover the tile's rows only.
      op_ptr = static_cast<const char*>(d.operands[si].ptr) + (uint64_t)m0 * op_row_bytes;
      op_bytes = d.operands[si].extent * 2 - (int64_t)m0 * (int64_t)op_row_bytes;
      if constexpr (SCHED != 6) static_for<0, LPS>([&](auto c) {
        const int r = (wave + NW * c) * RPD + lane / CPR;
        const int n = n0 + 8 * ((lane % CPR) ^ (r & 31));
        op_o[c] = n < N ? ((uint32_t)r * osm + (uint32_t)n) * 2u : kOOB;
      });
    }
    // Base and byte extent of slot `slot`'s part of the operand.
    auto op_slot_ptr = [&](int slot) -> const void* {
      return static_cast<const char*>(op_ptr) + (uint64_t)(slot * RPS) * op_row_bytes;
    };
    auto op_slot_bytes = [&](int slot) -> uint32_t {
      const int64_t rest = op_bytes - (int64_t)(slot * RPS) * (int64_t)op_row_bytes;
      return rest <= 0 ? 0u : (rest >= 0x7fffffffLL ? 0x7fffffffu : (uint32_t)rest);
    };
    // Operand chunks [c0, c1) of slot `slot`.
    auto load_op_chunks = [&](int slot, auto c0, auto c1) {
      const __amdgpu_buffer_rsrc_t rop = make_rsrc(op_slot_ptr(slot), op_slot_bytes(slot));
      char* st = smem + slot * STAGE;
      static_for<decltype(c0)::value, decltype(c1)::value>([&](auto c) {
        uint32_t oo;
        if constexpr (SCHED == 6) {  // computed here: 16 fewer registers held across the K loop
          const int r = (wave + NW * c) * RPD + lane / CPR;
          const int n = n0 + 8 * ((lane % CPR) ^ (r & 31));
          oo = n < N ? ((uint32_t)r * op_osm + (uint32_t)n) * 2u : kOOB;
        } else {
          oo = op_o[c];
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rop, (__attribute__((address_space(3))) void*)(st + (wave + NW * c) * 1024), 16, oo, 0, 0, 0);
      });
    };

    // Global -> LDS DMA.  One wave-wide buffer_load_dwordx4 ... lds writes 64 x 16
    // bytes contiguously from the LDS base in M0, i.e. kRowsPerDma whole stage
    // rows.  The swizzle is applied on the source side: the lane whose 16-byte
    // slot is physical chunk c of row r fetches logical chunk c ^ swizzle(r).
    // Rows past M (or N) are clamped to the last valid row: they load real data
    // whose results are never stored and are excluded from every reduction.
    uint32_t a_off[A_DMA], b_off[B_DMA];
    int a_k[A_DMA], b_k[B_DMA];
    static_for<0, A_DMA>([&](auto i) {
      const int row = (wave + NW * i) * G::kRowsPerDma + lane / G::kChunks;
      const int kc = (lane % G::kChunks) ^ G::swizzle(row);
      const int gm = min(row, M - 1 - m0);
      a_off[i] = (uint32_t)((int64_t)gm * d.lda * 2) + (uint32_t)(kc * 16);
      a_k[i] = kc * 8;
    });
    static_for<0, B_DMA>([&](auto i) {
      const int row = (wave + NW * i) * G::kRowsPerDma + lane / G::kChunks;
      const int kc = (lane % G::kChunks) ^ G::swizzle(row);
      const int gn = min(row, N - 1 - n0);
      b_off[i] = (uint32_t)((int64_t)gn * d.ldb * 2) + (uint32_t)(kc * 16);
      b_k[i] = kc * 8;
    });
    // Stage `kt` of K into LDS slot `slot`.  A chunk whose k range starts at or
    // past K reads zeros (K is a multiple of 8, so a chunk is wholly inside or
    // wholly outside [0,K)).
    // Chunks [c0, c1) of stage kt, A chunks first (0 .. A_DMA-1), then W chunks.
    // Chunk c of either kind fills the 1 KB at (wave + NW*c) KB of the slot, as
    // does the operand's chunk c (load_op_chunks).
    static_assert(G::kRowsPerDma * RB == 1024 && A_BYTES == A_DMA * NW * 1024, "1 KB DMA blocks");
    const int nk = (K + BK - 1) / BK;
    auto load_chunks = [&](int kt, int slot, auto c0, auto c1) {
      const int k0 = kt * BK;
      const uint32_t kb = (uint32_t)(k0 * 2);
      char* st = smem + slot * STAGE;
      // The whole-stage schedule runs only for K % 64 == 0 (choose_config): a
      // stage is wholly inside or outside [0, K), so its k offset is one
      // uniform value, passed as the buffer instruction's scalar offset (no
      // per-lane arithmetic: 33 fewer VALU instructions per stage, ~1% on the
      // bench shapes).  A stage past K re-reads stage 0's k range (in bounds);
      // nothing consumes it.
      const uint32_t sk = (SCHED == 6 && kt < nk) ? kb : 0u;
      static_for<decltype(c0)::value, decltype(c1)::value>([&](auto c) {
        uint32_t off;
        __amdgpu_buffer_rsrc_t r;
        if constexpr (c < A_DMA) {
          if constexpr (SCHED == 6) off = a_off[c];
          else off = (k0 + a_k[c] < K) ? a_off[c] + kb : kOOB;
          r = ra;
        } else {
          constexpr int i = c - A_DMA;
          if constexpr (SCHED == 6) off = b_off[i];
          else off = (k0 + b_k[i] < K) ? b_off[i] + kb : kOOB;
          r = rb;
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            r, (__attribute__((address_space(3))) void*)(st + (wave + NW * c) * 1024), 16, off, sk, 0, 0);
      });
    };
    auto load_stage = [&](int kt, int slot) {
      const int k0 = kt * BK;
      const uint32_t kb = (uint32_t)(k0 * 2);
      char* st = smem + slot * STAGE;
      static_for<0, A_DMA>([&](auto i) {
        const uint32_t off = (k0 + a_k[i] < K) ? a_off[i] + kb : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (__attribute__((address_space(3))) void*)(st + (wave + NW * i) * G::kRowsPerDma * RB), 16,
            off, 0, 0, 0);
      });
      static_for<0, B_DMA>([&](auto i) {
        const uint32_t off = (k0 + b_k[i] < K) ? b_off[i] + kb : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rb, (__attribute__((address_space(3))) void*)(st + A_BYTES + (wave + NW * i) * G::kRowsPerDma * RB),
            16, off, 0, 0, 0);
      });
    };

    f32x16_t acc[NI][NJ];
    static_for<0, NI>([&](auto i) {
      static_for<0, NJ>([&](auto j) {
        static_for<0, 16>([&](auto r) { acc[i][j][(int)r] = 0.0f; });
      });
    });

    const int l32 = lane & 31;
    const int khalf = lane >> 5;
    const int swz = G::swizzle(l32);  // == swizzle(row) for every fragment row this lane reads
    // Fragment row byte offsets inside a stage: rows of W feed MFMA "A", rows of x MFMA "B".
    const int fa_row = A_BYTES + (wn * TN + l32) * RB;
    const int fb_row = (wm * TM + l32) * RB;

    // MFMAs of one stage.  Fragments of k-step ks+1 are read from LDS while the
    // MFMAs of k-step ks run.
    constexpr int KS = BK / 16;
    auto compute = [&](const char* st) {
      i32x4_t fa[2][NI], fb[2][NJ];
      auto read_frags = [&](int ks, int buf) {
        const int chunk = ((2 * ks + khalf) ^ swz) << 4;
        static_for<0, NI>([&](auto i) {
          fa[buf][i] = *reinterpret_cast<const i32x4_t*>(st + fa_row + 32 * i * RB + chunk);
        });
        static_for<0, NJ>([&](auto j) {
          fb[buf][j] = *reinterpret_cast<const i32x4_t*>(st + fb_row + 32 * j * RB + chunk);
        });
      };
      read_frags(0, 0);
      static_for<0, KS>([&](auto ks) {
        constexpr int cur = decltype(ks)::value & 1;
        if constexpr (decltype(ks)::value + 1 < KS) read_frags(decltype(ks)::value + 1, cur ^ 1);
        static_for<0, NI>([&](auto i) {
          static_for<0, NJ>([&](auto j) { acc[i][j] = mfma32<T>(fa[cur][i], fb[cur][j], acc[i][j]); });
        });
      });
    };

    // Workgroup barrier that keeps the compiler from moving any instruction
    // (MFMAs included) across it.  A bare s_barrier: __syncthreads() would add a
    // release fence that drains every in-flight DMA.
    auto barrier = [&]() {
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
    };
    if constexpr (SCHED == 6) {
      // One wave per SIMD, two stages of BK=64, a whole stage's fragments in
      // registers.  Stage k (slot k % 2):
      //   k-step 0: MFMAs while the fragments of k-steps 1-3 are read;
      //   barrier 1 (after this wave's reads): no wave reads slot k % 2 any more;
      //   k-steps 1-3: MFMAs while stage k+2's DMA goes into slot k % 2, spread
      //   over the three k-steps (barrier 2 in k-step 3: stage k+1 landed and
      //   visible); k-step 3 also reads stage k+1's k-step 0 fragments.
      // Each k-step then carries at most ~21 KB of DMA writes or 24 KB of reads
      // per wave-quad, instead of two k-steps carrying both.  Each barrier sits
      // two MFMAs into its k-step (those two need nothing it guards), so the
      // reads that barrier 1 waits for have two more MFMAs to land (C5 -0.6
      // and -1.3%).
      static_assert(S == 2 && KS == 4 && NI == 4 && NJ == 4 && LPS == 16, "one-wave whole-stage geometry");
      i32x4_t fr[KS][NI + NJ];
      auto rd = [&](const char* st, auto ks, auto f) {
        const int chunk = ((2 * ks + khalf) ^ swz) << 4;
        if constexpr (f < NI)
          fr[ks][f] = *reinterpret_cast<const i32x4_t*>(st + fa_row + 32 * f * RB + chunk);
        else
          fr[ks][f] = *reinterpret_cast<const i32x4_t*>(st + fb_row + 32 * (f - NI) * RB + chunk);
      };
      auto issue = [&](int kt, int slot, auto c0, auto c1, auto tail) {
        if constexpr (decltype(tail)::value) {
          if (op_dma && kt >= nk) {
            load_op_chunks(slot, c0, c1);
            return;
          }
        }
        load_chunks(kt, slot, c0, c1);
      };
      // k-step ks: MFMAs from fr[ks]; fragment reads [r0, r1) of stage `rst`
      // (read r: k-step r / 8, fragment r % 8) and DMA chunks [c0, c1) of stage
      // kt, each spread evenly over the 16 MFMAs.
      // MFMAs [q0, q1) of k-step ks, the reads and DMAs spread over them.
      auto kstep_q = [&](auto ks, const char* rst, auto r0, auto r1, int kt, int slot, auto c0, auto c1, auto tail,
                         auto q0, auto q1) {
        constexpr int n_rd = decltype(r1)::value - decltype(r0)::value;
        constexpr int n_dma = decltype(c1)::value - decltype(c0)::value;
        constexpr int Q0 = decltype(q0)::value, NQ = decltype(q1)::value - Q0;
        static_for<0, NQ>([&](auto qq) {
          constexpr int q = Q0 + qq;
          constexpr int i = q / NJ, j = q % NJ;
          acc[i][j] = mfma32<T>(fr[ks][i], fr[ks][NI + j], acc[i][j]);
          static_for<0, n_rd>([&](auto m) {
            if constexpr ((m * NQ) / n_rd == qq) {
              constexpr int r = decltype(r0)::value + m;
              rd(rst, std::integral_constant<int, r / 8>{}, std::integral_constant<int, r % 8>{});
            }
          });
          static_for<0, n_dma>([&](auto m) {
            if constexpr ((m * NQ) / n_dma == qq) {
              constexpr int c = decltype(c0)::value + m;
              issue(kt, slot, std::integral_constant<int, c>{}, std::integral_constant<int, c + 1>{}, tail);
            }
          });
          __builtin_amdgcn_sched_barrier(0);
        });
      };
      using QA = std::integral_constant<int, 0>;
      using QS = std::integral_constant<int, 2>;
      using QE = std::integral_constant<int, NI * NJ>;
      auto kstep = [&](auto ks, const char* rst, auto r0, auto r1, int kt, int slot, auto c0, auto c1, auto tail) {
        kstep_q(ks, rst, r0, r1, kt, slot, c0, c1, tail, QA{}, QE{});
      };
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using I3 = std::integral_constant<int, 3>;
      using R0 = std::integral_constant<int, 0>;
      using R8 = std::integral_constant<int, 8>;
      using R32 = std::integral_constant<int, 32>;
      using D6 = std::integral_constant<int, 6>;
      using D11 = std::integral_constant<int, 11>;
      using D16 = std::integral_constant<int, 16>;
      auto body = [&](int k, auto tail) {
        const char* st = smem + (k & 1) * STAGE;
        const char* nst = smem + ((k + 1) & 1) * STAGE;
        kstep(I0{}, st, R8{}, R32{}, k + 2, k & 1, R0{}, R0{}, tail);
        kstep_q(I1{}, st, R0{}, R0{}, k + 2, k & 1, R0{}, R0{}, tail, QA{}, QS{});
        wait_lgkmcnt0();
        barrier();  // slot k % 2 retired
        kstep_q(I1{}, st, R0{}, R0{}, k + 2, k & 1, R0{}, D6{}, tail, QS{}, QE{});
        kstep(I2{}, st, R0{}, R0{}, k + 2, k & 1, D6{}, D11{}, tail);
        kstep_q(I3{}, nst, R0{}, R0{}, k + 2, k & 1, D11{}, D11{}, tail, QA{}, QS{});
        wait_vmcnt<11>();  // stage k+1 (only stage k+2's first 11 chunks are younger)
        barrier();
        kstep_q(I3{}, nst, R0{}, R8{}, k + 2, k & 1, D11{}, D16{}, tail, QS{}, QE{});
      };
      using Tail = std::true_type;
      issue(0, 0, R0{}, D16{}, Tail{});
      issue(1, 1, R0{}, D16{}, Tail{});
      wait_vmcnt<16>();  // stage 0
      barrier();
      static_for<0, NI + NJ>([&](auto f) { rd(smem, I0{}, f); });
      const int steady = op_dma ? nk - 2 : nk;
      int k = 0;
      for (; k < steady; ++k) body(k, std::false_type{});
      for (; k < nk; ++k) body(k, Tail{});
    } else if constexpr (SCHED == 3) {
      // One wave per SIMD, two stages of BK=64 (four MFMA k-steps each).  Stage k:
      //   k-steps 0..2: MFMAs of k-step s while k-step s+1's fragments are read;
      //   under k-step 0 the second half of stage k+1's DMA is issued (into
      //   stage k-1's slot, retired at barrier k-1);
      //   then this wave's LDS reads are complete and its DMA of stage k+1 has
      //   landed (nothing younger is in flight), and the workgroup barrier:
      //   stage k+1 is visible, and no wave reads stage k's slot any more
      //   (k-step 3's fragments are in registers);
      //   k-step 3: MFMAs while the first half of stage k+2's DMA is issued
      //   into stage k's slot and stage k+1's k-step 0 fragments are read.
      // The stage's 64 KB of LDS writes are split over two k-steps: written in
      // one burst they collide with the fragment reads (measured: writing them
      // with ds_write instead of the DMA costs the same), and issued later they
      // have less time to land (measured: halves 2% faster than thirds over
      // k-steps 3, 0 and 1).  Past the last stage the DMA reads nothing (zero
      // fill of a retired slot) and the fragments read are unused, so the loop
      // body is straight-line code.
      static_assert(S == 2 && KS == 4, "two stages of four k-steps");
      constexpr int P1 = LPS / 2, P2 = LPS;
      using C0 = std::integral_constant<int, 0>;
      using C1 = std::integral_constant<int, P1>;
      using C2 = std::integral_constant<int, P2>;
      using C3 = std::integral_constant<int, LPS>;
      i32x4_t fa[2][NI], fb[2][NJ];
      auto read = [&](const char* st, int ks, auto buf) {
        const int chunk = ((2 * ks + khalf) ^ swz) << 4;
        static_for<0, NI>([&](auto i) {
          fa[buf][i] = *reinterpret_cast<const i32x4_t*>(st + fa_row + 32 * i * RB + chunk);
        });
        static_for<0, NJ>([&](auto j) {
          fb[buf][j] = *reinterpret_cast<const i32x4_t*>(st + fb_row + 32 * j * RB + chunk);
        });
      };
      using Z = std::integral_constant<int, 0>;
      using O = std::integral_constant<int, 1>;
      // Chunks [c0, c1) of stage kt into `slot`.  In the tail iterations (the
      // last two), a stage kt >= nk is replaced by the operand's chunks of that
      // slot when op_dma is set.  The steady-state body has no such branch.
      auto issue = [&](int kt, int slot, auto c0, auto c1, auto tail) {
        if constexpr (decltype(tail)::value) {
          if (op_dma && kt >= nk) {
            load_op_chunks(slot, c0, c1);
            return;
          }
        }
        load_chunks(kt, slot, c0, c1);
      };
      // One k-step in a fixed order: for each MFMA q (acc[q / NJ][q % NJ] from
      // fragment buffer `buf`), the next k-step's fragment q (A rows first, then
      // B rows; k-step `ks` of stage `rst`, into buffer `rb`) and the DMA of
      // chunk c0+q if below c1, each triple its own scheduling region.  The
      // scheduler's own order (with sched_group_barrier hints) bunches the reads
      // and DMAs at the start and end of a k-step; measured 1.2-1.5% slower on
      // bias+GELU and residual epilogues at K = 4096 and 16384.
      auto kstep = [&](auto buf, const char* rst, int ks, auto rb, int kt, int slot, auto c0, auto c1,
                       auto tail) {
        const int chunk = ((2 * ks + khalf) ^ swz) << 4;
        static_for<0, NI * NJ>([&](auto q) {
          constexpr int i = q / NJ, j = q % NJ;
          acc[i][j] = mfma32<T>(fa[buf][i], fb[buf][j], acc[i][j]);
          if constexpr (q < NI)
            fa[rb][q] = *reinterpret_cast<const i32x4_t*>(rst + fa_row + 32 * q * RB + chunk);
          else if constexpr (q < NI + NJ)
            fb[rb][q - NI] = *reinterpret_cast<const i32x4_t*>(rst + fb_row + 32 * (q - NI) * RB + chunk);
          constexpr int c = decltype(c0)::value + q;
          if constexpr (c < decltype(c1)::value)
            issue(kt, slot, std::integral_constant<int, c>{}, std::integral_constant<int, c + 1>{}, tail);
          __builtin_amdgcn_sched_barrier(0);
        });
      };
      auto body = [&](int k, auto tail) {
        const char* st = smem + (k & 1) * STAGE;
        char* nst = smem + ((k + 1) & 1) * STAGE;
        kstep(Z{}, st, 1, O{}, k + 1, (k + 1) & 1, C1{}, C2{}, tail);
        kstep(O{}, st, 2, Z{}, k + 1, (k + 1) & 1, C2{}, C3{}, tail);
        kstep(Z{}, st, 3, O{}, k + 1, (k + 1) & 1, C3{}, C3{}, tail);
        wait_lgkmcnt0();
        wait_vmcnt<0>();  // this wave's DMA of stage k+1 (stage k+2 is not issued yet)
        barrier();
        kstep(O{}, nst, 0, Z{}, k + 2, k & 1, C0{}, C1{}, tail);
      };
      using Tail = std::true_type;
      issue(0, 0, C0{}, C3{}, Tail{});
      issue(1, 1, C0{}, C1{}, Tail{});
      wait_vmcnt<P1>();  // stage 0 (stage 1's first half may stay in flight)
      barrier();
      read(smem, 0, Z{});
      const int steady = op_dma ? nk - 2 : nk;
      int k = 0;
      for (; k < steady; ++k) body(k, std::false_type{});
      for (; k < nk; ++k) body(k, Tail{});
      // The operand's remaining chunks: those of the slot that held the last
      // stage (virtual stage nk+1, whose first half the last iteration issued).
      if (op_dma) load_op_chunks((nk + 1) & 1, C1{}, C3{});
    } else if constexpr (SCHED == 1) {
      // Ping-pong: waves 0-3 and 4-7 (one of each per SIMD) alternate between a
      // memory phase (wait for the stage's DMA, read all its fragments into
      // registers, issue the DMA S-1 stages ahead) and a compute phase (the
      // stage's MFMAs), one group a phase behind the other, so one group's LDS
      // traffic runs under the other group's MFMAs.  Every wave runs 2*nk+1
      // phases, each closed by a barrier.  Before each barrier a wave waits for
      // its own DMAs of the stage the next memory phase reads; a memory phase
      // also waits for its LDS reads, so the slot can be overwritten afterwards.
      static_assert(NW == 8 && KS == 2, "ping-pong pairs two groups of four waves");
      const int grp = wave >> 2;
      i32x4_t fr_a[KS][NI], fr_b[KS][NJ];
      using CL = std::integral_constant<int, LPS>;
      using C0 = std::integral_constant<int, 0>;
      // Slot p of a stage p >= nk, or of stage k+S-1 >= nk in memory phase k,
      // takes its share of the operand (slot nk+S-1 (mod S) after the loop).
      static_for<0, S - 1>([&](auto p) {
        if (p < nk)
          load_stage(p, p);
        else if (op_dma)
          load_op_chunks(p, C0{}, CL{});
      });
      int issued = op_dma ? S - 1 : min(nk, S - 1);  // stages (real or operand) issued
      // Memory phase k.  `steady`: stage k+S-1 exists (k + S - 1 < nk), so the
      // DMA needs no branch.
      auto mem = [&](int k, auto steady) {
        const char* st = smem + (k % S) * STAGE;
        static_for<0, KS>([&](auto ks) {
          const int chunk = ((2 * ks + khalf) ^ swz) << 4;
          static_for<0, NI>([&](auto i) {
            fr_a[ks][i] = *reinterpret_cast<const i32x4_t*>(st + fa_row + 32 * i * RB + chunk);
          });
          static_for<0, NJ>([&](auto j) {
            fr_b[ks][j] = *reinterpret_cast<const i32x4_t*>(st + fb_row + 32 * j * RB + chunk);
          });
        });
        if constexpr (decltype(steady)::value) {
          load_stage(k + S - 1, (k + S - 1) % S);
          issued = k + S;
        } else {
          if (k + S - 1 < nk)
            load_stage(k + S - 1, (k + S - 1) % S);
          else if (op_dma)
            load_op_chunks((k + S - 1) % S, C0{}, CL{});
          issued = op_dma ? k + S : min(nk, k + S);
        }
        wait_lgkmcnt0();
      };
      auto comp = [&]() {
        static_for<0, KS>([&](auto ks) {
          static_for<0, NI>([&](auto i) {
            static_for<0, NJ>([&](auto j) { acc[i][j] = mfma32<T>(fr_a[ks][i], fr_b[ks][j], acc[i][j]); });
          });
        });
      };
      // End of a phase: this wave's DMAs of stage `need` (read by the next
      // memory phase) have landed, then the workgroup barrier.
      auto phase_barrier = [&]() {
        // sched_barrier(0) keeps the scheduler from moving any instruction
        // (MFMAs included) across the phase boundary.
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
      };
      auto end_phase = [&](int need) {
        if (need < nk) {
          const int allowed = min(max(issued - need - 1, 0), S - 1);
          static_for<0, S>([&](auto a) {
            if (allowed == a) wait_vmcnt<LPS * a>();
          });
        }
        phase_barrier();
      };
      // The same at a point where `allowed` is known at compile time (in the
      // steady state the runtime choice above is a chain of branches per phase).
      auto end_phase_c = [&](auto allowed) {
        __builtin_amdgcn_sched_barrier(0);  // the wait stays behind the phase's work
        wait_vmcnt<LPS * decltype(allowed)::value>();
        phase_barrier();
      };
      // Memory phases 0 .. steady-1 issue a real stage; the rest run the
      // general code.  In the steady state a memory phase k leaves the stages
      // k+1 .. k+S-1 in flight after stage k: S-1 stages younger than the one
      // group 0 needs next (stage k), S-2 younger than stage k+1.
      const int steady = max(nk - (S - 1), 0);
      using A1 = std::integral_constant<int, S - 1>;
      using A2 = std::integral_constant<int, S - 2>;
      end_phase(0);    // stage 0 has landed before the first memory phase reads it
      if (grp == 0) {  // phases 2k: mem(k), 2k+1: comp(k), 2nk: idle
        int k = 0;
        for (; k < steady; ++k) {
          mem(k, std::true_type{});
          end_phase_c(A1{});
          comp();
          end_phase_c(A2{});
        }
        for (; k < nk; ++k) {
          mem(k, std::false_type{});
          end_phase(k);
          comp();
          end_phase(k + 1);
        }
        end_phase(nk);
      } else {  // phase 0: idle, 2k+1: mem(k), 2k+2: comp(k)
        end_phase(0);
        int k = 0;
        for (; k < steady; ++k) {
          mem(k, std::true_type{});
          end_phase_c(A2{});
          comp();
          end_phase_c(A2{});
        }
        for (; k < nk; ++k) {
          mem(k, std::false_type{});
          end_phase(k + 1);
          comp();
          end_phase(k + 1);
        }
      }
      if (op_dma) load_op_chunks((nk + S - 1) % S, C0{}, CL{});
    } else {
      // S-stage pipeline: stages kt+1 .. kt+S-2 stay in flight while stage kt is
      // consumed; one barrier per stage both publishes the DMA of stage kt (after
      // each wave's own vmcnt wait) and retires the slot the next DMA overwrites.
      static_for<0, S - 1>([&](auto p) {
        if (p < nk) load_stage(p, p);
      });
      // A bare s_barrier: __syncthreads() would add a release fence that drains
      // every in-flight DMA.  The asm statements only stop the compiler from
      // moving memory accesses across the barrier.
      auto stage_barrier = [&]() {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      };
      int slot = 0;
      auto next_slot = [&]() {
        int nslot = slot + S - 1;
        return nslot >= S ? nslot - S : nslot;
      };
      // While stage kt+S-1 exists, S-2 stages are in flight after kt and the
      // refill needs no branch; the last S-1 stages run the general code.
      const int steady = max(nk - (S - 1), 0);
      int kt = 0;
      for (; kt < steady; ++kt) {
        wait_vmcnt<LPS * (S - 2)>();
        stage_barrier();
        load_stage(kt + S - 1, next_slot());
        compute(smem + slot * STAGE);
        if (++slot == S) slot = 0;
      }
      for (; kt < nk; ++kt) {
        const int ahead = min(nk - 1 - kt, S - 2);  // stages issued after kt
        static_for<0, S - 1>([&](auto q) {
          if (ahead == q) wait_vmcnt<LPS * q>();
        });
        stage_barrier();
        if (kt + S - 1 < nk) load_stage(kt + S - 1, next_slot());
        compute(smem + slot * STAGE);
        if (++slot == S) slot = 0;
      }
    }
    for (int oi = 0; oi < d.n_operands; ++oi) {
      const int fl = d.operands[oi].reserved;
      if (!(fl & kFlagAux) || tid >= (d.operands[oi].stride_m == 0 ? BN : BM)) continue;
      const int slot = (fl >> 8) & (kAuxSlots - 1);
      const int dt = d.operands[oi].dtype;
      static_for<0, kAuxSlots>([&](auto q) {
        if (slot == q) aux[q * AUXLEN + tid] = elem_to_f32(aux_bits[q], dt);
      });
    }
    if (op_dma) wait_vmcnt<0>();  // this wave's operand DMAs have landed
    __syncthreads();  // the epilogue reuses the stage LDS; vector slots (and DMA-staged operand) written

    // ---------------------------------------------------------------------
    // Epilogue.  In accumulator block (i,j), register r of this lane holds
    //   m = m0 + wm*TM + 32j + (lane & 31)
    //   n = n0 + wn*TN + 32i + 8*(r>>2) + 4*(lane>>5) + (r&3).
    // That layout spreads each load/store instruction over 32 rows, so 2-D
    // operands and the output go through an LDS staging tile [BM][BN] of 16-bit
    // elements, filled and drained by whole-row coalesced 16-byte accesses.
    // ---------------------------------------------------------------------
    constexpr int RPP = NT / CPR;     // staged rows per cooperative pass
    static_assert(BM % RPP == 0 && BN % 128 == 0, "staging passes");
    static_assert(BM * SP <= S * STAGE, "staging tile fits in the pipeline's LDS");
    char* stg = smem;

    const int mw = m0 + wm * TM + l32;
    const int nw = n0 + wn * TN + 4 * khalf;
    const bool row_red = d.reduce_mask != 0 && d.reduce_axis == 1;
    const bool col_red = d.reduce_mask != 0 && d.reduce_axis == 0;
    const bool interior = m0 + BM <= M && n0 + BN <= N;  // every element of the tile in range
    const int crow = tid / CPR;  // cooperative-pass row and chunk of this thread
    const int cchk = tid % CPR;

    // (1) The staged operand, unless the DMA fetched it during the K loop: all
    // its global loads in flight together, one barrier.  The vector operands
    // were written to their slots before the barrier above.
    if (staged >= 0 && !op_dma) {
      const void* optr = d.operands[staged].ptr;
      const int64_t osm = d.operands[staged].stride_m;
      const __amdgpu_buffer_rsrc_t r = make_rsrc_at(optr, (int64_t)m0 * osm * 2, d.operands[staged].extent * 2);
      // Batches of 8 passes: the loads of a batch are all in flight before the
      // first LDS write.  Offsets in 32-bit arithmetic (exact for every in-range
      // element: the host bounds the operand's span below 2 GiB) and selected,
      // not branched on, so nothing serializes the loads.
      constexpr int NP = BM / RPP;
      constexpr int PB = NP < 8 ? NP : 8;
      static_assert(NP % PB == 0, "pass batches");
      static_for<0, NP / PB>([&](auto b) {
        i32x4_t x[PB];
        static_for<0, PB>([&](auto q) {
          const int rl = (b * PB + q) * RPP + crow;
          const int m = m0 + rl, n = n0 + 8 * cchk;
          const uint32_t o32 = ((uint32_t)rl * (uint32_t)osm + (uint32_t)n) * 2u;
          x[q] = __builtin_amdgcn_raw_buffer_load_b128(r, (m < M && n < N) ? o32 : kOOB, 0, 0);
        });
        static_for<0, PB>([&](auto q) {
          const int rl = (b * PB + q) * RPP + crow;
          *reinterpret_cast<i32x4_t*>(stg + stage_chunk<BN>(rl, cchk)) = stage_swapped<BN>(rl) ? swap_halves(x[q]) : x[q];
        });
      });
    }
    if (staged >= 0 && !op_dma) __syncthreads();

    // (2) The op chain, one column block at a time: for column block i, each op
    // runs over the NJ row blocks (NJ*16 independent elements) before the next
    // op, so each op's descriptor is read NI times rather than NI*NJ, and a row
    // vector's values (which depend only on the column) are read from LDS once
    // per column block.  Carrying one column block (not all of them) through the
    // runtime op loop keeps the loop's live values within the register file.
    const bool use_stage_out = d.out.ptr != nullptr && (d.out.reserved & kFlagStage) && !col_red;
    // Activations run a step at a time across EW values (independent VALU
    // chains).  16 instead of 8 for the one-wave schedule measured no faster.
    constexpr int EW = 8;
    const bool out_bf16 = d.out.dtype == FUSEML_BF16;
    float rs[NJ], rmx[NJ];  // row partials (sum, max) of this lane's rows
    static_for<0, NJ>([&](auto j) {
      rs[j] = 0.0f;
      rmx[j] = -INFINITY;
    });
    float* red_sum = reinterpret_cast<float*>(smem);
    float* red_max = red_sum + (d.reduce_axis == 1 ? WN * BM : WM * BN);
    // Fixed chains: the operands' LDS slots and the ADD alphas, read once per
    // tile (the host matched the op kinds and operand kinds to CH).  Op 0 is
    // the row-vector ADD of every chain that has one; the act-heavy chain's
    // second row vector is op 4, and the tile ADD of bias + tile is op 1.
    constexpr bool kFxRow0 = CH == kChainBias || CH == kChainBiasGeluErf || CH == kChainBiasGeluTanh ||
                             CH == kChainBiasRelu || CH == kChainBiasTile || CH == kChainActHeavy;
    int fx_slot0 = 0, fx_slot1 = 0;
    float fx_a0 = 1.0f, fx_a1 = 1.0f;
    if constexpr (kFxRow0) {
      fx_slot0 = (d.operands[d.ops[0].operand].reserved >> 8) & (kAuxSlots - 1);
      fx_a0 = d.ops[0].scalar;
    }
    if constexpr (CH == kChainBiasTile) fx_a1 = d.ops[1].scalar;
    if constexpr (CH == kChainActHeavy) {
      fx_slot1 = (d.operands[d.ops[4].operand].reserved >> 8) & (kAuxSlots - 1);
      fx_a1 = d.ops[4].scalar;
    }
    // A fixed chain over one column block (NJ row blocks x 16 values).  Every
    // op is the generic loop's arithmetic on the same values in the same order;
    // activations step across 16 independent values instead of 8.
    auto fixed_ops = [&](f32x16_t(&A)[NJ], const int i) {
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int l32 = ln & 31;
      const int khalf = ln >> 5;
      const int cb = wn * TN + 32 * i + 4 * khalf;  // this lane's first column of block i in the tile
      auto add_row = [&](int slot, float a) {
        const float* av = aux + slot * AUXLEN + cb;
        float x[16];
        static_for<0, 4>([&](auto g) {
          const float4 q = *reinterpret_cast<const float4*>(av + 8 * g);
          x[4 * g + 0] = q.x;
          x[4 * g + 1] = q.y;
          x[4 * g + 2] = q.z;
          x[4 * g + 3] = q.w;
        });
        static_for<0, NJ>([&](auto j) {
          static_for<0, 16>([&](auto r) { A[j][(int)r] = fmaf(a, x[r], A[j][(int)r]); });
        });
      };
      // The staged bf16 tile's values of this block, all row blocks' 8-byte
      // units read before any is used (32 registers).
      auto read_tile = [&](uint2(&wb)[NJ][4]) {
        const int u0 = (wn * TN + 32 * i) / 4 + khalf;
        static_for<0, NJ>([&](auto j) {
          const int r_loc = wm * TM + 32 * j + l32;
          static_for<0, 4>([&](auto g) {
            wb[j][g] = *reinterpret_cast<const uint2*>(stg + stage_unit<BN>(r_loc, u0 + 2 * g));
          });
        });
      };
      auto tile_value = [&](const uint2(&wb)[NJ][4], auto j, auto r) {
        const uint32_t w = (r & 2) ? wb[j][r / 4].y : wb[j][r / 4].x;
        return (r & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
      };
      auto relu_all = [&]() {
        static_for<0, NJ>([&](auto j) {
          static_for<0, 16>([&](auto r) { A[j][(int)r] = max_nan(A[j][(int)r], 0.0f); });
        });
      };
      auto activation = [&](auto fn) {
        static_for<0, NJ>([&](auto j) {
          float v[16];
          static_for<0, 16>([&](auto r) { v[r] = A[j][(int)r]; });
          fn(v);
          static_for<0, 16>([&](auto r) { A[j][(int)r] = v[r]; });
        });
      };
      if constexpr (kFxRow0) add_row(fx_slot0, fx_a0);
      if constexpr (CH == kChainBiasGeluErf) activation([](float* v) { gelu_erf_n<16>(v); });
      if constexpr (CH == kChainBiasGeluTanh) activation([](float* v) { gelu_tanh_n<16>(v); });
      if constexpr (CH == kChainBiasRelu || CH == kChainRelu || CH == kChainActHeavy) relu_all();
      if constexpr (CH == kChainBiasTile || CH == kChainActHeavy) {
        uint2 wb[NJ][4];
        read_tile(wb);
        static_for<0, NJ>([&](auto j) {
          static_for<0, 16>([&](auto r) {
            const float x = tile_value(wb, j, r);
            if constexpr (CH == kChainBiasTile)
              A[j][(int)r] = fmaf(fx_a1, x, A[j][(int)r]);
            else
              A[j][(int)r] = A[j][(int)r] * x;
          });
        });
      }
      if constexpr (CH == kChainActHeavy) {
        activation([](float* v) { sigmoid_n<16>(v); });
        add_row(fx_slot1, fx_a1);
      }
    };
    // One column block: its NJ accumulator blocks A[j] through the op chain, then
    // its stores, staged-output writes and reduction partials.
    auto column_block = [&](f32x16_t(&A)[NJ], const int i) {
      if constexpr (CH != kChainGeneric) fixed_ops(A, i);
      if constexpr (CH == kChainGeneric) for (int o = 0; o < d.n_ops; ++o) {
        // Lane coordinates through an opaque copy: the per-block addresses derived
        // from them are recomputed inside each op instead of being hoisted out of
        // the loop and held.
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int l32 = ln & 31;
        const int khalf = ln >> 5;
        const int mw = m0 + wm * TM + l32;
        const int nb = n0 + wn * TN + 32 * i + 4 * khalf;  // first column of block i
        const int kind = d.ops[o].kind;
        const float sc = d.ops[o].scalar;
        const int oi = d.ops[o].operand;
        if (kind == FUSEML_OP_ADD || kind == FUSEML_OP_MUL) {
          const int fl = d.operands[oi].reserved;
          const bool is_add = kind == FUSEML_OP_ADD;
          // v <- v + sc*x (ADD) or v * x (MUL), over one block's 16 elements.
          auto combine = [&](f32x16_t& v, const float* x) {
            if (is_add) {
              static_for<0, 16>([&](auto r) { v[(int)r] = fmaf(sc, x[r], v[(int)r]); });
            } else {
              static_for<0, 16>([&](auto r) { v[(int)r] = v[(int)r] * x[r]; });
            }
          };
          if (fl & kFlagAux) {
            const float* av = aux + ((fl >> 8) & (kAuxSlots - 1)) * AUXLEN;
            if (d.operands[oi].stride_m == 0) {  // row vector: four runs of 4 columns
              float x[16];
              static_for<0, 4>([&](auto g) {
                const float4 q = *reinterpret_cast<const float4*>(av + (nb - n0) + 8 * g);
                x[4 * g + 0] = q.x;
                x[4 * g + 1] = q.y;
                x[4 * g + 2] = q.z;
                x[4 * g + 3] = q.w;
              });
              static_for<0, NJ>([&](auto j) { combine(A[j], x); });
            } else {  // column vector: one value per row
              static_for<0, NJ>([&](auto j) {
                const float q = av[wm * TM + 32 * j + l32];
                float x[16];
                static_for<0, 16>([&](auto r) { x[r] = q; });
                combine(A[j], x);
              });
            }
          } else if (oi == staged) {
            // One uniform branch on the dtype (a staged operand is bf16 or fp16)
            // around straight-line blocks: a per-element choice of conversion
            // compiles to a branch tree per element (measured: C3's chain 10%
            // of the kernel's time).  Register r of a block is half r % 2 of
            // word (r / 2) % 2 of 8-byte unit u0 + 2 * (r / 4).
            const int u0 = (wn * TN + 32 * i) / 4 + khalf;
            auto read_block = [&](auto j, uint2(&wb)[4]) {
              const int r_loc = wm * TM + 32 * j + l32;
              static_for<0, 4>([&](auto g) {
                wb[g] = *reinterpret_cast<const uint2*>(stg + stage_unit<BN>(r_loc, u0 + 2 * g));
              });
            };
            auto run = [&](auto cvt) {
              static_for<0, NJ>([&](auto j) {
                uint2 wb[4];
                read_block(j, wb);
                float x[16];
                static_for<0, 4>([&](auto g) {
                  const uint2 q = wb[g];
                  x[4 * g + 0] = cvt(q.x & 0xffffu);
                  x[4 * g + 1] = cvt(q.x >> 16);
                  x[4 * g + 2] = cvt(q.y & 0xffffu);
                  x[4 * g + 3] = cvt(q.y >> 16);
                });
                combine(A[j], x);
              });
            };
            if (d.operands[oi].dtype == FUSEML_BF16)
              run([](uint32_t h) { return bf16_bits_to_f32(h); });
            else
              run([](uint32_t h) { return f16_bits_to_f32(h); });
          } else {
            static_for<0, NJ>([&](auto j) {
              const int m = mw + 32 * j;
              float x[16];
              static_for<0, 4>([&](auto g) {
                const int n = nb + 8 * g;
                load_operand4(d.operands[oi], m0, n0, m, n, m < M && n < N, x + 4 * g);
              });
              combine(A[j], x);
            });
          }
          continue;
        }
        switch (kind) {
          case FUSEML_OP_STORE:
            static_for<0, NJ>([&](auto j) {
              static_for<0, 4>([&](auto g) {
                const float x[4] = {A[j][4 * g], A[j][4 * g + 1], A[j][4 * g + 2],
                                    A[j][4 * g + 3]};
                store_out4(d.extra[oi], mw + 32 * j, nb + 8 * g, M, N, x);
              });
            });
            break;
#define FUSEML_EACH(expr)                                \
  static_for<0, NJ>([&](auto j) {                        \
    static_for<0, 16>([&](auto r) {                      \
      const float v = A[j][(int)r];                 \
      A[j][(int)r] = (expr);                        \
    });                                                  \
  })
          case FUSEML_OP_RELU:  // one v_maximum3_f32; NaN passes through, as in torch.relu
            FUSEML_EACH(max_nan(v, 0.0f));
            break;
#define FUSEML_EACH_N(fn)                                \
  static_for<0, NJ>([&](auto j) {                        \
    static_for<0, 16 / EW>([&](auto h) {                 \
      float xw[EW];                                      \
      static_for<0, EW>([&](auto e) { xw[e] = A[j][EW * h + e]; }); \
      fn<EW>(xw);                                        \
      static_for<0, EW>([&](auto e) { A[j][EW * h + e] = xw[e]; }); \
    });                                                  \
  })
          case FUSEML_OP_GELU_ERF:
            FUSEML_EACH_N(gelu_erf_n);
            break;
          case FUSEML_OP_GELU_TANH:
            FUSEML_EACH_N(gelu_tanh_n);
            break;
          case FUSEML_OP_SIGMOID:
            FUSEML_EACH_N(sigmoid_n);
            break;
#undef FUSEML_EACH_N
          case FUSEML_OP_SCALE:
            FUSEML_EACH(v * sc);
            break;
          case FUSEML_OP_ADD_SCALAR:
            FUSEML_EACH(v + sc);
            break;
          case FUSEML_OP_ADD_SELF:
            FUSEML_EACH(fmaf(sc, v, v));
            break;
          case FUSEML_OP_MUL_SELF:
            FUSEML_EACH(v * v);
            break;
#undef FUSEML_EACH
          default:
            break;
        }
      }

      // The column block's final values: unstaged stores, reduction partials and
      // the staged output, before the next column block, so that its NJ*16
      // values stay in registers from the first op to the LDS write.  The staged
      // output overwrites the staged operand in place: each 8-byte unit is read
      // (above) and written (here) by the same lane.
      float cs[16], cmx[16];
      static_for<0, 16>([&](auto r) {
        cs[r] = 0.0f;
        cmx[r] = -INFINITY;
      });
      // Coordinates from an opaque lane copy, as in the op loop: derived from
      // the tile-wide ones, their 64-bit forms are hoisted and held (spilled).
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int l32 = ln & 31;
      const int khalf = ln >> 5;
      const int mw = m0 + wm * TM + l32;
      const int nw = n0 + wn * TN + 4 * khalf;
      // The block's NJ row blocks into the staged output under one dtype
      // branch (or stored unstaged), then the reduction partials, each kind for
      // all row blocks at once: branches per row block would keep the row
      // blocks' independent work in separate basic blocks, which at one wave
      // per SIMD leaves every dependent step's latency exposed.
      if (use_stage_out) {
        const int u0 = (wn * TN + 32 * i) / 4 + khalf;
        if (out_bf16) {
          static_for<0, NJ>([&](auto j) {
            const int r_loc = wm * TM + 32 * j + l32;
            static_for<0, 4>([&](auto g) {
              const f32x16_t& v = A[j];
              *reinterpret_cast<uint2*>(stg + stage_unit<BN>(r_loc, u0 + 2 * g)) =
                  make_uint2(pack_bf16x2(v[4 * g], v[4 * g + 1]), pack_bf16x2(v[4 * g + 2], v[4 * g + 3]));
            });
          });
          asm volatile("; staged output block, bf16");
        } else {
          static_for<0, NJ>([&](auto j) {
            const int r_loc = wm * TM + 32 * j + l32;
            static_for<0, 4>([&](auto g) {
              const f32x16_t& v = A[j];
              *reinterpret_cast<uint2*>(stg + stage_unit<BN>(r_loc, u0 + 2 * g)) =
                  make_uint2(pack_f16x2(v[4 * g], v[4 * g + 1]), pack_f16x2(v[4 * g + 2], v[4 * g + 3]));
            });
          });
          asm volatile("; staged output block, fp16");
        }
      } else if (d.out.ptr != nullptr) {
        static_for<0, NJ>([&](auto j) {
          const int m = mw + 32 * j;
          const int nb = nw + 32 * i;
          static_for<0, 4>([&](auto g) {
            const float x[4] = {A[j][4 * g], A[j][4 * g + 1], A[j][4 * g + 2], A[j][4 * g + 3]};
            store_out4(d.out, m, nb + 8 * g, M, N, x);
          });
        });
      }
      // Partial reductions exclude every element outside [0,M) x [0,N) (the
      // reference lets padded tile elements through, kernel_generator.py:1959-1960,
      // 1983-1984).  Row partials of an interior tile need no masks: each row
      // block's 16 values of the row are summed (and maxed) as a pairwise tree,
      // four dependent steps instead of a 16-long chain.
      if constexpr (RED) {
        if (row_red && interior) {
          static_for<0, NJ>([&](auto j) {
            float s8[8], m8[8];
            static_for<0, 8>([&](auto e) {
              s8[e] = A[j][2 * e] + A[j][2 * e + 1];
              m8[e] = max_nan(A[j][2 * e], A[j][2 * e + 1]);
            });
            static_for<0, 4>([&](auto e) {
              s8[e] = s8[2 * e] + s8[2 * e + 1];
              m8[e] = max_nan(m8[2 * e], m8[2 * e + 1]);
            });
            static_for<0, 2>([&](auto e) {
              s8[e] = s8[2 * e] + s8[2 * e + 1];
              m8[e] = max_nan(m8[2 * e], m8[2 * e + 1]);
            });
            rs[j] += s8[0] + s8[1];
            rmx[j] = max_nan(rmx[j], max_nan(m8[0], m8[1]));
          });
        } else if (row_red || col_red) {
          static_for<0, NJ>([&](auto j) {
            const int m = mw + 32 * j;
            const int nb = nw + 32 * i;
            static_for<0, 16>([&](auto r) {
              const int n = nb + 8 * (r >> 2) + (r & 3);
              const bool in = (m < M) && (n < N);
              const float x = A[j][(int)r];
              if (row_red && in) {
                rs[j] += x;
                rmx[j] = max_nan(rmx[j], x);
              }
              if (col_red && in) {
                cs[r] += x;
                cmx[r] = max_nan(cmx[r], x);
              }
            });
          });
        }
      }
      if (RED && col_red) {
        // Column partials: reduce over the 32 rows held by each half-wave.  Column
        // reductions use neither a staged output nor a staged operand (the host
        // does not flag them), so the staging tile's LDS is free here.
        static_for<0, 16>([&](auto r) {
  #pragma unroll
          for (int sh = 1; sh < 32; sh <<= 1) {
            cs[r] += __shfl_xor(cs[r], sh);
            cmx[r] = max_nan(cmx[r], __shfl_xor(cmx[r], sh));
          }
          if (l32 == 0) {
            const int col = wn * TN + 32 * i + 8 * (r >> 2) + 4 * khalf + (r & 3);
            red_sum[wm * BN + col] = cs[r];
            red_max[wm * BN + col] = cmx[r];
          }
        });
      }
    };
    if constexpr (SCHED >= 3) {
      // A runtime loop over the column blocks, so that the op code exists once
      // (not NI times: at NI = 4 the copies cost instruction-cache misses on
      // every tile).  Each block is copied out of the AGPRs by a uniform branch
      // (the asm markers keep the four copies from being merged into selects)
      // and enters the op loop in VGPRs: a value carried around the op loop in
      // an AGPR would be copied out and back on every op.
#pragma clang loop unroll(disable)
      for (int i = 0; i < NI; ++i) {
        f32x16_t A[NJ];
        // An if/else chain, so that every path defines A: with four
        // independent ifs the compiler carries an undefined path's registers
        // around the loop (32 64-bit copies per column block).
        static_assert(NI == 4, "four column blocks");
        auto pick = [&](auto ii) {
          static_for<0, NJ>([&](auto j) { A[j] = acc[ii][j]; });
          asm volatile("; column block %0" ::"n"((int)ii));
        };
        if (i == 0)
          pick(std::integral_constant<int, 0>{});
        else if (i == 1)
          pick(std::integral_constant<int, 1>{});
        else if (i == 2)
          pick(std::integral_constant<int, 2>{});
        else
          pick(std::integral_constant<int, 3>{});
        static_for<0, NJ>([&](auto j) {
          static_for<0, 16>([&](auto r) {
            float x = A[j][(int)r];
            asm volatile("" : "+v"(x));
            A[j][(int)r] = x;
          });
        });
        column_block(A, i);
      }
    } else {
      // Also one copy of the op code: block i is processed in acc[0] and the
      // later blocks are shifted down after it (acc lives in VGPRs here; copying
      // a block out instead, as above, needs more registers than two waves per
      // SIMD have).
#pragma clang loop unroll(disable)
      for (int i = 0; i < NI; ++i) {
        column_block(acc[0], i);
        static_for<0, NI - 1>([&](auto q) {
          static_for<0, NJ>([&](auto j) { acc[q][j] = acc[q + 1][j]; });
        });
      }
    }

    // (3) Staged output: the LDS tile (written above), drained by whole-row
    // 16-byte stores.
    if (use_stage_out) {
      __syncthreads();
      // 16 passes unrolled: their LDS reads are in flight together (measured 2%
      // faster than 4 at 16384x4096x1024 with no ops; the kernel's code is small
      // enough since the column blocks share one copy of the op code).
#pragma unroll 16
      for (int p = 0; p < BM / RPP; ++p) {
        const int rl = p * RPP + crow;
        const int m = m0 + rl, n = n0 + 8 * cchk;
        i32x4_t x = *reinterpret_cast<const i32x4_t*>(stg + stage_chunk<BN>(rl, cchk));
        if (stage_swapped<BN>(rl)) x = swap_halves(x);
        if (m < M && n < N) {
          uint16_t* dst = reinterpret_cast<uint16_t*>(d.out.ptr) + (int64_t)m * d.out.ld + n;
          *reinterpret_cast<i32x4_t*>(dst) = x;
        }
      }
    }

    if (!RED || d.reduce_mask == 0) continue;
    if (row_red) {
      // The partials overwrite the staging tile, which other waves may still be
      // draining (staged output) or reading (staged operand).
      if (use_stage_out || staged >= 0) lds_barrier();
      // Row partials: the other half-wave holds the other 4-column runs of the same rows.
      static_for<0, NJ>([&](auto j) {
        const float s2 = rs[j] + __shfl_xor(rs[j], 32);
        const float m2 = max_nan(rmx[j], __shfl_xor(rmx[j], 32));
        if (lane < 32) {
          const int row = wm * TM + 32 * j + lane;
          red_sum[wn * BM + row] = s2;
          red_max[wn * BM + row] = m2;
        }
      });
    }
    lds_barrier();

    const int len = row_red ? BM : BN;
    const int nparts = row_red ? WN : WM;
    const int base = row_red ? m0 : n0;
    const int lim = row_red ? M : N;
    const float inv = 1.0f / (float)(row_red ? N : M);
    for (int t = tid; t < len; t += NT) {
      const int idx = base + t;
      if (idx >= lim) continue;
      float s = 0.0f, mx = -INFINITY;
      for (int w = 0; w < nparts; ++w) {
        s += red_sum[w * len + t];
        mx = max_nan(mx, red_max[w * len + t]);
      }
      if (d.reduce_mask & FUSEML_RED_SUM) atomicAdd(d.reduce_out[0] + idx, s);
      if (d.reduce_mask & FUSEML_RED_AMAX) atomic_max_f32(d.reduce_out[1] + idx, mx);
      if (d.reduce_mask & FUSEML_RED_MEAN) atomicAdd(d.reduce_out[2] + idx, s * inv);
    }
  }
}

}  // namespace fuseml_gemm

// Explicit instantiation of one tile variant's four generic kernels (bf16/f16
// operands, with and without reductions), and of fixed-chain kernels.
#define FUSEML_GEMM_INSTANTIATE_ONE(C, T, R, CH)                                                  \
  template __global__ void fuseml_gemm::gemm_epilogue_kernel<C.bm, C.bn, C.bk, C.stages, C.wm, C.wn, \
                                                              C.sched, T, R, CH>(const fuseml_gemm_desc);
#define FUSEML_GEMM_INSTANTIATE(C)                                             \
  FUSEML_GEMM_INSTANTIATE_ONE(C, __bf16, false, fuseml_gemm::kChainGeneric)    \
  FUSEML_GEMM_INSTANTIATE_ONE(C, __bf16, true, fuseml_gemm::kChainGeneric)     \
  FUSEML_GEMM_INSTANTIATE_ONE(C, _Float16, false, fuseml_gemm::kChainGeneric)  \
  FUSEML_GEMM_INSTANTIATE_ONE(C, _Float16, true, fuseml_gemm::kChainGeneric)
