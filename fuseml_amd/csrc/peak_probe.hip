// peak_probe.hip — the achievable bf16 MFMA rate of this device at its
// sustained clock, for the benchmark's roofline.
//
// The spec peak (2.5 PFLOP/s dense bf16 on MI355X) assumes the 2.4 GHz peak
// clock; under a long MFMA load with random operands the device runs at its
// power-limited clock instead.  This kernel issues only MFMAs
// (v_mfma_f32_32x32x16_bf16, the instruction the GEMM kernels use) from every
// SIMD of every CU, on register operands holding pseudo-random bf16 values (so
// the datapath toggles as it does on real data), with eight independent
// accumulators per wave so that consecutive MFMAs never wait on each other.
// FLOPs per launch = workgroups * 4 waves * iters * 8 MFMAs * 2*32*32*16.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "fuseml_hip.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kAcc = 8;

// bf16 with a random sign and mantissa and exponent 126 (|v| in [0.5, 1)).
__device__ __forceinline__ uint32_t rand_bf16x2(uint32_t h) {
  h ^= h >> 16;
  h *= 0x7feb352dU;
  h ^= h >> 15;
  h *= 0x846ca68bU;
  h ^= h >> 16;
  return (h & 0x807f807fU) | 0x3f003f00U;
}

__global__ __launch_bounds__(256) void mfma_peak_kernel(int64_t iters, float* sink) {
  const uint32_t seed = (blockIdx.x * 256u + threadIdx.x) * 8u;
  i32x4_t a, b;
  a.x = (int)rand_bf16x2(seed + 0);
  a.y = (int)rand_bf16x2(seed + 1);
  a.z = (int)rand_bf16x2(seed + 2);
  a.w = (int)rand_bf16x2(seed + 3);
  b.x = (int)rand_bf16x2(seed + 4);
  b.y = (int)rand_bf16x2(seed + 5);
  b.z = (int)rand_bf16x2(seed + 6);
  b.w = (int)rand_bf16x2(seed + 7);
  f32x16_t acc[kAcc];
#pragma unroll
  for (int q = 0; q < kAcc; ++q)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[q][r] = 0.0f;
  for (int64_t i = 0; i < iters; ++i) {
#pragma unroll
    for (int q = 0; q < kAcc; ++q)
      acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                        __builtin_bit_cast(bf16x8_t, b), acc[q], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int q = 0; q < kAcc; ++q)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[q][r];
  // One value per thread keeps the MFMAs live; the caller's buffer has
  // workgroups * 256 floats.
  sink[blockIdx.x * 256u + threadIdx.x] = s;
}

}  // namespace

extern "C" int fuseml_mfma_peak_probe(int64_t iters, int32_t workgroups, float* sink, void* stream) {
  if (iters <= 0 || workgroups <= 0 || sink == nullptr) return FUSEML_EINVAL;
  hipLaunchKernelGGL(mfma_peak_kernel, dim3((unsigned)workgroups), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), iters, sink);
  return hipGetLastError() == hipSuccess ? FUSEML_OK : FUSEML_EHIP;
}
