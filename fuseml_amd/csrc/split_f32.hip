// split_f32.hip — fp32 GEMM operands as bf16 parts for the MFMA kernels.
//
// gfx950 has no fp32-input MFMA faster than v_mfma_f32_32x32x2_f32 (1/16 of
// the bf16 rate) and no xf32 format.  An fp32 value x is split into
//     hi = bf16(x)            (round to nearest even)
//     lo = bf16(x - hi)       (x - hi is exact in fp32)
// so x = hi + lo to within 2^-17 |x|.  With both GEMM operands split, the
// three-term product
//     a.b  ~=  hi(a) hi(b) + hi(a) lo(b) + lo(a) hi(b)
// drops only lo(a) lo(b) (at most 2^-16 |a b|); bf16 products are exact in the
// MFMA's fp32 accumulator.  The three terms are one bf16 GEMM over a K axis
// three times as long: row r of the split operand is three segments of k_pad
// columns, segment s holding hi or lo parts of row r, so that
//     A3 = [hi(A) | hf(A) | lo(A)],   B3 = [hi(B) | lo(B) | hf(B)]
// gives A3 . B3 = the three-term product, and the existing GEMM+epilogue
// kernels run unchanged on (A3, B3, K' = 3 k_pad).
// Non-finite values: lo(inf) = lo(NaN) = 0, and hf(x) is hi(x) with every
// non-finite x written as 0.  Only the hi.hi segment then carries inf and
// NaN: the cross terms hf(a) lo(b) and lo(a) hf(b) are finite, where
// hi(inf) lo(b) would be inf * 0 = NaN for any b exact in bf16.  So a row
// with an inf gives inf (or NaN where fp32 gives NaN: inf * 0, inf - inf),
// as fp32 does.
//
// The reference runs fp32 GEMM inputs through Triton's default tf32 `tl.dot`
// (fuseml/codegen/kernel_generator.py:1536), whose inputs keep 10 mantissa
// bits; the split keeps about 16.
//
// The split itself is HBM-bound byte work (4 bytes read, 6 written per
// element): one thread per 8 consecutive k of a row, 32-byte reads and three
// 16-byte writes, consecutive threads on consecutive k.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include "fuseml_hip.h"

namespace fuseml_detail {
// The library's error text (fuseml_last_error), shared with gemm_epilogue.hip.
void set_error_text(const char* msg);
}  // namespace fuseml_detail

namespace {

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr float kBf16Max = 3.38953139e38f;  // largest finite bf16, (2 - 2^-7) 2^127

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// hi, lo and hf parts of two values, packed as bf16 pairs.  A value whose
// nearest bf16 would overflow (|x| above the largest finite bf16) takes the
// truncated hi part instead, so that hi stays finite and lo carries the rest.
// Inf and NaN have lo = 0 and hf = 0 (hf is hi with non-finite values zeroed).
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo, uint32_t& hf) {
  uint32_t h = pack_bf16x2(a, b);
  const uint32_t ta = __float_as_uint(a) >> 16, tb = __float_as_uint(b) & 0xffff0000u;
  const bool fa = __builtin_isfinite(a), fb = __builtin_isfinite(b);
  if (__builtin_fabsf(a) > kBf16Max && fa) h = (h & 0xffff0000u) | ta;
  if (__builtin_fabsf(b) > kBf16Max && fb) h = (h & 0x0000ffffu) | tb;
  const float ha = __uint_as_float(h << 16), hb = __uint_as_float(h & 0xffff0000u);
  const float ra = fa ? a - ha : 0.0f;
  const float rb = fb ? b - hb : 0.0f;
  hi = h;
  lo = pack_bf16x2(ra, rb);
  hf = h & ((fa ? 0x0000ffffu : 0u) | (fb ? 0xffff0000u : 0u));
}

// Thread t of the grid-stride loop handles row t / groups, columns
// 8 (t % groups) .. +7, groups = k_pad / 8.  Columns at or past K read as 0.
template <bool kContig>
__global__ void __launch_bounds__(kThreads)
split_bf16x3_kernel(const float* __restrict__ src, int64_t rows, int64_t K, int64_t stride_r, int64_t stride_k,
                    uint16_t* __restrict__ dst, int64_t ld_dst, int64_t k_pad, uint32_t seg_codes) {
  const int64_t groups = k_pad / 8;
  const int64_t total = rows * groups;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (int64_t)gridDim.x * kThreads) {
    const int64_t r = t / groups;
    const int64_t k0 = (t - r * groups) * 8;
    float x[8];
    if (kContig && k0 + 8 <= K) {
      const float4* p = reinterpret_cast<const float4*>(src + r * stride_r + k0);
      const float4 u = p[0], v = p[1];
      x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
      x[4] = v.x; x[5] = v.y; x[6] = v.z; x[7] = v.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = k0 + e < K ? src[r * stride_r + (k0 + e) * stride_k] : 0.0f;
    }
    uint32_t hi[4], lo[4], hf[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) split2(x[2 * q], x[2 * q + 1], hi[q], lo[q], hf[q]);
    const uint4 H = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    const uint4 L = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    const uint4 HF = make_uint4(hf[0], hf[1], hf[2], hf[3]);
    uint16_t* row = dst + r * ld_dst + k0;
    // seg_codes is uniform: a branch per segment (a select of the vectors
    // would go through scratch memory).
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      uint4* p = reinterpret_cast<uint4*>(row + s * k_pad);
      const uint32_t code = (seg_codes >> (2 * s)) & 3u;
      if (code == FUSEML_SEG_LO)
        *p = L;
      else if (code == FUSEML_SEG_HI_FINITE)
        *p = HF;
      else
        *p = H;
    }
  }
}

void set_error(const char* msg) { fuseml_detail::set_error_text(msg); }

}  // namespace

extern "C" {

int fuseml_split_bf16x3(const float* src, int64_t rows, int64_t K, int64_t stride_r, int64_t stride_k, void* dst,
                        int64_t ld_dst, int64_t k_pad, uint32_t seg_codes, void* stream) {
  set_error("");
  bool codes_ok = (seg_codes >> 6) == 0;
  for (int s = 0; s < 3; ++s) codes_ok = codes_ok && ((seg_codes >> (2 * s)) & 3u) <= FUSEML_SEG_HI_FINITE;
  if (rows < 0 || K < 0 || stride_r < 0 || stride_k < 0 || k_pad < K || k_pad % 8 != 0 || !codes_ok ||
      ld_dst < 3 * k_pad || ld_dst % 8 != 0) {
    set_error("split_bf16x3: bad sizes (need 0 <= K <= k_pad, k_pad % 8 == 0, ld_dst >= 3 k_pad, ld_dst % 8 == 0, "
              "three 2-bit segment codes each <= FUSEML_SEG_HI_FINITE)");
    return FUSEML_EINVAL;
  }
  if (rows == 0 || k_pad == 0) return FUSEML_OK;
  if (dst == nullptr || (K > 0 && src == nullptr) || ((uintptr_t)dst & 15)) {
    set_error("split_bf16x3: null pointer or destination not 16-byte aligned");
    return FUSEML_EINVAL;
  }
  if (rows >= ((int64_t)1 << 40) || k_pad >= ((int64_t)1 << 30)) {
    set_error("split_bf16x3: size exceeds 2^40 rows or 2^30 columns");
    return FUSEML_EUNSUPPORTED;
  }
  const bool contig = stride_k == 1 && stride_r % 4 == 0 && ((uintptr_t)src & 15) == 0;
  const int64_t total = rows * (k_pad / 8);
  int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 65536) blocks = 65536;  // grid-stride beyond 16M threads
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  uint16_t* d = reinterpret_cast<uint16_t*>(dst);
  if (contig)
    hipLaunchKernelGGL(split_bf16x3_kernel<true>, dim3((unsigned)blocks), dim3(kThreads), 0, s, src, rows, K,
                       stride_r, stride_k, d, ld_dst, k_pad, seg_codes);
  else
    hipLaunchKernelGGL(split_bf16x3_kernel<false>, dim3((unsigned)blocks), dim3(kThreads), 0, s, src, rows, K,
                       stride_r, stride_k, d, ld_dst, k_pad, seg_codes);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char msg[256];
    strncpy(msg, "split_bf16x3 launch: ", sizeof(msg) - 1);
    msg[sizeof(msg) - 1] = '\0';
    strncat(msg, hipGetErrorString(e), sizeof(msg) - strlen(msg) - 1);
    set_error(msg);
    return FUSEML_EHIP;
  }
  return FUSEML_OK;
}

}  // extern "C"
