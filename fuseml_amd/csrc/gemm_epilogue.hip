// gemm_epilogue.hip — the gfx950 fused GEMM+epilogue kernel family and its C ABI.
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
// Kernel structure (per workgroup = one BM x BN output tile):
//   * Both operands are K-contiguous in HBM (A = x[M,K]; B = t(W), i.e. W[N,K]),
//     so both are staged into LDS as [rows][BK=64] bf16 rows of 128 bytes, with
//     the 16-byte chunk index XOR-swizzled by (row & 7) so that the 32 lanes of a
//     ds_read_b128 that read one chunk column of 32 consecutive rows hit 8
//     distinct chunk slots per 8 rows (no bank conflicts).
//   * Two LDS stages (double buffering): the global loads of K-tile t+1 are
//     issued into registers before the MFMAs of tile t, and written to the
//     other stage afterwards; one barrier per K-tile.
//   * Global loads are raw buffer loads: an out-of-range offset returns zeros,
//     which implements the M/N/K boundary masking with no branches.
//   * MFMA roles are swapped (MFMA "A" = rows of W, MFMA "B" = rows of x) so that
//     each lane's accumulator holds one output row m and runs of 4 consecutive
//     columns n: epilogue operands are read and the output is written as 8-byte
//     vectors, and a row reduction needs a single cross-half-wave exchange.
//   * The workgroup -> tile map is XCD-aware: the hardware deals workgroups to
//     the 8 XCDs round-robin, so each XCD is given a contiguous range of
//     logical tiles, ordered in GROUP_M-row column strips for L2 reuse.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fuseml_hip.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));

constexpr int kBK = 64;                 // K elements per LDS stage
constexpr int kRowBytes = kBK * 2;      // one LDS row = 64 x 16-bit = 128 bytes
constexpr int kGroupM = 8;              // tile-row strip height of the tile order
constexpr uint32_t kOOB = 0x80000000u;  // buffer offset that always reads zero
constexpr int kRsrcWord3 = 0x00020000;  // buffer descriptor word 3 for gfx9 (32-bit data)
constexpr float kFp16Max = 65504.0f;

thread_local char g_last_error[512];

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
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

__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
  // Saturate to the finite fp16 range before narrowing
  // (fuseml/codegen/kernel_generator.py:1575-1581).
  x = fminf(fmaxf(x, -kFp16Max), kFp16Max);
  _Float16 h = (_Float16)x;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ int dtype_bytes(int dtype) { return dtype == FUSEML_F32 ? 4 : 2; }

// Load the 4 operand values at (m, n..n+3).  `ok` says the whole run of four is
// inside [0,M) x [0,N); an invalid run reads zeros through the buffer bound.
__device__ __forceinline__ void load_operand4(const fuseml_operand& op, int m, int n, bool ok,
                                              float v[4]) {
  const int dt = op.dtype;
  const int eb = dtype_bytes(dt);
  const __amdgpu_buffer_rsrc_t r = make_rsrc(op.ptr, (uint32_t)(op.extent * eb));
  const int64_t base = (int64_t)m * op.stride_m + (int64_t)n * op.stride_n;
  if (op.stride_n == 1 && op.reserved) {
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
__device__ __forceinline__ void store_out4(const fuseml_output& o, int m, int n, int M, int N,
                                           const float v[4]) {
  if (m >= M || n >= N) return;
  const int64_t base = (int64_t)m * o.ld + n;
  if (o.dtype == FUSEML_F32) {
    float* p = reinterpret_cast<float*>(o.ptr) + base;
    if (o.reserved) {
      *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      for (int e = 0; e < 4 && n + e < N; ++e) p[e] = v[e];
    }
    return;
  }
  uint32_t h[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    h[e] = (o.dtype == FUSEML_BF16) ? f32_to_bf16_bits(v[e]) : f32_to_f16_bits(v[e]);
  uint16_t* p = reinterpret_cast<uint16_t*>(o.ptr) + base;
  if (o.reserved) {
    uint2 w;
    w.x = h[0] | (h[1] << 16);
    w.y = h[2] | (h[3] << 16);
    *reinterpret_cast<uint2*>(p) = w;
  } else {
    for (int e = 0; e < 4 && n + e < N; ++e) p[e] = (uint16_t)h[e];
  }
}

// Float atomic max through integer atomics: non-negative floats order like
// signed ints, negative floats order inversely like unsigned ints.
__device__ __forceinline__ void atomic_max_f32(float* p, float v) {
  if (v >= 0.0f)
    atomicMax(reinterpret_cast<int*>(p), __float_as_int(v));
  else
    atomicMin(reinterpret_cast<unsigned int*>(p), __float_as_uint(v));
}

__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

__device__ __forceinline__ float gelu_tanh(float x) {
  // sqrt(2/pi) = 0.7978845608...; cubic coefficient 0.044715 (Hendrycks & Gimpel 2016).
  const float u = 0.79788456080286536f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(u));
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// Run the epilogue op chain on one 32x32 accumulator block of this lane:
// v[4g+e] is element (m, nb + 8g + e).  The chain is read from the kernel
// arguments, so the loop and its switch are uniform (scalar) control flow.
__device__ __forceinline__ void epilogue_block(const fuseml_gemm_desc& d, f32x16_t& v, int m,
                                               int nb, int M, int N) {
  for (int o = 0; o < d.n_ops; ++o) {
    const int kind = d.ops[o].kind;
    const float sc = d.ops[o].scalar;
    const int oi = d.ops[o].operand;
    switch (kind) {
      case FUSEML_OP_ADD:
      case FUSEML_OP_MUL: {
        float x[16];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = nb + 8 * g;
          load_operand4(d.operands[oi], m, n, m < M && n < N, x + 4 * g);
        }
        if (kind == FUSEML_OP_ADD) {
#pragma unroll
          for (int r = 0; r < 16; ++r) v[r] = fmaf(sc, x[r], v[r]);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) v[r] = v[r] * x[r];
        }
        break;
      }
      case FUSEML_OP_STORE: {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float x[4] = {v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
          store_out4(d.extra[oi], m, nb + 8 * g, M, N, x);
        }
        break;
      }
      case FUSEML_OP_RELU:
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = v[r] > 0.0f ? v[r] : 0.0f;
        break;
      case FUSEML_OP_GELU_ERF:
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = gelu_erf(v[r]);
        break;
      case FUSEML_OP_GELU_TANH:
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = gelu_tanh(v[r]);
        break;
      case FUSEML_OP_SIGMOID:
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = sigmoid(v[r]);
        break;
      case FUSEML_OP_SCALE:
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = v[r] * sc;
        break;
      case FUSEML_OP_ADD_SCALAR:
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = v[r] + sc;
        break;
      case FUSEML_OP_ADD_SELF:
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = fmaf(sc, v[r], v[r]);
        break;
      case FUSEML_OP_MUL_SELF:
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = v[r] * v[r];
        break;
      default:
        break;
    }
  }
}

// ---------------------------------------------------------------------------
// The kernel
// ---------------------------------------------------------------------------

template <int BM, int BN, int WM, int WN, typename T>
__global__ __launch_bounds__(WM* WN * 64) void gemm_epilogue_kernel(const fuseml_gemm_desc d) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM;  // wave tile rows (m)
  constexpr int TN = BN / WN;  // wave tile cols (n)
  constexpr int NJ = TM / 32;  // 32x32 blocks along m (MFMA "B" operand)
  constexpr int NI = TN / 32;  // 32x32 blocks along n (MFMA "A" operand)
  constexpr int A_BYTES = BM * kRowBytes;
  constexpr int STAGE = (BM + BN) * kRowBytes;
  constexpr int A_LD = BM * 8 / NT;  // 16-byte chunks per thread per A stage
  constexpr int B_LD = BN * 8 / NT;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert((BM * 8) % NT == 0 && (BN * 8) % NT == 0, "stage loads must divide evenly");

  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN;
  const int wn = wave % WN;

  const int M = (int)d.M, N = (int)d.N, K = (int)d.K;
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;

  // XCD-aware tile order.
  const int nwg = gridDim.x;
  int lid = blockIdx.x;
  if ((nwg & 7) == 0) lid = (lid & 7) * (nwg >> 3) + (lid >> 3);
  const int strip = kGroupM * tiles_n;
  const int first_m = (lid / strip) * kGroupM;
  const int strip_h = min(tiles_m - first_m, kGroupM);
  const int pid_m = first_m + (lid % strip) % strip_h;
  const int pid_n = (lid % strip) / strip_h;
  const int m0 = pid_m * BM;
  const int n0 = pid_n * BN;

  // Operand buffer resources (the host guarantees the byte extents fit in 31 bits).
  const uint32_t a_bytes = (uint32_t)(((int64_t)(M - 1) * d.lda + K) * 2);
  const uint32_t b_bytes = (uint32_t)(((int64_t)(N - 1) * d.ldb + K) * 2);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(d.a, a_bytes);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(d.b, b_bytes);

  // Per-thread global chunk coordinates (constant over the K loop).
  uint32_t a_row_off[A_LD], b_row_off[B_LD];
  int a_kc[A_LD], b_kc[B_LD];
  uint32_t a_lds[A_LD], b_lds[B_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int c = tid + NT * i;
    const int row = c >> 3, kc = c & 7;
    const int gm = m0 + row;
    a_row_off[i] = gm < M ? (uint32_t)((int64_t)gm * d.lda * 2) : kOOB;
    a_kc[i] = kc;
    a_lds[i] = row * kRowBytes + ((kc ^ (row & 7)) << 4);
  }
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const int c = tid + NT * i;
    const int row = c >> 3, kc = c & 7;
    const int gn = n0 + row;
    b_row_off[i] = gn < N ? (uint32_t)((int64_t)gn * d.ldb * 2) : kOOB;
    b_kc[i] = kc;
    b_lds[i] = A_BYTES + row * kRowBytes + ((kc ^ (row & 7)) << 4);
  }

  i32x4_t ga[A_LD], gb[B_LD];
  auto load_tile = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int k = k0 + a_kc[i] * 8;
      const uint32_t off = (a_row_off[i] != kOOB && k < K) ? a_row_off[i] + (uint32_t)(k * 2) : kOOB;
      ga[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int k = k0 + b_kc[i] * 8;
      const uint32_t off = (b_row_off[i] != kOOB && k < K) ? b_row_off[i] + (uint32_t)(k * 2) : kOOB;
      gb[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0);
    }
  };
  auto store_tile = [&](int stage) {
    char* s = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) *reinterpret_cast<i32x4_t*>(s + a_lds[i]) = ga[i];
#pragma unroll
    for (int i = 0; i < B_LD; ++i) *reinterpret_cast<i32x4_t*>(s + b_lds[i]) = gb[i];
  };

  f32x16_t acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // Fragment row offsets inside a stage: rows of W for MFMA "A", rows of x for MFMA "B".
  const int l32 = lane & 31;
  const int khalf = lane >> 5;
  const int swz = lane & 7;  // == row & 7 for every fragment row this lane reads

  const int nk = (K + kBK - 1) / kBK;
  if (nk > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int stage = kt & 1;
    if (kt + 1 < nk) load_tile(kt + 1);
    const char* s = smem + stage * STAGE;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int kc = 2 * ks + khalf;
      const int chunk = (kc ^ swz) << 4;
      i32x4_t fa[NI], fb[NJ];
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int row = wn * TN + 32 * i + l32;
        fa[i] = *reinterpret_cast<const i32x4_t*>(s + A_BYTES + row * kRowBytes + chunk);
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int row = wm * TM + 32 * j + l32;
        fb[j] = *reinterpret_cast<const i32x4_t*>(s + row * kRowBytes + chunk);
      }
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32<T>(fa[i], fb[j], acc[i][j]);
    }
    if (kt + 1 < nk) store_tile(stage ^ 1);
    __syncthreads();
  }

  // ---------------------------------------------------------------------
  // Epilogue, one 32x32 accumulator block at a time.  In block (i,j),
  // register r of this lane holds
  //   m = m0 + wm*TM + 32j + (lane & 31)
  //   n = n0 + wn*TN + 32i + 8*(r>>2) + 4*(lane>>5) + (r&3)
  // ---------------------------------------------------------------------
  const int mw = m0 + wm * TM + l32;
  const int nw = n0 + wn * TN + 4 * khalf;
  const bool row_red = d.reduce_mask != 0 && d.reduce_axis == 1;
  const bool col_red = d.reduce_mask != 0 && d.reduce_axis == 0;
  float* red_sum = reinterpret_cast<float*>(smem);  // LDS is free after the K loop
  float* red_max = red_sum + (d.reduce_axis == 1 ? WN * BM : WM * BN);

  float rs[NJ], rmx[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    rs[j] = 0.0f;
    rmx[j] = -INFINITY;
  }

#pragma unroll
  for (int i = 0; i < NI; ++i) {
    float cs[16], cmx[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      cs[r] = 0.0f;
      cmx[r] = -INFINITY;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int m = mw + 32 * j;
      const int nb = nw + 32 * i;
      f32x16_t v = acc[i][j];
      epilogue_block(d, v, m, nb, M, N);
      if (d.out.ptr != nullptr) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float x[4] = {v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
          store_out4(d.out, m, nb + 8 * g, M, N, x);
        }
      }
      // Partial reductions exclude every element outside [0,M) x [0,N) (the
      // reference lets padded tile elements through, kernel_generator.py:1959-1960,
      // 1983-1984).
      if (row_red || col_red) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int n = nb + 8 * (r >> 2) + (r & 3);
          const bool in = (m < M) && (n < N);
          const float x = v[r];
          if (row_red && in) {
            rs[j] += x;
            rmx[j] = fmaxf(rmx[j], x);
          }
          if (col_red && in) {
            cs[r] += x;
            cmx[r] = fmaxf(cmx[r], x);
          }
        }
      }
    }
    if (col_red) {
      // Column partials: reduce over the 32 rows held by each half-wave.
#pragma unroll
      for (int r = 0; r < 16; ++r) {
#pragma unroll
        for (int sh = 1; sh < 32; sh <<= 1) {
          cs[r] += __shfl_xor(cs[r], sh);
          cmx[r] = fmaxf(cmx[r], __shfl_xor(cmx[r], sh));
        }
        if (l32 == 0) {
          const int col = wn * TN + 32 * i + 8 * (r >> 2) + 4 * khalf + (r & 3);
          red_sum[wm * BN + col] = cs[r];
          red_max[wm * BN + col] = cmx[r];
        }
      }
    }
  }

  if (row_red) {
    // Row partials: the other half-wave holds the other 4-column runs of the same rows.
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float s2 = rs[j] + __shfl_xor(rs[j], 32);
      const float m2 = fmaxf(rmx[j], __shfl_xor(rmx[j], 32));
      if (lane < 32) {
        const int row = wm * TM + 32 * j + lane;
        red_sum[wn * BM + row] = s2;
        red_max[wn * BM + row] = m2;
      }
    }
  }
  if (d.reduce_mask == 0) return;
  __syncthreads();

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
      mx = fmaxf(mx, red_max[w * len + t]);
    }
    if (d.reduce_mask & FUSEML_RED_SUM) atomicAdd(d.reduce_out[0] + idx, s);
    if (d.reduce_mask & FUSEML_RED_AMAX) atomic_max_f32(d.reduce_out[1] + idx, mx);
    if (d.reduce_mask & FUSEML_RED_MEAN) atomicAdd(d.reduce_out[2] + idx, s * inv);
  }
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

struct TileConfig {
  int bm, bn, wm, wn;
};

constexpr TileConfig kLarge = {256, 256, 2, 4};  // 8 waves, 128 KB LDS
constexpr TileConfig kSmall = {128, 128, 2, 2};  // 4 waves,  64 KB LDS

constexpr int64_t kMaxBytes = (int64_t)1 << 31;

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

TileConfig choose_config(const fuseml_gemm_desc& d) {
  // A 256x256 tile keeps the LDS traffic per MFMA low enough for the MFMA pipe
  // to stay busy; below one full wave of 256-tile work the 128x128 variant
  // fills more CUs.
  const int64_t large_tiles = cdiv(d.M, 256) * cdiv(d.N, 256);
  return large_tiles >= 128 ? kLarge : kSmall;
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
  if (d.K > 0 &&
      (((d.M - 1) * d.lda + d.K) * 2 >= kMaxBytes || ((d.N - 1) * d.ldb + d.K) * 2 >= kMaxBytes)) {
    set_error("GEMM operand spans 2 GiB or more");
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
    if (op.extent * (op.dtype == FUSEML_F32 ? 4 : 2) >= kMaxBytes) {
      set_error("operand %d spans 2 GiB or more", i);
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

// Fill in the host-derived vector-path flags (kept in the `reserved` fields).
void derive_flags(fuseml_gemm_desc& d) {
  for (int i = 0; i < d.n_operands; ++i) {
    fuseml_operand& op = d.operands[i];
    const int eb = op.dtype == FUSEML_F32 ? 4 : 2;
    const bool vec = op.stride_n == 1 && (op.stride_m % 4 == 0) && (d.N % 4 == 0) &&
                     ((uintptr_t)op.ptr % (4 * eb) == 0);
    op.reserved = vec ? 1 : 0;
  }
  auto out_flag = [&](fuseml_output& o) {
    const int eb = o.dtype == FUSEML_F32 ? 4 : 2;
    o.reserved = (o.ptr != nullptr && o.ld % 4 == 0 && d.N % 4 == 0 &&
                  (uintptr_t)o.ptr % (4 * eb) == 0)
                     ? 1
                     : 0;
  };
  out_flag(d.out);
  for (int i = 0; i < d.n_extra; ++i) out_flag(d.extra[i]);
}

template <int BM, int BN, int WM, int WN>
hipError_t launch_variant(const fuseml_gemm_desc& d, hipStream_t stream) {
  const int64_t tiles = cdiv(d.M, BM) * cdiv(d.N, BN);
  const dim3 grid((unsigned)tiles), block(WM * WN * 64);
  if (d.ab_dtype == FUSEML_BF16)
    hipLaunchKernelGGL((gemm_epilogue_kernel<BM, BN, WM, WN, __bf16>), grid, block, 0, stream, d);
  else
    hipLaunchKernelGGL((gemm_epilogue_kernel<BM, BN, WM, WN, _Float16>), grid, block, 0, stream, d);
  return hipGetLastError();
}

}  // namespace

extern "C" {

const char* fuseml_last_error(void) { return g_last_error; }

int fuseml_abi_version(void) { return FUSEML_ABI_VERSION; }

size_t fuseml_desc_size(void) { return sizeof(fuseml_gemm_desc); }

int fuseml_gemm_epilogue_supported(const fuseml_gemm_desc* desc) {
  g_last_error[0] = '\0';
  return validate(desc) == FUSEML_OK ? 1 : 0;
}

int fuseml_gemm_epilogue_config(const fuseml_gemm_desc* desc, int32_t cfg[4]) {
  g_last_error[0] = '\0';
  const int rc = validate(desc);
  if (rc != FUSEML_OK) return rc;
  const TileConfig c = choose_config(*desc);
  cfg[0] = c.bm;
  cfg[1] = c.bn;
  cfg[2] = c.wm * c.wn;
  cfg[3] = 2 * (c.bm + c.bn) * kRowBytes;
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
  char arch[64];
  if (fuseml_device_arch(dev, arch, sizeof(arch)) != FUSEML_OK) return FUSEML_EHIP;
  if (strncmp(arch, "gfx950", 6) != 0) {
    set_error("device %d is %s; kernels are built for gfx950 only", dev, arch);
    return FUSEML_EDEVICE;
  }

  fuseml_gemm_desc d = *desc;
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

  const TileConfig c = choose_config(d);
  if (c.bm == kLarge.bm && c.bn == kLarge.bn)
    e = launch_variant<kLarge.bm, kLarge.bn, kLarge.wm, kLarge.wn>(d, stream);
  else
    e = launch_variant<kSmall.bm, kSmall.bn, kSmall.wm, kSmall.wn>(d, stream);
  if (e != hipSuccess) {
    set_error("gemm_epilogue launch: %s", hipGetErrorString(e));
    return FUSEML_EHIP;
  }
  return FUSEML_OK;
}

}  // extern "C"
