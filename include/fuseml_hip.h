/*
 * fuseml_hip.h — C ABI of the MI355X (gfx950) fused GEMM+epilogue kernel family.
 *
 * One call computes, for one fusion group (addmm|mm -> pointwise* -> [row/col
 * reduction]):
 *
 *     acc[m,n]  = sum_k A[m,k] * B[k,n]              (bf16|f16 MFMA, fp32 accumulate)
 *     v[m,n]    = ops[n_ops-1]( ... ops[0](acc) ...)  (fp32, in registers)
 *     out[m,n]  = cast(v)                             (one store, optional)
 *     red[m|n]  = sum / amax / mean of v along N or M (fp32 atomics, optional)
 *
 * The entry points replace the reference's kernel-side ABI:
 *   - fuseml_gemm_epilogue replaces the Triton launch
 *       `kernel_fn[grid](ptrs..., M, N, K, strides...)`
 *     at fuseml/codegen/kernel_launcher.py:793-796 and 811-814 (argument layout
 *     built at kernel_launcher.py:766-785, kernel signature emitted at
 *     fuseml/codegen/kernel_generator.py:1182-1262), and the cuBLASLt
 *     `addmm_bias_residual` extension entry point at
 *     fuseml/codegen/cublas_epilogue.py:355-557 (called at 655-676).
 *   - fuseml_gemm_epilogue_supported replaces the "can this group be fused"
 *     decisions of fuseml/passes/topology.py:479-571 (is_compute_bound_gemm) and
 *     fuseml/codegen/cublas_epilogue.py:166-258 (match_cublas_epilogue): with one
 *     kernel family the only question left is whether a variant exists.
 *   - fuseml_last_error replaces the exception text Triton raises through
 *     EagerFallbackGuard (fuseml/codegen/eager_fallback.py:147-166).
 *
 * Conventions
 *   - All pointers are device pointers owned by the caller (PyTorch's caching
 *     allocator).  The library allocates nothing and frees nothing.
 *   - Strides are in ELEMENTS.  A is [M,K] with unit stride along K; B is the
 *     graph's right operand [K,N] with unit stride along K (the `t(W)` view of an
 *     nn.Linear weight W[N,K]); `ldb` is its stride along N.
 *   - Every call is asynchronous on `stream` and captures no host state, so it
 *     is safe inside HIP graph capture.  Reduction buffers are initialised by a
 *     fill kernel on the same stream (no hipMemset).
 *   - Operands and outputs may exceed 2 GiB: buffer accesses are based at each
 *     tile's origin, so only the elements one 256x256 tile reaches must span
 *     less than 2 GiB.
 *   - Return value: 0 on success, a negative FUSEML_E* code otherwise; the
 *     message is available from fuseml_last_error() on the calling thread.
 */
#ifndef FUSEML_HIP_H_
#define FUSEML_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FUSEML_ABI_VERSION 6

#define FUSEML_MAX_OPS 16
#define FUSEML_MAX_OPERANDS 8
#define FUSEML_MAX_EXTRA_OUT 4

/* Element types (operands, outputs). */
enum {
  FUSEML_BF16 = 0,
  FUSEML_F16 = 1,
  FUSEML_F32 = 2
};

/* Epilogue op codes.  The op vocabulary is the reference's supported-op table
 * (fuseml/passes/graph_cut.py:37-55) plus what addmm's own arguments need. */
enum {
  FUSEML_OP_NONE = 0,
  FUSEML_OP_ADD = 1,        /* v = v + scalar * operand[m,n]   (add.Tensor, addmm bias)   */
  FUSEML_OP_MUL = 2,        /* v = v * operand[m,n]                                        */
  FUSEML_OP_RELU = 3,       /* v = v > 0 ? v : 0                                           */
  FUSEML_OP_GELU_ERF = 4,   /* v = 0.5 v (1 + erf(v / sqrt 2))      gelu approximate=none  */
  FUSEML_OP_GELU_TANH = 5,  /* v = 0.5 v (1 + tanh(sqrt(2/pi)(v + 0.044715 v^3)))          */
  FUSEML_OP_SIGMOID = 6,    /* v = 1 / (1 + exp(-v))                                       */
  FUSEML_OP_SCALE = 7,      /* v = v * scalar                (addmm alpha, mul by scalar)  */
  FUSEML_OP_ADD_SCALAR = 8, /* v = v + scalar                (add of a Python number)      */
  FUSEML_OP_STORE = 9,      /* extra[operand][m,n] = cast(v) (escape / intermediate store) */
  FUSEML_OP_ADD_SELF = 10,  /* v = v + scalar * v            (add(x, x, alpha))            */
  FUSEML_OP_MUL_SELF = 11   /* v = v * v                     (mul(x, x))                   */
};

/* Reduction selection (bit mask) — fuseml/codegen/kernel_generator.py:1933-2018. */
enum {
  FUSEML_RED_SUM = 1,
  FUSEML_RED_AMAX = 2,
  FUSEML_RED_MEAN = 4
};

/* Error codes. */
enum {
  FUSEML_OK = 0,
  FUSEML_EINVAL = -1,       /* malformed descriptor                                */
  FUSEML_EUNSUPPORTED = -2, /* valid request with no kernel variant (eager bypass) */
  FUSEML_EHIP = -3,         /* HIP runtime error at launch                         */
  FUSEML_EDEVICE = -4       /* current device is not gfx950                        */
};

typedef struct fuseml_epi_op {
  int32_t kind;    /* FUSEML_OP_*                                            */
  int32_t operand; /* operand index (ADD/MUL), extra-output index (STORE)   */
  float scalar;    /* ADD: operand multiplier (alpha); SCALE/ADD_SCALAR/ADD_SELF */
  int32_t reserved;
} fuseml_epi_op;

/* A broadcastable epilogue operand: element (m,n) is at
 * ptr[m*stride_m + n*stride_n].  A [N] row vector has stride_m = 0, an [M,1]
 * column has stride_n = 0, a 0-d tensor has both 0, an expanded view keeps its
 * zero strides.  `extent` is one past the largest element offset reachable,
 * i.e. (M-1)*stride_m + (N-1)*stride_n + 1 for the group's M,N. */
typedef struct fuseml_operand {
  const void* ptr;
  int64_t stride_m;
  int64_t stride_n;
  int64_t extent;
  int32_t dtype; /* FUSEML_BF16 | FUSEML_F16 | FUSEML_F32 */
  int32_t reserved;
} fuseml_operand;

/* A row-major [M,N] output: element (m,n) at ptr[m*ld + n]. */
typedef struct fuseml_output {
  void* ptr;
  int64_t ld;
  int32_t dtype;
  int32_t reserved;
} fuseml_output;

typedef struct fuseml_gemm_desc {
  int64_t M, N, K;
  const void* a; /* A[M,K]: element (m,k) at a[m*lda + k]                 */
  int64_t lda;
  const void* b; /* B[K,N]: element (k,n) at b[n*ldb + k]  (B = t(W))    */
  int64_t ldb;
  int32_t ab_dtype; /* FUSEML_BF16 | FUSEML_F16                          */
  int32_t n_ops;
  fuseml_epi_op ops[FUSEML_MAX_OPS];
  int32_t n_operands;
  int32_t n_extra;
  fuseml_operand operands[FUSEML_MAX_OPERANDS];
  fuseml_output out;                         /* ptr NULL: no tile store       */
  fuseml_output extra[FUSEML_MAX_EXTRA_OUT]; /* targets of FUSEML_OP_STORE    */
  int32_t reduce_axis;                       /* 1: over N -> [M]; 0: over M -> [N] */
  uint32_t reduce_mask;                      /* FUSEML_RED_* bits             */
  float* reduce_out[3];                      /* fp32 [M] or [N]: sum, amax, mean */
} fuseml_gemm_desc;

/* Launch the fused kernel for `desc` on `stream` (a hipStream_t; NULL = the
 * null stream).  Replaces kernel_launcher.py:793-796/811-814 and
 * cublas_epilogue.py:542-551. */
int fuseml_gemm_epilogue(const fuseml_gemm_desc* desc, void* stream);

/* 1 if a kernel variant exists for `desc` (shapes, strides, alignment,
 * dtypes), 0 if not (reason in fuseml_last_error()).  Touches no device state.
 * Replaces topology.py:479-571 and cublas_epilogue.py:166-258. */
int fuseml_gemm_epilogue_supported(const fuseml_gemm_desc* desc);

/* Tile configuration the library would launch for `desc`: writes BM, BN,
 * waves per workgroup and LDS bytes into cfg[0..3].  Replaces the launch
 * parameter selection of kernel_launcher.py:134-306 / sram_autotuner.py. */
int fuseml_gemm_epilogue_config(const fuseml_gemm_desc* desc, int32_t cfg[4]);

/* The epilogue a launch of `desc` would compile in: 0 for the generic op loop
 * (the descriptor's ops interpreted at run time), else the id of the fixed
 * chain kernel (1 none, 2 bias, 3 bias+GELU(erf), 4 bias+GELU(tanh),
 * 5 bias+ReLU, 6 bias+2-D add, 7 bias,ReLU,2-D mul,sigmoid,row add, 8 ReLU
 * with or without reductions) — the same arithmetic as straight-line code,
 * built for the one-wave whole-stage variant and bf16 operands.  A negative
 * FUSEML_E* code for an invalid descriptor.  For tests and measurement; it
 * replaces reading which Triton kernel source was generated
 * (fuseml/codegen/kernel_generator.py:1067-1141). */
int fuseml_gemm_epilogue_chain(const fuseml_gemm_desc* desc);

/* Pin the kernel variant for every later launch in this process: "large"
 * (256x256 ping-pong), "deep" (256x256 one wave per SIMD), "deep3" (the same
 * with whole-stage fragments; K % 64 == 0, else deep), "deep3-generic"
 * (deep3 with the generic op loop even where a fixed chain matches), "small"
 * (128x128), "narrow64" (64x128), "narrow32" (32x128), "large128" (256x128
 * ping-pong), "small64" (128x128 at BK = 64), or NULL / "" / "auto" for the
 * automatic choice.  The environment variable
 * FUSEML_HIP_TILE sets the initial value; it is read once per process.  For
 * tuning sweeps and per-variant parity tests; it replaces pinning a Triton
 * autotune config (fuseml/codegen/kernel_generator.py:587-615).  Returns
 * FUSEML_EINVAL for an unknown name. */
int fuseml_gemm_epilogue_force_variant(const char* name);

/* Thread-local text of the last error on this thread ("" if none). */
const char* fuseml_last_error(void);

/* gcnArchName of `device` (e.g. "gfx950:sramecc+:xnack-") into buf. */
int fuseml_device_arch(int device, char* buf, int buflen);

/* ------------------------------------------------------------------------
 * The whole MLP block in one launch (opt-in):
 *
 *     y = post(GELU(x W1^T + b1)) W2^T + b2 + r
 *
 * with h = post(GELU(x W1^T + b1)) kept on chip (never written to HBM);
 * post is up to FUSEML_MLP_MAX_POST scalar ops (FUSEML_OP_SCALE: v * s,
 * FUSEML_OP_ADD_SCALAR: v + s) applied in order in fp32, as the first
 * group's epilogue would (the reference's activation-heavy block,
 * benchmarks/bench_mlp_block.py:185-207, scales and shifts the GELU).  The
 * reference has no counterpart: it runs the block as two launches of its
 * generated kernel (kernel_launcher.py:793-796 / 811-814, once per group),
 * because an addmm ends a fusion group (fuseml/passes/topology.py:63-64) and
 * absorption needs a single user (fuseml/passes/fusion_pass.py:203-206).
 * Operand layouts are the graph's: x [M,D] row-major; W1 as t(W1) [D,I]
 * (element (k,i) at w1[i*ldw1 + k]); W2 as t(W2) [I,D] (element (i,d) at
 * w2[d*ldw2 + i]); b1 [I], b2 [D] (may be NULL), r [M,D] (may be NULL), y [M,D].
 * Limits: D in {256, 512, 1024} (the 64 x D fp32 accumulator of a row block
 * lives in registers), I a multiple of 32, all tensors bf16 or all fp16.
 * ------------------------------------------------------------------------ */
#define FUSEML_MLP_MAX_POST 4

typedef struct fuseml_mlp_desc {
  int64_t M, D, I;
  const void* x;
  int64_t ldx;
  const void* w1;
  int64_t ldw1;
  const void* b1;
  const void* w2;
  int64_t ldw2;
  const void* b2;
  const void* r;
  int64_t ldr;
  void* y;
  int64_t ldy;
  int32_t dtype; /* FUSEML_BF16 | FUSEML_F16, for every tensor     */
  int32_t gelu;  /* FUSEML_OP_GELU_ERF | FUSEML_OP_GELU_TANH       */
  /* Optional: W1 and W2 repacked by fuseml_mlp_pack_weights (NULL: read
   * W1 and W2 as they are).  Used where the kernel streams weight fragments
   * (D of 256 or 512, I a multiple of 128); w1 and w2 are still required. */
  const void* wpack;
  /* Scalar ops applied to GELU's output before it is rounded to h: kinds
   * FUSEML_OP_SCALE or FUSEML_OP_ADD_SCALAR, n_post of them (0 to
   * FUSEML_MLP_MAX_POST). */
  int32_t n_post;
  int32_t post_kind[FUSEML_MLP_MAX_POST];
  float post_scalar[FUSEML_MLP_MAX_POST];
} fuseml_mlp_desc;

/* Launch the single-kernel MLP block on `stream`.  0 or a FUSEML_E* code. */
int fuseml_mlp_block(const fuseml_mlp_desc* desc, void* stream);

/* 1 if fuseml_mlp_block accepts `desc`, 0 if not (reason in fuseml_last_error()). */
int fuseml_mlp_block_supported(const fuseml_mlp_desc* desc);

/* Bytes of the repacked weights for `desc` (4 * D * I: W1 and W2 reordered),
 * or 0 if its shape does not stream weight fragments (D not 256 or 512, or I
 * not a multiple of 128).  Host only. */
int64_t fuseml_mlp_pack_bytes(const fuseml_mlp_desc* desc);

/* Write desc's W1 and W2 into `wpack` (fuseml_mlp_pack_bytes(desc) bytes,
 * 16-byte aligned) in the order the single-kernel MLP consumes them: per
 * 128-column slice of I and per wave, each 16-byte-per-lane MFMA fragment as
 * one contiguous 1 KB block, so every fragment load is whole cache lines
 * (read from W1 and W2 as they are, each lane takes 32 bytes from each of 32
 * rows).  Asynchronous on `stream`.  The caller re-packs after changing W1 or
 * W2.  No reference counterpart: the reference has no single-kernel MLP. */
int fuseml_mlp_pack_weights(const fuseml_mlp_desc* desc, void* wpack, void* stream);

/* ------------------------------------------------------------------------
 * fp32 GEMM operands.  Writes the bf16 parts of an fp32 matrix so that the
 * fused kernel can run an fp32 group as one bf16 GEMM over a K axis three
 * times as long (a three-term split product, about 16 mantissa bits per
 * input).  Replaces Triton's default tf32 `tl.dot` on fp32 inputs
 * (fuseml/codegen/kernel_generator.py:1536), which keeps 10.
 *
 * src element (r,k) is src[r*stride_r + k*stride_k], r < rows, k < K (any
 * non-negative strides).  Row r of dst (bf16, row stride ld_dst) is three
 * segments of k_pad columns; segment s holds the part named by the 2-bit code
 * (seg_codes >> 2s) & 3:
 *   FUSEML_SEG_HI        hi(x) = bf16(x) (round to nearest even; the truncated
 *                        bits where that would overflow a finite x),
 *   FUSEML_SEG_LO        lo(x) = bf16(x - hi(x)), 0 for inf and NaN,
 *   FUSEML_SEG_HI_FINITE hi(x), with 0 for inf and NaN;
 * columns K..k_pad-1 are 0.  With A3 from FUSEML_SPLIT_A (hi|hf|lo) and B3
 * from FUSEML_SPLIT_B (hi|lo|hf), A3 . B3 = hi.hi + hf.lo + lo.hf: the cross
 * terms are finite, so inf and NaN reach the product only through hi.hi, as
 * fp32 gives them.  Needs k_pad % 8 == 0, k_pad >= K, ld_dst % 8 == 0,
 * ld_dst >= 3 k_pad and a 16-byte aligned dst.
 * Asynchronous on `stream`; 0 or a FUSEML_E* code.
 * ------------------------------------------------------------------------ */
#define FUSEML_SEG_HI 0u
#define FUSEML_SEG_LO 1u
#define FUSEML_SEG_HI_FINITE 2u
#define FUSEML_SPLIT_A (FUSEML_SEG_HI | (FUSEML_SEG_HI_FINITE << 2) | (FUSEML_SEG_LO << 4))
#define FUSEML_SPLIT_B (FUSEML_SEG_HI | (FUSEML_SEG_LO << 2) | (FUSEML_SEG_HI_FINITE << 4))
int fuseml_split_bf16x3(const float* src, int64_t rows, int64_t K, int64_t stride_r, int64_t stride_k, void* dst,
                        int64_t ld_dst, int64_t k_pad, uint32_t seg_codes, void* stream);

/* Measurement only (no reference counterpart; the reference's benchmark
 * prices against a spec table, benchmarks/bench_mlp_block.py:228-412): launch
 * `workgroups` workgroups of 4 waves, each wave issuing `iters` x 8 independent
 * v_mfma_f32_32x32x16_bf16 on random register operands and nothing else, on
 * `stream`.  FLOPs = workgroups * 4 * iters * 8 * 32768.  `sink` is a device
 * buffer of workgroups * 256 floats.  Timed by the caller, this is the bf16
 * MFMA rate the device sustains at its power-limited clock. */
int fuseml_mfma_peak_probe(int64_t iters, int32_t workgroups, float* sink, void* stream);

/* FUSEML_ABI_VERSION, sizeof(fuseml_gemm_desc) and sizeof(fuseml_mlp_desc),
 * for binding checks. */
int fuseml_abi_version(void);
size_t fuseml_desc_size(void);
size_t fuseml_mlp_desc_size(void);

#ifdef __cplusplus
}
#endif

#endif /* FUSEML_HIP_H_ */
