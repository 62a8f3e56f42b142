/*
 * mx355.h — C ABI of the MI355X (gfx950) batched decode step.
 *
 * Drop-in boundary for rust-mlx's decode hot path.  Every compute entry point
 * replaces one reference wrapper that today records a JIT Metal kernel through
 * `metal::Kernel::launch` (reference src/metal.rs:264-325) or a native MLX op;
 * the replaced interface is cited beside each declaration.
 *
 * Conventions (all entry points):
 *  - bf16 tensors travel as uint16_t bit patterns, row-major, caller-owned
 *    device memory.  Outputs are preallocated by the caller; nothing is
 *    allocated behind the caller's back except where a function says so.
 *  - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *    Launches are asynchronous; no entry point synchronises unless it says so.
 *  - Return MX_OK (0) or an error code; mx_last_error() returns the message of
 *    the most recent failure on the calling thread.  Unsupported geometry is an
 *    error (MX_EUNSUPPORTED): there is no silent fallback path.
 *  - Affine quantisation follows MLX's layout: value k of output row n sits at
 *    bit k*bits of the row's little-endian bitstream of uint32 words;
 *    w = scale[n][k/gs] * q + bias[n][k/gs].
 */
#ifndef MX355_H
#define MX355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mx_status {
  MX_OK = 0,
  MX_EINVAL = 1,        /* malformed arguments (shape, null pointer, range) */
  MX_EUNSUPPORTED = 2,  /* geometry this build has no kernel for */
  MX_EHIP = 3,          /* HIP runtime error */
  MX_ENOMEM = 4,        /* device allocation failed */
  MX_ESTATE = 5         /* engine / cache state violates a precondition */
} mx_status;

/* Affine-quantised weight matrix [n, k] in MLX layout (reference
 * src/weights.rs:102-108 `Linear` {weight, scales, biases, quant}). */
typedef struct mx_qweight {
  const uint32_t* codes;   /* [n, k*bits/32] */
  const uint16_t* scales;  /* bf16 [n, k/group_size] */
  const uint16_t* biases;  /* bf16 [n, k/group_size] */
  int32_t n;
  int32_t k;
  int32_t bits;        /* 4, 5, 6 or 8 */
  int32_t group_size;  /* 32, 64 or 128 */
} mx_qweight;

/* ---- errors / version -------------------------------------------------- */
const char* mx_last_error(void);
int32_t mx_abi_version(void);

/* ---- device plumbing used by hosts and tests (no reference counterpart:
 *      MLX owns memory in the reference) ---------------------------------- */
mx_status mx_malloc(void** ptr, size_t bytes);
mx_status mx_free(void* ptr);
mx_status mx_memcpy_htod(void* dst, const void* src, size_t bytes);
mx_status mx_memcpy_dtoh(void* dst, const void* src, size_t bytes);
mx_status mx_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream);
mx_status mx_memset(void* dst, int value, size_t bytes, void* stream);
mx_status mx_stream_create(void** stream);
mx_status mx_stream_destroy(void* stream);
mx_status mx_stream_sync(void* stream);
mx_status mx_device_sync(void);
mx_status mx_event_create(void** event);
mx_status mx_event_destroy(void* event);
mx_status mx_event_record(void* event, void* stream);
mx_status mx_event_elapsed_ms(void* start, void* stop, float* ms);
/* Fill `count` bf16 values with a seeded counter-based generator.
 * dist 0: U(a, b); dist 1: N(0,1)*a + b (Irwin-Hall(12) approximation). */
mx_status mx_fill_bf16(uint16_t* dst, size_t count, uint64_t seed, int32_t dist,
                       float a, float b, void* stream);
/* Fill `count` random codes of `bits` bits, uniform over [0, 2^bits), packed
 * in MLX layout as rows of `k` values (count must be rows*k). */
mx_status mx_fill_codes(uint32_t* dst, int64_t rows, int32_t k, int32_t bits,
                        uint64_t seed, void* stream);
/* Evaluate the library's deterministic scalar functions elementwise on fp32
 * (op 0 exp, 1 log1p, 2 sigmoid, 3 softplus, 4 round-to-bf16), so tests can
 * pin the device arithmetic against a CPU restatement. */
mx_status mx_eval_math(int32_t op, const float* in, float* out, int64_t n, void* stream);

/* ---- A3: affine quantised matvec / skinny GEMM --------------------------
 * y[m, n] = sum_k x[m, k] * (s[n, k/gs] * q[n, k] + b[n, k/gs]), 1 <= m <= 8.
 * Replaces qmv_kernel::project / project_unfiltered (reference
 * src/qmv_kernel.rs:49-180, kernels/verify_qmv.{h,metal}) and the native
 * `quantized_matmul` / `gather_qmm` row paths of Linear::forward_rows
 * (src/weights.rs:111-202).  Requires k % 32 == 0 and k % group_size == 0. */
mx_status mx_qmv(const mx_qweight* w, const uint16_t* x, int32_t m, uint16_t* y,
                 void* stream);

/* ---- A4: affine dequantisation of selected rows (embedding) --------------
 * out[i, :] = bf16(s * q + b) of row ids[i].  Replaces Linear::embedding
 * (src/weights.rs:203-226: take_axis + ops::dequantize). */
mx_status mx_dequant_rows(const mx_qweight* w, const uint32_t* ids, int32_t count,
                          uint16_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MX355_H */
