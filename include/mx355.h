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

/* A bank of equally shaped expert matrices stored back to back (MLX
 * SwitchLinear layout, reference src/hybrid.rs:129-143 `switch_mlp.*_proj`):
 * codes [experts, n, k*bits/32], scales/biases bf16 [experts, n, k/group_size]. */
typedef struct mx_qbank {
  const uint32_t* codes;
  const uint16_t* scales;
  const uint16_t* biases;
  int32_t experts;
  int32_t n;
  int32_t k;
  int32_t bits;
  int32_t group_size;
} mx_qbank;

/* GatedDeltaNet geometry (reference src/hybrid.rs:12-38 HybridConfig
 * linear_num_{key,value}_heads, linear_{key,value}_head_dim, linear_conv_kernel_dim). */
typedef struct mx_gdn_dims {
  int32_t hk;      /* key heads */
  int32_t hv;      /* value heads (a multiple of hk) */
  int32_t dk;      /* key head dim (128) */
  int32_t dv;      /* value head dim (128) */
  int32_t conv_k;  /* depthwise conv taps */
} mx_gdn_dims;

/* Synthetic hybrid model (BASELINE config 3 / 4): `layers` layers, layer i a
 * gated full-attention layer when i % attn_every == attn_every - 1, else a
 * GatedDeltaNet layer; every layer has attention and MLP hyper-connections
 * (hc streams, low rank hc_rank) and a sparse MoE with one shared expert;
 * a mixer hyper-connection and a greedy vocabulary head close the stack
 * (reference src/hybrid.rs:12-38 HybridConfig, 500-685 HybridModel).
 * Weights are random affine-quantised tensors drawn from `seed`. */
#define MX_MAX_LAYERS 128
typedef struct mx_model_config {
  int32_t hidden;
  int32_t layers;
  int32_t attn_every;
  int32_t vocab;
  int32_t hc;
  int32_t hc_rank;
  int32_t gdn_hk, gdn_hv, gdn_dk, gdn_dv, conv_k;
  int32_t heads, kv_heads, head_dim, rotary_dim;
  float rope_theta;
  float rms_eps;
  int32_t experts, top_k, moe_inter, shared_inter;
  int32_t bits;        /* projections and expert gate/up */
  int32_t down_bits;   /* expert and shared-expert down */
  int32_t embed_bits, head_bits, group_size;
  int32_t mixed_bits;  /* nonzero: per-layer bits drawn from {4,5,6,8} by seed (config 4) */
  int32_t max_slots, max_context, max_verify;
  uint64_t seed;
  int32_t mtp;         /* nonzero: one MTP draft layer for speculative generation (config 4) */
  /* Per-layer widths read from a checkpoint's per-module quantization
   * (src/weights.rs:70-90), 0 = not given.  Entry 2 i: layer i's projections,
   * hyper-connections, router and expert / shared-expert gate and up; entry
   * 2 i + 1: its expert and shared-expert down.  Index `layers` is the MTP
   * draft layer (its fc_embedding / fc_hidden and draft mixer take entry
   * 2 layers).  A nonzero entry overrides bits / down_bits and the
   * mixed_bits draw for that layer. */
  uint8_t layer_widths[2 * (MX_MAX_LAYERS + 1)];
} mx_model_config;

typedef struct mx_engine mx_engine;

/* Speculative generation counters (mx_engine_generate). */
typedef struct mx_generate_stats {
  int32_t rounds;    /* verify blocks run */
  int32_t drafted;   /* draft tokens proposed */
  int32_t accepted;  /* draft tokens accepted */
} mx_generate_stats;

/* What one profiled decode step measured (HIP events on the engine stream)
 * and its algorithmic HBM bytes (each distinct weight, state and KV byte once). */
typedef struct mx_step_profile {
  int32_t rows;
  int32_t layers;             /* MoE layers profiled */
  double distinct_experts;    /* routed experts touched, summed over layers */
  double gate_up_ms;          /* expert gate/up kernel time, summed over layers */
  double down_ms;             /* expert down kernel time, summed over layers */
  double gate_up_bytes;       /* algorithmic bytes of those launches */
  double down_bytes;
  double step_ms;             /* the whole (eager, instrumented) step */
  double step_bytes;          /* algorithmic bytes of the whole step */
} mx_step_profile;

/* Expert kernels of every MoE layer timed back to back (HIP events): totals
 * over `launches` launches of each kernel and their algorithmic bytes. */
typedef struct mx_expert_timing {
  int32_t launches;
  double distinct_experts;  /* routed experts of the routing used (per launch) */
  double gate_up_ms;
  double gate_up_bytes;
  double down_ms;
  double down_bytes;
} mx_expert_timing;

/* ---- errors / version -------------------------------------------------- */
const char* mx_last_error(void);
int32_t mx_abi_version(void);
/* Tokens per chunk of mx_engine_prefill_chunked (and of mx_engine_generate's
 * chunked prompt): the most rows any matrix-core entry takes.  No reference
 * counterpart (speculative::prepare takes the chunk as an argument). */
int32_t mx_prefill_chunk_tokens(void);

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

/* ---- A3/A15: the same projection on the matrix cores --------------------
 * y = x . dequant(W)^T for 1 <= m <= 512 rows with v_mfma_f32_16x16x32_bf16.
 * Up to 16 rows the codes enter as exact bf16 integers and each 64-value
 * group's fp32 partial is scaled in registers; beyond 16 rows a GEMM stages
 * 128-row blocks of x in LDS and dequantises each workgroup's weight rows
 * there as w = s q + b split into two bf16 parts (hi + lo within 2^-17 of w).
 * Results equal mx_qmv's up to fp32 summation order and that split (the
 * north star's tolerance, not bit for bit).  Requires group_size 64 and
 * k <= 8192.  Deterministic: a workgroup splits k among its own waves and adds
 * their sums in a fixed order.  The MFMA verify/prefill slot of the reference
 * (matrix_kernel::project, src/matrix_kernel.rs:113-254,
 * kernels/matrix_packed.metal). */
mx_status mx_qmm(const mx_qweight* w, const uint16_t* x, int32_t m, uint16_t* y, void* stream);
/* ---- A3/A15: the exact-integer projection on the int8 matrix cores -------
 * y[m, n] = bf16 of the affine projection computed exactly: per 64-value
 * group, x is put on an integer grid anchored at the group's largest bf16
 * exponent (X = trunc(x 2^(156 - Eb)), |X| < 2^30), P = sum X q and
 * Q = sum X are exact integer sums (signed int8 digits of X against the
 * codes on v_mfma_i32_16x16x64_i8), v = fma(P, s, Q b) 2^(Eb - 156) in fp64,
 * groups added in fp64 in order within slices of two consecutive groups
 * (the last slice of an odd count holds one), the slice sums in order, one
 * rounding to fp32, then bf16.  Bit-exact with the CPU oracle (oracle/xq.c);
 * no result depends on the number of rows or the launch shape.  1 <= m <= 8,
 * group_size 64, k a multiple of 64 up to 512, or 1024, 2048, 4096, 8192.
 * The product path of the
 * decode engine's exact mode.  Replaces the same reference interfaces as
 * mx_qmv (src/qmv_kernel.rs:49-180, kernels/verify_qmv.{h,metal}: the
 * affine formula of verify_qmv.h:112). */
mx_status mx_xq(const mx_qweight* w, const uint16_t* x, int32_t m, uint16_t* y, void* stream);
/* mx_qmm_conv: mx_qmm (4-bit, 1..8 rows, one token per row) with the GDN
 * causal conv fused into its output: columns below conv_channels are conv
 * channels, convolved with the slot's cached window (conv_state bf16 [slots,
 * conv_k-1, conv_channels], updated in place; conv_w fp32 [conv_k,
 * conv_channels]; conv_k in 2..4) and written as bf16(silu(bf16(conv))) to
 * conv_out — mx_gdn_conv's arithmetic on the projection's bf16 outputs, bit
 * for bit; columns from conv_channels on go to y.  Rows' slots must be
 * distinct.  Replaces the in_proj + decode_conv pair of Gdn::forward
 * (src/hybrid.rs:374-400, src/compiled.rs:88-95). */
mx_status mx_qmm_conv(const mx_qweight* w, const uint16_t* x, int32_t m, int32_t conv_channels,
                      int32_t conv_k, const int32_t* slots, uint16_t* conv_state,
                      const float* conv_w, uint16_t* conv_out, int64_t conv_stride, uint16_t* y,
                      int64_t y_stride, void* stream);

/* ---- A4: affine dequantisation of selected rows (embedding) --------------
 * out[i, :] = bf16(s * q + b) of row ids[i].  Replaces Linear::embedding
 * (src/weights.rs:203-226: take_axis + ops::dequantize). */
mx_status mx_dequant_rows(const mx_qweight* w, const uint32_t* ids, int32_t count,
                          uint16_t* out, void* stream);

/* ---- A6: MoE routing tail -----------------------------------------------
 * Per row: softmax of `experts` bf16 logits (fp32), bf16 gates, top_k by the
 * (bf16 gate, expert id) key — ids[row, k-1] is the largest, as the reference
 * slices the last k of an ascending sort — bf16 renormalised scores, and
 * factor = bf16 sigmoid(shared_logit).  Rows are `logit_stride` /
 * `shared_stride` elements apart, so both may point into one fused projection
 * output.  Replaces moe_route::tail (src/moe_route.rs:25-70,
 * kernels/moe_route_tail.{h,metal}) and the native softmax / argpartition /
 * renormalise of MoE::parts (src/hybrid.rs:217-222, 284). */
mx_status mx_moe_route(const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
                       int64_t shared_stride, int32_t rows, int32_t experts, int32_t top_k,
                       uint32_t* ids, uint16_t* scores, uint16_t* factor, void* stream);

/* ---- A7+A8: gathered expert MLPs ------------------------------------------
 * For every row r and slot j < top_k, expert e = ids[r, j]:
 *   h = bf16(bf16(silu(bf16(gate_e x))) * bf16(up_e x)),
 *   partial[r, j] = bf16(bf16(down_e h) * scores[r, j]);
 * slot top_k holds the shared expert's bf16(down(h)), unweighted.
 * partial is bf16 [rows, top_k + 1, hidden]; workspace holds
 * mx_moe_workspace_bytes(rows, top_k, max(inter, shared inter)) bytes.
 * Routes naming the same expert are served together, so each selected
 * expert's weights stream once per call.  ids are expert indices below the
 * banks' expert count (at most 1024), distinct within a row, as a top-k
 * routing gives them.  Replaces moe_kernel::gate_up
 * (src/moe_kernel.rs:10-118), the gather_qmm gate/up/down of MoE::parts
 * (src/hybrid.rs:245-271), moe_down::reduce's expert QMV + score product
 * (src/moe_down.rs:34-137) and the shared Mlp (src/dense.rs:292-298). */
size_t mx_moe_workspace_bytes(int32_t rows, int32_t top_k, int32_t inter);
mx_status mx_moe_experts(const uint16_t* x, const uint32_t* ids, const uint16_t* scores,
                         int32_t rows, int32_t top_k, const mx_qbank* gate, const mx_qbank* up,
                         const mx_qbank* down, const mx_qweight* shared_gate,
                         const mx_qweight* shared_up, const mx_qweight* shared_down,
                         void* workspace, uint16_t* partial, void* stream);
/* mx_moe_experts on the matrix cores (same contract, fp32 summation order
 * within tolerance of the exact kernels), for 1..512 rows: beyond eight rows
 * (a prefill chunk) the routes are grouped by expert into 16-route matrix-core
 * tiles, each expert's weights read once per 16 of its routes, and the banks
 * may hold at most 1023 experts. */
mx_status mx_moe_experts_mfma(const uint16_t* x, const uint32_t* ids, const uint16_t* scores,
                              int32_t rows, int32_t top_k, const mx_qbank* gate,
                              const mx_qbank* up, const mx_qbank* down,
                              const mx_qweight* shared_gate, const mx_qweight* shared_up,
                              const mx_qweight* shared_down, void* workspace, uint16_t* partial,
                              void* stream);
/* The routing tail and the matrix-core experts in one call: mx_moe_route's
 * contract for ids / scores / factor (bit-identical results), then
 * mx_moe_experts_mfma's for partial.  With 512 routed experts and hidden 2048
 * the expert gate/up kernel routes its rows itself, saving the routing launch.
 * Replaces moe_route::tail (src/moe_route.rs:25-70) followed by the expert
 * MLPs of MoE::parts (src/hybrid.rs:217-271). */
mx_status mx_moe_routed_experts_mfma(const uint16_t* logits, int64_t logit_stride,
                                     const uint16_t* shared_logit, int64_t shared_stride,
                                     int32_t experts, const uint16_t* x, int32_t rows,
                                     int32_t top_k, const mx_qbank* gate, const mx_qbank* up,
                                     const mx_qbank* down, const mx_qweight* shared_gate,
                                     const mx_qweight* shared_up, const mx_qweight* shared_down,
                                     void* workspace, uint32_t* ids, uint16_t* scores,
                                     uint16_t* factor, uint16_t* partial, void* stream);
/* The whole MoE sublayer after the router projection, in two launches:
 * mx_moe_routed_experts_mfma, then mx_moe_reduce_hc_epilogue(partial, factor,
 * residual = out = hcs, gate = hc_gate), with the down projection, the slot
 * sum and the stream write in one kernel (ids / scores / factor / hcs
 * bit-identical to those two calls).  hc == 4, top_k <= 15 and 512-deep
 * experts (routed and shared) only; MX_EUNSUPPORTED otherwise.  hcs:
 * [rows][4][hidden] residual streams, updated in place; hc_gate: [rows][4].
 * workspace: mx_moe_workspace_bytes.  Replaces moe_route::tail
 * (src/moe_route.rs:25-70), the expert MLPs and slot sum of MoE::parts
 * (src/hybrid.rs:217-271, kernels/moe_down_tail.metal:83-99) and
 * moe_epilogue::apply (src/moe_epilogue.rs:17-73). */
mx_status mx_moe_routed_experts_hc_mfma(
    const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
    int64_t shared_stride, int32_t experts, const uint16_t* x, int32_t rows, int32_t top_k,
    int32_t hc, const mx_qbank* gate, const mx_qbank* up, const mx_qbank* down,
    const mx_qweight* shared_gate, const mx_qweight* shared_up, const mx_qweight* shared_down,
    void* workspace, uint32_t* ids, uint16_t* scores, uint16_t* factor, const uint16_t* hc_gate,
    uint16_t* hcs, void* stream);
/* routed[r] = bf16 sum of partial[r, 0..top_k-1] in the reference's slot
 * order (kernels/moe_down_tail.h:20, moe_down_tail.metal:83-99). */
mx_status mx_moe_reduce(const uint16_t* partial, int32_t rows, int32_t top_k, int32_t hidden,
                        uint16_t* routed, void* stream);

/* ---- A3: hyper-connection input projection on the matrix cores ----------
 * mixed[r] = mean_s sigmoid(up_s(lo)) * bf16(norm_s(h[r]) (scale_s + 1)), with
 * lo = silu(down(norm(h)) / hc) over the first `rank` down rows and inj =
 * 2 sigmoid(down(norm(h)) / hc) over the hc inject rows (down rows rank ..
 * rank + hc - 1, when present): the per-stream RMS norm is factored out of
 * the down projection.  Matrix-core sums and the hardware exp2 / reciprocal /
 * rsqrt (the fast mode's arithmetic, within the north star's tolerance of the
 * fixed-order path), in two launches.  workspace: mx_hc_workspace_bytes(down
 * rows).  Replaces HyperConnection::forward_reference (src/hybrid.rs:78-99)
 * and compiled::activate / injection / mix (src/compiled.rs:46-86). */
size_t mx_hc_workspace_bytes(int32_t n_down);
mx_status mx_hc_forward_mfma(const mx_qweight* down, const mx_qweight* up, const uint16_t* h,
                             const uint16_t* scale, int32_t rows, int32_t hc, int32_t hidden,
                             int32_t rank, float eps, void* workspace, uint16_t* mixed,
                             uint16_t* inj, void* stream);

/* ---- A9: MoE hyper-connection epilogue ------------------------------------
 * out[r, s, c] = bf16(residual[r, s, c] + bf16(bf16(routed + bf16(shared * factor[r]))
 *                                               * gate[r, s]))
 * Replaces moe_epilogue::apply (src/moe_epilogue.rs:17-73,
 * kernels/moe_hc_epilogue.metal) / HyperConnection::write after MoE::forward
 * (src/hybrid.rs:100-105, 292-307).  out may alias residual. */
mx_status mx_moe_hc_epilogue(const uint16_t* routed, const uint16_t* shared,
                             const uint16_t* factor, const uint16_t* residual,
                             const uint16_t* gate, int32_t rows, int32_t hc, int32_t hidden,
                             uint16_t* out, void* stream);
/* mx_moe_reduce followed by mx_moe_hc_epilogue with shared = partial[r, top_k],
 * in one pass (same bits). */
mx_status mx_moe_reduce_hc_epilogue(const uint16_t* partial, const uint16_t* factor,
                                    const uint16_t* residual, const uint16_t* gate, int32_t rows,
                                    int32_t top_k, int32_t hc, int32_t hidden, uint16_t* out,
                                    void* stream);

/* ---- A14: greedy head ------------------------------------------------------
 * tokens[m] = argmax_n bf16(head_n . x_m): largest value, lowest id on ties,
 * NaN never wins, 0 when nothing exceeds -inf.  Logits are reduced on chip
 * and never written.  workspace: mx_head_workspace_bytes(n, k, m) bytes.
 * Replaces greedy_head::project (src/greedy_head.rs:40-126,
 * kernels/greedy_{head,reduce}.metal) and the default
 * argmax_axis(head.forward_rows(x)) (src/bin/batch-bench.rs:118-120). */
size_t mx_head_workspace_bytes(int32_t n, int32_t k, int32_t m);
mx_status mx_head_argmax(const mx_qweight* w, const uint16_t* x, int32_t m, uint32_t* tokens,
                         void* workspace, void* stream);
/* mx_head_argmax for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): no
 * workspace argument and no allocation of any kind.  The partials live in a
 * static device array of 1 MiB per GPU, held until the process ends; the
 * call returns MX_EUNSUPPORTED when mx_head_workspace_bytes(n, k, m) exceeds
 * mx_head_noalloc_max_bytes() (1 MiB: a 262144-row head at k >= 2048 and
 * m = 8).  Every call on one GPU shares that array: calls that overlap on
 * one GPU (different streams or threads) race.  Same tokens as
 * mx_head_argmax bit for bit (same kernels).  No counterpart in the
 * reference: an addition for callers that cannot allocate. */
size_t mx_head_noalloc_max_bytes(void);
mx_status mx_head_argmax_noalloc(const mx_qweight* w, const uint16_t* x, int32_t m,
                                 uint32_t* tokens, void* stream);
/* mx_head_argmax with the head projection on the matrix cores (fp32
 * summation order differs from the exact kernel, so near-ties may resolve
 * differently; the selection rule is the same).  Requires group_size 64,
 * k % 512 == 0 and k <= 2048; same workspace size. */
mx_status mx_head_argmax_mfma(const mx_qweight* w, const uint16_t* x, int32_t m,
                              uint32_t* tokens, void* workspace, void* stream);
/* argmax over bf16 logits [rows, n] with the same rule (MLX argmax_axis). */
mx_status mx_argmax_bf16(const uint16_t* logits, int32_t rows, int32_t n, uint32_t* tokens,
                         void* stream);

/* ---- A10/A11/A12: GatedDeltaNet -------------------------------------------
 * Rows are `groups` sequences of `t` consecutive tokens (row = g*t + i);
 * slots[g] (device int32) selects the group's cached conv window and state.
 *
 * mx_gdn_conv: causal depthwise conv of the cached window and the new qkv
 * rows, then SiLU; out[row] = bf16(silu(bf16(sum_j x_j * w[j]))) per channel.
 * conv_state bf16 [slots, conv_k-1, channels] is updated in place; conv_w is
 * fp32 [conv_k, channels]; window_history (nullable) receives the full window
 * bf16 [groups, conv_k-1+t, channels] for verify rollback.  Replaces
 * compiled::decode_conv + silu and the conv-state slice of
 * Gdn::forward_reference (src/compiled.rs:88-95, src/hybrid.rs:374-400). */
mx_status mx_gdn_conv(const uint16_t* qkv, int64_t row_stride, int32_t groups, int32_t t,
                      const int32_t* slots, uint16_t* conv_state, const float* conv_w,
                      int32_t channels, int32_t conv_k, uint16_t* out, int64_t out_stride,
                      uint16_t* window_history, void* stream);
/* mx_gdn_recurrence: q/k L2 norm (q scaled by dk^-1/2), beta = sigmoid(b),
 * g = exp(-exp(a_log) * softplus(a + dt_bias)), the delta rule on the fp32
 * state, and the gated RMS norm y = rms_norm(o, norm_w, eps) * sigmoid(z).
 * conv_out rows hold [q (hk*dk) | k (hk*dk) | v (hv*dv)]; z, a, b rows are
 * zab_stride elements apart.  state fp32 [slots, hv, dk, dv] is updated in
 * place (note: dk-major, the transpose of MLX's [B, Hv, Dv, Dk]); history
 * (nullable) receives the state after every token, fp32 [groups*t, hv, dk, dv].
 * y is bf16 [groups*t, hv*dv].  Replaces gdn_kernel::recurrent /
 * recurrent_with_history (src/gdn_kernel.rs:7-142, kernels/gated_delta{,_history}.metal)
 * with the surrounding ops of Gdn::forward_reference (src/hybrid.rs:401-453). */
mx_status mx_gdn_recurrence(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                            const uint16_t* a, const uint16_t* b, int64_t zab_stride,
                            const float* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                            float eps, const mx_gdn_dims* dims, int32_t groups, int32_t t,
                            const int32_t* slots, float* state, float* history, uint16_t* y,
                            void* stream);

/* ---- A16: unquantised bf16 GEMV for short rows ------------------------------
 * mx_gemv_bf16: y[r, o] = bf16(sum_k w[o, k] x[r, k]) for rows 1..8, w bf16
 * [n, k] row-major, x bf16 [rows, k], k % 128 == 0.  Each row keeps the order
 * of a single-row call (32 partial sums over 128-value blocks, fma per
 * product, then a shuffle-down tree 16, 8, 4, 2, 1), so batching never
 * changes a row's result.  Replaces gemv_kernel::project
 * (src/gemv_kernel.rs:30-90, kernels/shared_gemv.metal). */
mx_status mx_gemv_bf16(const uint16_t* w, int32_t n, int32_t k, const uint16_t* x, int32_t rows,
                       uint16_t* y, void* stream);

/* ---- gated full attention (decode / verify rows) ---------------------------
 * mx_attn_decode: scaled dot-product attention of each row's normalised and
 * rotated q heads (q bf16 [rows, heads, head_dim]) over the cached positions
 * 0..pos[r] of its slot, then the output gate:
 *   out[r, h] = bf16(bf16(softmax(q k^T / sqrt(head_dim)) v) * sigmoid(gate[r, h]))
 * with gate[r, h] = qkv[r * qkv_stride + h * 2 * head_dim + head_dim ..] (the
 * projected rows, [heads][q | gate][head_dim] per row).  Caches are bf16
 * [slot][kv_head][max_ctx][head_dim] with slot_stride elements between slots.
 * flags bit 0: the matrix-core kernel (fp32 sums in another order, within
 * tolerance) instead of the fixed-order kernel that the CPU oracle restates.
 * flags bit 1: the matrix-core prefill form (within the same tolerance) for
 * the rows of one slot's prompt chunk: blocks of 8 * 16 / (heads / kv_heads)
 * rows share each 64-key tile, with partials per 256-key split; every row
 * must name the same slot; needs head_dim 128 or 256 and 2, 4 or 8 q heads
 * per kv head (MX_EUNSUPPORTED otherwise).
 * workspace: mx_attn_workspace_bytes(rows, heads, head_dim, max_ctx) bytes.
 * Replaces the fast::scaled_dot_product_attention call and output gate of
 * Attention::forward_selection (src/dense.rs:139-270, 249-256). */
typedef struct mx_attn_dims {
  int32_t heads;     /* q heads */
  int32_t kv_heads;  /* heads of the cache (heads is a multiple) */
  int32_t head_dim;  /* <= 256, a multiple of 8 */
  int32_t max_ctx;   /* positions per (slot, kv head) in the cache */
  int64_t slot_stride;
} mx_attn_dims;
size_t mx_attn_workspace_bytes(int32_t rows, int32_t heads, int32_t head_dim, int32_t max_ctx);
mx_status mx_attn_decode(const uint16_t* q, const uint16_t* qkv, int64_t qkv_stride, int32_t rows,
                         const int32_t* slots, const int32_t* pos, const uint16_t* k_cache,
                         const uint16_t* v_cache, const mx_attn_dims* dims, int32_t flags,
                         void* workspace, uint16_t* out, void* stream);

/* mx_gdn_recurrence_fast: mx_gdn_recurrence's contract (groups of t tokens,
 * optional per-token history) with the matrix-core engine's fast-mode
 * arithmetic: the same fp32 delta rule, hardware exp2 / log2 / reciprocal /
 * rsqrt for beta, the decay, the L2 and RMS norms and the gate, within the
 * north star's tolerances of the fixed-order kernel.  Every token's
 * arithmetic is independent of t, so a t-token verify block gives the bits
 * of t one-token calls (the decode step) and greedy acceptance stays
 * lossless.  Replaces the same reference interfaces as mx_gdn_recurrence
 * (src/gdn_kernel.rs:7-142, src/hybrid.rs:401-453). */
mx_status mx_gdn_recurrence_fast(const uint16_t* conv_out, int64_t conv_stride,
                                 const uint16_t* z, const uint16_t* a, const uint16_t* b,
                                 int64_t zab_stride, const float* a_log, const uint16_t* dt_bias,
                                 const uint16_t* norm_w, float eps, const mx_gdn_dims* dims,
                                 int32_t groups, int32_t t, const int32_t* slots, float* state,
                                 float* history, uint16_t* y, void* stream);

/* ---- A1/A17/A18: the decode engine ---------------------------------------
 * Owns the model weights, a slot arena of caches (GDN state + conv window, KV)
 * and one HIP stream; every call is synchronous (one sync per step, like the
 * reference's eval) and must come from the thread that created the engine.
 *
 * mx_engine_decode_batch: one token for each of `rows` (1..8) distinct slots
 * that sit at the same offset; writes each row's greedy next token and
 * advances the slots.  Replaces HybridModel::decode_batch (src/batching.rs:34-170);
 * unequal offsets are rejected with MX_ESTATE as in batching.rs:47-53, and
 * out-of-vocabulary tokens with MX_EINVAL.
 * mx_engine_decode_rows: the same step without the equal-offset rule (each
 * row attends to its own context), for ragged continuous batching.
 * mx_engine_prefill: feeds `count` tokens to one slot in chunks of up to 8
 * (speculative::prepare, src/speculative.rs:38-68); *next = greedy token after
 * the last one.
 * mx_engine_verify / mx_engine_commit: an MTP verify block of 1..max_verify
 * tokens (argmax at every position into `argmax`), then accept the first
 * `keep` (0..count) of them (generate_prepared + HybridCache::commit_verified,
 * src/speculative.rs:370-416, src/hybrid.rs:699-759).
 * mx_engine_clone_slot: copy one slot's caches to another (prefix reuse,
 * PrefixCache src/speculative.rs:70-117). */
mx_status mx_engine_create(const mx_model_config* cfg, mx_engine** out);
mx_status mx_engine_destroy(mx_engine* e);
mx_status mx_engine_reset_slot(mx_engine* e, int32_t slot);
mx_status mx_engine_clone_slot(mx_engine* e, int32_t src, int32_t dst);
int32_t mx_engine_offset(mx_engine* e, int32_t slot);
/* 1 when a failed step left the slot's caches partly updated (GDN state and
 * conv windows are advanced in place; the reference's lazy evaluation never
 * writes a cache before the whole step succeeded, src/batching.rs:136-137):
 * every step, prefill, verify, commit and clone from that slot then returns
 * MX_ESTATE until mx_engine_reset_slot or mx_engine_clone_slot (into it)
 * replaces its caches.  A failed verify block restores its snapshot instead,
 * so its slot stays usable.  0 otherwise, -1 for a bad slot. */
int32_t mx_engine_slot_failed(mx_engine* e, int32_t slot);
/* Test hook with no reference counterpart: the engine's next step stops with
 * MX_EHIP after launching `after_layers` layers (eager), as a launch that
 * fails mid-step would, so failure handling can be tested without a device
 * fault.  0 disarms. */
mx_status mx_engine_inject_failure(mx_engine* e, int32_t after_layers);
mx_status mx_engine_decode_batch(mx_engine* e, const int32_t* slots, const uint32_t* tokens,
                                 int32_t rows, uint32_t* next);
mx_status mx_engine_decode_rows(mx_engine* e, const int32_t* slots, const uint32_t* tokens,
                                int32_t rows, uint32_t* next);
/* mx_engine_decode_batch that also returns what HybridModel::decode_batch
 * returns (src/batching.rs:34-170, `Ok((logits, hidden))` at 169): the
 * step's bf16 logits [rows, vocab] and final hidden streams bf16
 * [rows, hc * hidden] (before the mixer), written to caller-owned device
 * buffers; either may be NULL.  `next` holds the greedy tokens, which are
 * the argmax of these logits (largest, lowest id on ties).  Same equal-offset
 * rule as mx_engine_decode_batch. */
mx_status mx_engine_decode_batch_outputs(mx_engine* e, const int32_t* slots,
                                         const uint32_t* tokens, int32_t rows, uint32_t* next,
                                         uint16_t* logits, uint16_t* hidden);
mx_status mx_engine_prefill(mx_engine* e, int32_t slot, const uint32_t* tokens, int32_t count,
                            uint32_t* next);
/* mx_engine_prefill_chunked: the same contract in chunks of up to 512 tokens
 * (mx_prefill_chunk_tokens; speculative::prepare's loop,
 * src/speculative.rs:38-68, one model forward per chunk: the reference calls
 * it with 128, and a chunk four times longer reads each expert's weights once
 * per 512 prompt tokens instead of once per 128).  A chunk's projections run as a
 * matrix-core GEMM over all of its rows, its routes grouped by expert into
 * 16-route tiles (each expert's weights read once per 16 of its routes), its
 * attention is causal over the chunk, and its GDN layers take the chunked
 * scan (64-token sub-chunks on the fp32 matrix cores); *next comes from the
 * last row's logits.  The matrix-core arithmetic agrees with
 * mx_engine_prefill's exact kernels to fp32 summation order, not bit for bit
 * (whatever mx_engine_set_flags chose for decode steps).  A failure marks the
 * slot failed (see mx_engine_slot_failed); MX_ESTATE when the tokens exceed
 * the slot's remaining context. */
mx_status mx_engine_prefill_chunked(mx_engine* e, int32_t slot, const uint32_t* tokens,
                                    int32_t count, uint32_t* next);
mx_status mx_engine_verify(mx_engine* e, int32_t slot, const uint32_t* tokens, int32_t count,
                           uint32_t* argmax);
mx_status mx_engine_commit(mx_engine* e, int32_t slot, int32_t keep);
/* Greedy generation from an empty slot: prefill `prompt`, then emit up to
 * `max_tokens` tokens (the first is the prefill's greedy token).  depth 0:
 * one decode step per token.  depth 1..min(7, max_verify - 1): MTP
 * speculation (the model needs mtp = 1): the draft layer proposes `depth`
 * tokens, a verify block accepts the matching prefix plus the target's next
 * token, and the draft layer is resynchronised on the target's hidden states;
 * the tokens equal the depth-0 ones wherever verify and decode agree (always
 * in exact mode).  Replaces speculative::generate_prepared
 * (src/speculative.rs:225-483) with the draft model Mtp::forward
 * (src/mtp.rs:72-127), default policies (full-vocabulary greedy draft head,
 * fixed depth, no EOS).  drafts (optional, max_tokens * depth entries): every
 * round's drafted tokens in order (stats->drafted of them), like the
 * reference's recorded draft tokens.  With flag bit 10 (mx_engine_set_flags)
 * the prompt is prefilled as mx_engine_prefill_chunked does, the draft
 * layer's pass over the prompt running chunk by chunk on the same kernels. */
mx_status mx_engine_generate(mx_engine* e, int32_t slot, const uint32_t* prompt,
                             int32_t n_prompt, int32_t max_tokens, int32_t depth,
                             uint32_t* tokens, int32_t* n_tokens, mx_generate_stats* stats,
                             uint32_t* drafts);
/* Test/inspection hooks: flags (bit 0: also write bf16 logits of each step;
 * bit 1: run eagerly instead of replaying captured HIP graphs; bit 2: exact
 * mode, every projection on the fixed-order kernels that the CPU oracle
 * reproduces bit for bit, instead of the matrix-core kernels; bits 3..9, a
 * diagnostic mask of the components that run exact while the rest stays on
 * the matrix cores: 3 hyper-connections, 4 GDN projections, 5 GDN
 * recurrence, 6 attention projections, 7 attention core, 8 router + routing
 * + experts, 9 vocabulary head); bit 10: mx_engine_generate prefills its
 * prompt in matrix-core chunks), and reads of
 * the last step's "hidden" (bf16 [rows, hc*hidden]) / "logits" (bf16
 * [rows, vocab]) or of any named weight/cache tensor into host memory. */
mx_status mx_engine_set_flags(mx_engine* e, int32_t flags);
/* Measurement hook (no reference counterpart): gives `slot` a synthetic
 * context of `length` positions (random K/V, GDN state and conv window drawn
 * from `seed`) in place of a prefill; decode cost depends on the length only. */
mx_status mx_engine_fill_slot(mx_engine* e, int32_t slot, int32_t length, uint64_t seed);
/* One decode step like mx_engine_decode_rows, run eagerly with the expert
 * kernels timed per layer (no reference counterpart: the reference could not
 * attribute GPU time per kernel, docs/performance.md:41). */
mx_status mx_engine_profile_step(mx_engine* e, const int32_t* slots, const uint32_t* tokens,
                                 int32_t rows, uint32_t* next, mx_step_profile* out);
/* Measurement hook (no reference counterpart): one MTP verify block like
 * mx_engine_verify (a commit must follow, as after mx_engine_verify), run
 * eagerly with the expert kernels timed per layer; out->step_bytes holds the
 * block's algorithmic bytes (weights outside the expert banks, the routed
 * experts the block touches, the GDN state read once and written after every
 * token, conv windows, the KV positions up to the block's last). */
mx_status mx_engine_profile_verify(mx_engine* e, int32_t slot, const uint32_t* tokens,
                                   int32_t count, uint32_t* argmax, mx_step_profile* out);
/* Measurement hook (no reference counterpart): algorithmic bytes of one MTP
 * draft step of one row at cache position `pos` (the draft layer outside its
 * expert banks, top_k of its experts, one embedding row, the greedy head, the
 * draft layer's KV positions).  MX_EUNSUPPORTED without an MTP layer. */
mx_status mx_engine_draft_bytes(mx_engine* e, int32_t pos, double* bytes);
/* Measurement hook (no reference counterpart): the expert gate/up kernels of
 * all MoE layers launched back to back on the routing and activations of the
 * last step, then all down kernels, each group between two events on the
 * engine stream.  Caches are not changed. */
mx_status mx_engine_time_experts(mx_engine* e, int32_t rows, mx_expert_timing* out);
mx_status mx_engine_read(mx_engine* e, const char* what, void* host, size_t bytes);
/* Test hook (no reference counterpart): one eager decode step of `rows`
 * rows at their own offsets in which every layer i takes its input streams
 * from h_in[i] (host bf16 [layers + 1][rows][hc * hidden]) instead of the
 * previous layer's output, so each layer can be compared with a CPU model
 * fed the same inputs ("teacher forcing").  Layer i's output streams go to
 * h_out[i] (host, [layers][rows][hc * hidden]) and its top-k expert ids to
 * ids_out[i] (host uint32 [layers][rows][top_k]); the mixer and the head run
 * on h_in[layers] and write `next`.  Caches and offsets advance as in
 * mx_engine_decode_rows. */
mx_status mx_engine_decode_forced(mx_engine* e, const int32_t* slots, const uint32_t* tokens,
                                  int32_t rows, const uint16_t* h_in, uint16_t* h_out,
                                  uint32_t* ids_out, uint32_t* next);
mx_status mx_engine_tensor(mx_engine* e, const char* name, void** device_ptr, size_t* bytes);

/* ---- checkpoint loading (§8(f)#3) ------------------------------------------
 * Tensor dtypes as safetensors names them. */
#define MX_DT_U32 0
#define MX_DT_BF16 1
#define MX_DT_F16 2
#define MX_DT_F32 3
/* Writes one checkpoint tensor, named as in an MLX checkpoint of the hybrid
 * model (the names Weights / HybridModel::load / Mtp::load read:
 * src/weights.rs:22-99, src/hybrid.rs:56-66, 130-142, 335-352, 529-567,
 * src/mtp.rs:39-70; an optional "language_model." prefix), into the engine's
 * matrices: in_proj_qkv / z / a / b fill rows of the fused GDN input
 * projection, mlp.gate and mlp.shared_expert_gate the router's rows,
 * input_mix_weight_down and block_inject_weight the hyper-connection's down
 * rows, q_proj / k_proj / v_proj the attention input rows; conv1d.weight
 * [channels, taps, 1] is stored as the engine's fp32 [taps, channels].
 * ".weight" (U32 packed codes), ".scales", ".biases" of a quantised linear
 * must match the engine's width and group size (MX_EUNSUPPORTED names the
 * difference).  Float tensors are taken only where the engine keeps their
 * exact values: into an fp32 tensor (A_log, conv1d.weight) any float dtype;
 * into a bf16 tensor (scales, biases, norm weights, dt_bias) BF16, or F16 /
 * F32 whose every value is a bf16 value -- otherwise MX_EUNSUPPORTED names
 * the tensor and the first value that would round.  MX_EUNSUPPORTED for modules the
 * engine does not build (per-layer n-gram embeddings "ple.", the attention
 * indexer "self_attn.indexer."), MX_EINVAL for unknown names or shapes.  The
 * engine is created from the checkpoint's config.json first (mx_model_config
 * field for field); tensors not loaded keep their seeded values. */
mx_status mx_engine_load_tensor(mx_engine* e, const char* name, int32_t dtype,
                                const int64_t* shape, int32_t ndim, const void* data,
                                size_t bytes);
/* The mapping of mx_engine_load_tensor without an engine or a device: where
 * `name` goes for configuration `cfg`.  tensor receives the engine tensor's
 * name (at most cap bytes with the terminator); info[0..7] = kind (0
 * quantised rows, 1 bf16 vector, 2 fp32 vector, 3 conv weight), part (0
 * codes, 1 scales, 2 biases), first row, rows, matrix rows n, matrix depth
 * k, bits, vector length.  Same statuses as mx_engine_load_tensor. */
mx_status mx_checkpoint_target(const mx_model_config* cfg, const char* name, char* tensor,
                               size_t cap, int32_t* info);
/* Every tensor of one .safetensors file through mx_engine_load_tensor (the
 * file read in order; vision towers and n-gram table row shards skipped, as
 * the reference's loader does); *loaded = tensors written.  Stops at the
 * first error. */
mx_status mx_engine_load_safetensors(mx_engine* e, const char* path, int32_t* loaded);
/* Every check of mx_engine_load_safetensors without an engine or a device:
 * the file's header (offsets inside the file, positive dims, bytes matching
 * shape and dtype), each tensor's target, width, group count and exact float
 * values for configuration cfg.  *checked = tensors that pass; the first
 * failure returns its status and names the tensor (mx_last_error).  The
 * reference loads through MLX (src/weights.rs:22-99) and fails at its first
 * bad tensor too; this entry lets a caller refuse a checkpoint before it
 * allocates an engine. */
mx_status mx_checkpoint_check(const mx_model_config* cfg, const char* path, int32_t* checked);

/* mx_gdn_scan: the delta rule alone, on given inputs — the reference's
 * gdn_kernel::recurrent / recurrent_with_history interface (src/gdn_kernel.rs:7-142):
 * q, k bf16 [groups*t, hk, dk] (already normalised), v bf16 [groups*t, hv, dv],
 * g fp32 [groups*t, hv], beta bf16 [groups*t, hv]; y = bf16(state . q)
 * [groups*t, hv, dv]; state / history as for mx_gdn_recurrence. */
mx_status mx_gdn_scan(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                      const uint16_t* beta, const mx_gdn_dims* dims, int32_t groups, int32_t t,
                      const int32_t* slots, float* state, float* history, uint16_t* y,
                      void* stream);

/* mx_gdn_prefill_chunked: the delta rule of mx_gdn_scan over `t` tokens of each
 * of `groups` sequences, in the chunked form (64-token chunks; per chunk the
 * triangular transform T = (I + A)^-1 with A[t][s] = beta_t (gamma_t/gamma_s)
 * k_t.k_s, then D = U - W S, y = (gamma Q) S + P D, S' = gamma_C S + K'^T D, all
 * products that touch the fp32 state on fp32 matrix cores).  Inputs, state
 * and y as for mx_gdn_scan (no history).  workspace:
 * mx_gdn_prefill_workspace_bytes(groups, hv, t) bytes of device memory.
 * Replaces the T-token call of gdn_kernel::recurrent (src/gdn_kernel.rs:7-71,
 * kernels/gated_delta.metal), which the reference runs token by token. */
size_t mx_gdn_prefill_workspace_bytes(int32_t groups, int32_t hv, int32_t t);
mx_status mx_gdn_prefill_chunked(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const float* g, const uint16_t* beta, const mx_gdn_dims* dims,
                                 int32_t groups, int32_t t, const int32_t* slots, float* state,
                                 uint16_t* y, void* workspace, void* stream);

/* ---- A18: cooperative equal-offset scheduler with a prefix cache -----------
 * Host-side serving loop over the engine (or any backend with the same three
 * operations).  Replaces batch::serve / admit / Row::emit
 * (src/bin/server/batch.rs:240-349, 28-140) and PrefixCache::get_or_prepare
 * (src/speculative.rs:70-117):
 *  - up to batch_size rows are active; queued jobs are admitted in submission
 *    order while a row is free (admission prefills the prompt, or copies the
 *    cached state of an identical prompt, and emits its greedy token);
 *  - each mx_sched_step decodes, together, the active rows at the smallest
 *    cache offset among active rows;
 *  - a row ends on a stop token (reported, not emitted) or after max_tokens
 *    emitted tokens; prompt + max_tokens > max_context is rejected;
 *  - the prefix cache keeps up to prefix_entries prepared prompts within
 *    prefix_tokens tokens, least recently used evicted first, each in its own
 *    cache slot (a hit is a slot copy).
 * The scheduler is not thread safe; one owning thread, like the engine. */
typedef struct mx_sched mx_sched;
typedef struct mx_sched_backend {
  void* ctx;
  /* fresh cache in `slot`, then the prompt; *next = greedy token after it */
  mx_status (*prefill)(void* ctx, int32_t slot, const uint32_t* tokens, int32_t count,
                       uint32_t* next);
  /* one token for each of `rows` slots at equal offsets */
  mx_status (*decode)(void* ctx, const int32_t* slots, const uint32_t* tokens, int32_t rows,
                      uint32_t* next);
  mx_status (*clone)(void* ctx, int32_t src, int32_t dst);
} mx_sched_backend;
typedef struct mx_sched_config {
  int32_t batch_size;      /* rows decoded together, 1..8 */
  int32_t slots;           /* cache slots for rows and prefix entries (>= batch_size) */
  int32_t prefix_entries;  /* prefix-cache entries (0: no cache) */
  int32_t prefix_tokens;   /* token budget of the prefix cache */
  int32_t max_context;     /* prompt + max_tokens limit */
  int32_t n_stop;          /* stop tokens used (0..8) */
  uint32_t stop[8];
} mx_sched_config;
enum {
  MX_SCHED_TOKEN = 0,   /* `token` emitted; detail = 1 on a prompt's first token after a cache hit */
  MX_SCHED_STOP = 1,    /* finished on stop token `token` (not emitted) */
  MX_SCHED_LENGTH = 2,  /* finished after max_tokens tokens */
  MX_SCHED_ERROR = 3    /* rejected or failed; detail = mx_status */
};
typedef struct mx_sched_event {
  uint64_t job;
  uint32_t token;
  int32_t kind;
  int32_t detail;
} mx_sched_event;
mx_status mx_sched_create(const mx_sched_config* cfg, const mx_sched_backend* backend,
                          mx_sched** out);
mx_status mx_sched_create_for_engine(mx_engine* e, const mx_sched_config* cfg, mx_sched** out);
mx_status mx_sched_destroy(mx_sched* s);
mx_status mx_sched_submit(mx_sched* s, uint64_t job, const uint32_t* prompt, int32_t count,
                          int32_t max_tokens, int32_t use_prefix_cache);
/* drops a queued or active job (its slot is freed); MX_EINVAL if unknown */
mx_status mx_sched_cancel(mx_sched* s, uint64_t job);
/* one scheduler iteration; `capacity` >= 4 * batch_size events */
mx_status mx_sched_step(mx_sched* s, mx_sched_event* events, int32_t capacity, int32_t* count,
                        int32_t* decoded_rows);
int32_t mx_sched_pending(const mx_sched* s);  /* queued + active jobs */
int32_t mx_sched_cached(const mx_sched* s);   /* prefix-cache entries */

#ifdef __cplusplus
}
#endif

#endif /* MX355_H */
