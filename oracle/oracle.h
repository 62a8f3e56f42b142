/*
 * oracle.h — CPU restatement of rust-mlx's decode-step arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (libmx355) never links, imports or calls it.
 *
 * Every function states the reference file:line whose behaviour it restates
 * and the fixed operation order it shares with the GPU kernels, so GPU and
 * oracle agree bit for bit where the order is shared and within tolerance
 * where it is not.  Plain C99, compiled with -ffp-contract=off so that every
 * fused multiply-add is an explicit fmaf().
 */
#ifndef MX_ORACLE_H
#define MX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---- */
float mxo_bf16_to_f32(uint16_t h);
uint16_t mxo_f32_to_bf16(float f);
float mxo_expf(float x);
float mxo_log1pf(float x);
float mxo_sigmoidf(float x);
float mxo_softplusf(float x);
void mxo_eval_math(int op, const float* in, float* out, int64_t n);

/* ---- counter-based generator (same streams as the device generator) ---- */
uint64_t mxo_rng_u64(uint64_t seed, uint64_t idx);
void mxo_fill_bf16(uint16_t* dst, size_t count, uint64_t seed, int dist, float a, float b);
void mxo_fill_codes(uint32_t* dst, int64_t rows, int k, int bits, uint64_t seed);

/* ---- A3/A4: affine quantisation ---- */
uint32_t mxo_code(const uint32_t* row_words, int k, int bits);
void mxo_dequant_rows(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases,
                      int n, int k, int bits, int gs, const uint32_t* ids, int count,
                      uint16_t* out);
float mxo_qmv_row(const uint32_t* row_words, const uint16_t* scale_row, const uint16_t* bias_row,
                  int k, int bits, int gs, const uint16_t* x);
void mxo_qmv(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases, int n, int k,
             int bits, int gs, const uint16_t* x, int m, uint16_t* y);
void mxo_qmv_f64(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases, int n,
                 int k, int bits, int gs, const uint16_t* x, int m, double* y);

/* ---- exact-integer affine projection (xq.c): the engine's bit-exact path ---- */
int mxo_xq_slices(int k);
int64_t mxo_xq_int(uint16_t h, int eb);
int mxo_xq_group_exp(const uint16_t* x);
float mxo_xq_row(const uint32_t* row_words, const uint16_t* scale_row, const uint16_t* bias_row,
                 int k, int bits, const uint16_t* x);
void mxo_xq(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases, int n, int k,
            int bits, const uint16_t* x, int m, float* y);

/* ---- quantised weights as plain structs ----
 * mode 0: projections in the fixed fp32 order of mxo_qmv_row; mode 1: the
 * exact-integer projection of mxo_xq_row (group size 64). */
typedef struct mxo_qw {
  const uint32_t* codes;
  const uint16_t* scales;
  const uint16_t* biases;
  int n, k, bits, gs, mode;
} mxo_qw;
typedef struct mxo_qbank {
  const uint32_t* codes;
  const uint16_t* scales;
  const uint16_t* biases;
  int experts, n, k, bits, gs, mode;
} mxo_qbank;

/* ---- A6-A9: MoE ---- */
float mxo_sigmoid_bf16(float x);
float mxo_softplus_bf16(float x);
void mxo_moe_route(const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
                   int64_t shared_stride, int rows, int experts, int top_k, uint32_t* ids,
                   uint16_t* scores, uint16_t* factor);
void mxo_moe_experts(const uint16_t* x, const uint32_t* ids, const uint16_t* scores, int rows,
                     int top_k, const mxo_qbank* gate, const mxo_qbank* up, const mxo_qbank* down,
                     const mxo_qw* sgate, const mxo_qw* sup, const mxo_qw* sdown, uint16_t* p);
void mxo_moe_reduce(const uint16_t* p, int rows, int top_k, int hidden, uint16_t* routed);
void mxo_moe_hc_epilogue(const uint16_t* routed, const uint16_t* shared, const uint16_t* factor,
                         const uint16_t* residual, const uint16_t* gate, int rows, int hc,
                         int hidden, uint16_t* out);

/* ---- A10-A12: GatedDeltaNet ---- */
void mxo_gdn_conv(const uint16_t* qkv, int64_t row_stride, int groups, int t, const int32_t* slots,
                  uint16_t* conv_state, const float* w, int channels, int taps, uint16_t* out,
                  int64_t out_stride, uint16_t* window_history);
void mxo_gdn_recurrence(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                        const uint16_t* a, const uint16_t* b, int64_t zab_stride,
                        const float* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                        float eps, int hk_heads, int hv_heads, int groups, int t,
                        const int32_t* slots, float* state, float* history, uint16_t* y);

void mxo_gdn_scan(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                  const uint16_t* beta, int hk_heads, int hv_heads, int groups, int t,
                  const int32_t* slots, float* state, float* history, uint16_t* y);

/* ---- A16: unquantised bf16 GEMV for short rows ---- */
void mxo_gemv_bf16(const uint16_t* w, int n, int k, const uint16_t* x, int rows, uint16_t* y);

/* ---- A14: greedy head ---- */
void mxo_argmax_bf16(const uint16_t* logits, int rows, int n, uint32_t* tokens);
void mxo_head_argmax(const mxo_qw* w, const uint16_t* x, int m, uint32_t* tokens, float* scratch);

/* ---- model step pieces (model.c) ---- */
void mxo_hc_norm(const uint16_t* x, const uint16_t* scale, int rows, int hc, int hidden, float eps,
                 uint16_t* y);
void mxo_hc_down(const mxo_qw* w, const uint16_t* xn, int rows, int rank, int hc, uint16_t* lo,
                 uint16_t* inj);
void mxo_hc_up_mix(const mxo_qw* w, const uint16_t* lo, const uint16_t* xn, int rows, int hidden,
                   uint16_t* mixed);
void mxo_hc_write(const mxo_qw* w, const uint16_t* y, int rows, int hc, uint16_t* residual,
                  const uint16_t* inj);
void mxo_embed(const mxo_qw* w, const uint32_t* ids, int count, int hc, uint16_t* out);
void mxo_attn_prep(const uint16_t* qkv, int64_t qkv_stride, int rows, const int32_t* slots,
                   const int32_t* pos, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                   const float* rope_cos, const float* rope_sin, int heads, int kv_heads, int hd,
                   int rot, int max_ctx, int64_t slot_stride, uint16_t* q_out, uint16_t* k_cache,
                   uint16_t* v_cache);
void mxo_attention(const uint16_t* q, const uint16_t* qkv, int64_t qkv_stride, int rows,
                   const int32_t* slots, const int32_t* pos, const uint16_t* k_cache,
                   const uint16_t* v_cache, int heads, int kv_heads, int hd, int max_ctx,
                   int64_t slot_stride, uint16_t* out);
void mxo_rope_table(int max_ctx, int rot, float theta, float* cos_out, float* sin_out);

int mxo_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif
