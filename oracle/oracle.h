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
void mxo_qmv(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases, int n, int k,
             int bits, int gs, const uint16_t* x, int m, uint16_t* y);
void mxo_qmv_f64(const uint32_t* codes, const uint16_t* scales, const uint16_t* biases, int n,
                 int k, int bits, int gs, const uint16_t* x, int m, double* y);

int mxo_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif
