/*
 * model.c — hyper-connection projections, attention and embedding of the
 * hybrid model step, restated on the CPU.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Same IEEE single-precision operations in the same order as the library's
 * kernels (proj.hip, attn.hip), so results agree bit for bit.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static float rbf(float f) { return mxo_bf16_to_f32(mxo_f32_to_bf16(f)); }
static float bf(uint16_t h) { return mxo_bf16_to_f32(h); }

static float butterfly64(float* v) {
  float tmp[64];
  for (int o = 32; o > 0; o >>= 1) {
    for (int l = 0; l < 64; ++l) tmp[l] = v[l] + v[l ^ o];
    for (int l = 0; l < 64; ++l) v[l] = tmp[l];
  }
  return v[0];
}

static float row_dot(const mxo_qw* w, int64_t row, const uint16_t* x) {
  const int64_t wpr = ((int64_t)w->k * w->bits) >> 5;
  const int gpr = w->k / w->gs;
  if (w->mode == 1)
    return mxo_xq_row(w->codes + row * wpr, w->scales + row * gpr, w->biases + row * gpr, w->k,
                      w->bits, x);
  return mxo_qmv_row(w->codes + row * wpr, w->scales + row * gpr, w->biases + row * gpr, w->k,
                     w->bits, w->gs, x);
}

/* Grouped zero-centred RMS norm (compiled::norm over [hc, H], reference
 * src/compiled.rs:22-28, src/hybrid.rs:39-44): lane t of 256 sums x^2 over
 * columns t, t+256, ... (product rounded, then added); xor butterfly per
 * 64-lane wave; the four wave sums added in order; y = bf16((x*inv)*(w+1)). */
void mxo_hc_norm(const uint16_t* x, const uint16_t* scale, int rows, int hc, int hidden, float eps,
                 uint16_t* y) {
  for (int r = 0; r < rows; ++r)
    for (int s = 0; s < hc; ++s) {
      const uint16_t* xr = x + ((int64_t)r * hc + s) * hidden;
      float lanes[256];
      for (int t = 0; t < 256; ++t) {
        float acc = 0.0f;
        for (int c = t; c < hidden; c += 256) {
          const float v = bf(xr[c]);
          acc = acc + v * v;
        }
        lanes[t] = acc;
      }
      float w4[4];
      for (int w = 0; w < 4; ++w) w4[w] = butterfly64(lanes + 64 * w);
      const float total = ((w4[0] + w4[1]) + w4[2]) + w4[3];
      const float inv = 1.0f / sqrtf(total / (float)hidden + eps);
      uint16_t* yr = y + ((int64_t)r * hc + s) * hidden;
      const uint16_t* sc = scale + (int64_t)s * hidden;
      for (int c = 0; c < hidden; ++c) yr[c] = mxo_f32_to_bf16((bf(xr[c]) * inv) * (bf(sc[c]) + 1.0f));
    }
}

/* HC down (+ inject) projection (compiled::activate / injection, reference
 * src/compiled.rs:46-58): t = bf16(bf16(v) / hc); rows < rank:
 * lo = bf16(t * sigmoid_bf16(t)); rows >= rank: inj = bf16(sigmoid_bf16(t) * 2). */
void mxo_hc_down(const mxo_qw* w, const uint16_t* xn, int rows, int rank, int hc, uint16_t* lo,
                 uint16_t* inj) {
  const int64_t xs = w->k;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < w->n; ++n)
    for (int m = 0; m < rows; ++m) {
      const float t = rbf(rbf(row_dot(w, n, xn + m * xs)) / (float)hc);
      if (n < rank)
        lo[(int64_t)m * rank + n] = mxo_f32_to_bf16(t * mxo_sigmoid_bf16(t));
      else
        inj[(int64_t)m * hc + (n - rank)] = mxo_f32_to_bf16(mxo_sigmoid_bf16(t) * 2.0f);
    }
}

/* HC up projection + mix (compiled::mix, reference src/compiled.rs:68-86):
 * mixed[c] = bf16(bf16(sum_s bf16(sigmoid_bf16(bf16(p_s)) * xn_s)) / 4), the
 * sum over the four streams in order; p_s is row c + s*H of the projection. */
void mxo_hc_up_mix(const mxo_qw* w, const uint16_t* lo, const uint16_t* xn, int rows, int hidden,
                   uint16_t* mixed) {
#pragma omp parallel for schedule(static)
  for (int c = 0; c < hidden; ++c)
    for (int m = 0; m < rows; ++m) {
      float sum = 0.0f;
      for (int s = 0; s < 4; ++s) {
        const float p = rbf(row_dot(w, (int64_t)c + (int64_t)s * hidden, lo + (int64_t)m * w->k));
        const float x = bf(xn[(int64_t)m * 4 * hidden + (int64_t)s * hidden + c]);
        sum = sum + rbf(mxo_sigmoid_bf16(p) * x);
      }
      mixed[(int64_t)m * hidden + c] = mxo_f32_to_bf16(rbf(sum) / 4.0f);
    }
}

/* Branch output projection with the HC write (HyperConnection::write,
 * reference src/hybrid.rs:100-105): residual[s][c] =
 * bf16(residual + bf16(bf16(v_c) * inj[s])), in place. */
void mxo_hc_write(const mxo_qw* w, const uint16_t* y, int rows, int hc, uint16_t* residual,
                  const uint16_t* inj) {
#pragma omp parallel for schedule(static)
  for (int c = 0; c < w->n; ++c)
    for (int m = 0; m < rows; ++m) {
      const float v = rbf(row_dot(w, c, y + (int64_t)m * w->k));
      for (int s = 0; s < hc; ++s) {
        uint16_t* res = residual + (int64_t)m * hc * w->n + (int64_t)s * w->n + c;
        const float in = rbf(v * bf(inj[(int64_t)m * hc + s]));
        *res = mxo_f32_to_bf16(bf(*res) + in);
      }
    }
}

/* Embedding: bf16(s*q + b) of row ids[i], broadcast to hc streams. */
void mxo_embed(const mxo_qw* w, const uint32_t* ids, int count, int hc, uint16_t* out) {
  uint16_t* row = (uint16_t*)malloc(sizeof(uint16_t) * w->k);
  for (int i = 0; i < count; ++i) {
    mxo_dequant_rows(w->codes, w->scales, w->biases, w->n, w->k, w->bits, w->gs, ids + i, 1, row);
    for (int s = 0; s < hc; ++s) memcpy(out + ((int64_t)i * hc + s) * w->k, row, sizeof(uint16_t) * w->k);
  }
  free(row);
}

/* q/k norm + RoPE + KV append (reference src/dense.rs:158-200, src/rope.rs,
 * kernels/text_rope.metal).  Norm per head: lane l of 64 sums x^2 over
 * l, l+64, ... in order, xor butterfly; y = bf16((x*inv)*(w+1)).  RoPE on the
 * first `rot` values: out[i] = bf16(x1 c - x2 s), out[i+h] = bf16(x2 c + x1 s).
 * Cache layout [slot][kv head][position][hd] with `slot_stride` elements
 * between slots (one layer's view). */
void mxo_attn_prep(const uint16_t* qkv, int64_t qkv_stride, int rows, const int32_t* slots,
                   const int32_t* pos, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
                   const float* rope_cos, const float* rope_sin, int heads, int kv_heads, int hd,
                   int rot, int max_ctx, int64_t slot_stride, uint16_t* q_out, uint16_t* k_cache,
                   uint16_t* v_cache) {
  const int half = rot / 2;
  float buf[256];
  for (int r = 0; r < rows; ++r) {
    const uint16_t* xr = qkv + (int64_t)r * qkv_stride;
    const int p = pos[r];
    const int64_t off = (int64_t)slots[r] * slot_stride;
    for (int head = 0; head < heads + 2 * kv_heads; ++head) {
      if (head >= heads + kv_heads) {
        const int kvh = head - heads - kv_heads;
        memcpy(v_cache + off + ((int64_t)kvh * max_ctx + p) * hd,
               xr + (int64_t)heads * 2 * hd + (int64_t)kv_heads * hd + (int64_t)kvh * hd,
               sizeof(uint16_t) * hd);
        continue;
      }
      const int is_q = head < heads;
      const int h = is_q ? head : head - heads;
      const uint16_t* src = is_q ? xr + (int64_t)h * 2 * hd : xr + (int64_t)heads * 2 * hd + (int64_t)h * hd;
      const uint16_t* w = is_q ? q_norm : k_norm;
      float lanes[64];
      for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int c = l; c < hd; c += 64) {
          const float v = bf(src[c]);
          acc = acc + v * v;
        }
        lanes[l] = acc;
      }
      const float total = butterfly64(lanes);
      const float inv = 1.0f / sqrtf(total / (float)hd + eps);
      for (int c = 0; c < hd; ++c) buf[c] = rbf((bf(src[c]) * inv) * (bf(w[c]) + 1.0f));
      uint16_t* dst = is_q ? q_out + ((int64_t)r * heads + h) * hd
                           : k_cache + off + ((int64_t)h * max_ctx + p) * hd;
      const float* cs = rope_cos + (int64_t)p * half;
      const float* sn = rope_sin + (int64_t)p * half;
      for (int c = 0; c < hd; ++c) {
        float v;
        if (c < half)
          v = buf[c] * cs[c] - buf[c + half] * sn[c];
        else if (c < 2 * half)
          v = buf[c] * cs[c - half] + buf[c - half] * sn[c - half];
        else
          v = buf[c];
        dst[c] = mxo_f32_to_bf16(v);
      }
    }
  }
}

/* Scaled dot-product attention over positions 0..pos[r] in chunks of 256 with
 * the kernels' order (attn.hip), then the output gate:
 *   per chunk: s_j = ((q.k_j) as four fma chains d mod 4, (c0+c1)+(c2+c3)) * scale;
 *   m = max s; p_j = e^(s_j - m); l = per-64 butterflies of p summed in wave order;
 *   o[d] = ((o_0 + o_1) + o_2) + o_3, o_w the fma chain over the chunk's
 *   positions 64 w .. 64 w + 63 (ascending) of p_j v_j[d];
 *   combine: M = max m_c; w_c = e^(m_c - M); L = fma(l_c, w_c, L); O = fma(o_c, w_c, O);
 *   y = bf16(bf16(O / L) * sigmoid_bf16(gate)). */
void mxo_attention(const uint16_t* q, const uint16_t* qkv, int64_t qkv_stride, int rows,
                   const int32_t* slots, const int32_t* pos, const uint16_t* k_cache,
                   const uint16_t* v_cache, int heads, int kv_heads, int hd, int max_ctx,
                   int64_t slot_stride, uint16_t* out) {
  enum { CH = 256 };
  const int G = heads / kv_heads;
  const float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int r = 0; r < rows; ++r)
    for (int h = 0; h < heads; ++h) {
      const int kvh = h / G;
      const int n_pos = pos[r] + 1;
      const int chunks = (n_pos + CH - 1) / CH;
      const int64_t base = (int64_t)slots[r] * slot_stride + (int64_t)kvh * max_ctx * hd;
      float qf[256];
      for (int d = 0; d < hd; ++d) qf[d] = bf(q[((int64_t)r * heads + h) * hd + d]);
      float* ms = (float*)malloc(sizeof(float) * chunks * 2);
      float* os = (float*)malloc(sizeof(float) * chunks * hd);
      for (int c = 0; c < chunks; ++c) {
        const int j0 = c * CH;
        float p[CH];
        float m = -INFINITY;
        for (int t = 0; t < CH; ++t) {
          const int j = j0 + t;
          if (j < n_pos) {
            const uint16_t* kr = k_cache + base + (int64_t)j * hd;
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int d = 0; d < hd; ++d) a[d & 3] = fmaf(qf[d], bf(kr[d]), a[d & 3]);
            p[t] = ((a[0] + a[1]) + (a[2] + a[3])) * scale;
          } else {
            p[t] = -INFINITY;
          }
          if (p[t] > m) m = p[t];
        }
        float w4[4];
        for (int t = 0; t < CH; ++t) p[t] = (j0 + t < n_pos) ? mxo_expf(p[t] - m) : 0.0f;
        for (int w = 0; w < 4; ++w) {
          float lanes[64];
          memcpy(lanes, p + 64 * w, sizeof lanes);
          w4[w] = butterfly64(lanes);
        }
        ms[2 * c] = m;
        ms[2 * c + 1] = ((w4[0] + w4[1]) + w4[2]) + w4[3];
        const int jend = n_pos - j0 < CH ? n_pos - j0 : CH;
        for (int d = 0; d < hd; ++d) {
          float ow[4];
          for (int w = 0; w < 4; ++w) {
            ow[w] = 0.0f;
            const int jb = jend < 64 * w + 64 ? jend : 64 * w + 64;
            for (int jj = 64 * w; jj < jb; ++jj)
              ow[w] = fmaf(p[jj], bf(v_cache[base + (int64_t)(j0 + jj) * hd + d]), ow[w]);
          }
          os[(int64_t)c * hd + d] = ((ow[0] + ow[1]) + ow[2]) + ow[3];
        }
      }
      float M = ms[0];
      for (int c = 1; c < chunks; ++c)
        if (ms[2 * c] > M) M = ms[2 * c];
      for (int d = 0; d < hd; ++d) {
        float L = 0.0f, O = 0.0f;
        for (int c = 0; c < chunks; ++c) {
          const float wc = mxo_expf(ms[2 * c] - M);
          L = fmaf(ms[2 * c + 1], wc, L);
          O = fmaf(os[(int64_t)c * hd + d], wc, O);
        }
        const float attn = rbf(O / L);
        const float gate = bf(qkv[(int64_t)r * qkv_stride + (int64_t)h * 2 * hd + hd + d]);
        out[((int64_t)r * heads + h) * hd + d] = mxo_f32_to_bf16(attn * mxo_sigmoid_bf16(gate));
      }
      free(ms);
      free(os);
    }
}

/* RoPE table (reference src/rope.rs:20-24): inv_freq[i] = 1 / powf(theta, 2i/rot)
 * in fp32; the angle is the fp32 product pos * inv_freq, as
 * kernels/text_rope.metal computes it (`float angle = pos*float(inv_freq)`),
 * so its rounding error grows with the position; cos/sin of that fp32 angle
 * are evaluated in double and rounded to fp32 (the last ulp of metal::cos is
 * parity unpinned). */
void mxo_rope_table(int max_ctx, int rot, float theta, float* cos_out, float* sin_out) {
  const int half = rot / 2;
  for (int i = 0; i < half; ++i) {
    const float power = (float)(2 * i) / (float)rot;
    const float inv = 1.0f / powf(theta, power);
    for (int p = 0; p < max_ctx; ++p) {
      const float a = (float)p * inv;
      cos_out[(int64_t)p * half + i] = (float)cos((double)a);
      sin_out[(int64_t)p * half + i] = (float)sin((double)a);
    }
  }
}
