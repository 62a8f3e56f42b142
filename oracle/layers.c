/*
 * layers.c — MoE routing/experts/epilogue, GatedDeltaNet conv + recurrence and
 * the greedy head, restated on the CPU.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Each function performs the same IEEE single-precision operations in the same
 * order as the library's kernels, so results agree bit for bit; comments cite
 * the reference behaviour each step restates.
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

static float rbf(float f) { return mxo_bf16_to_f32(mxo_f32_to_bf16(f)); }
static float bf(uint16_t h) { return mxo_bf16_to_f32(h); }

/* MLX Sigmoid evaluated at bfloat: y = 1/(1+e^|x|), each operation rounded to
 * bf16 (reference kernels/moe_route_tail.metal:119-123). */
float mxo_sigmoid_bf16(float x) {
  const float e = rbf(mxo_expf(fabsf(x)));
  const float d = rbf(1.0f + e);
  const float y = rbf(1.0f / d);
  return x < 0.0f ? y : rbf(1.0f - y);
}

/* MLX LogAddExp(x, 0) at bfloat with per-operation rounding (compiled::decay,
 * reference src/compiled.rs:14-15). */
float mxo_softplus_bf16(float x) {
  if (isnan(x)) return x;
  const float hi = x > 0.0f ? x : 0.0f;
  const float lo = x > 0.0f ? 0.0f : x;
  if (isinf(hi) || (isinf(lo) && lo < 0)) return hi;
  const float d = rbf(lo - hi);
  const float e = rbf(mxo_expf(d));
  const float l = rbf(mxo_log1pf(e));
  return rbf(hi + l);
}

/* xor butterfly over n (power of two) lanes; returns lane 0's value, which
 * every lane holds. */
static float butterfly(float* v, int n) {
  float tmp[128];
  for (int o = n >> 1; o > 0; o >>= 1) {
    for (int l = 0; l < n; ++l) tmp[l] = v[l] + v[l ^ o];
    for (int l = 0; l < n; ++l) v[l] = tmp[l];
  }
  return v[0];
}

/* ---------------------------------------------------------------- MoE ---- */

/* Routing tail (reference kernels/moe_route_tail.metal, moe_route.rs:25-70):
 * softmax in fp32 (max, e^(x-max), sum, * 1/sum) with lane l of 64 owning
 * experts l*PER .. l*PER+PER-1 (sequential lane sums, xor butterfly);
 * bf16 gates; top-k by the order-preserving (bf16 key << 16 | index) key,
 * slot k-1 holding the largest; bf16 renormalisation with one bf16 add per
 * slot in ascending order; bf16 sigmoid of the shared-expert logit. */
void mxo_moe_route(const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
                   int64_t shared_stride, int rows, int experts, int top_k, uint32_t* ids,
                   uint16_t* scores, uint16_t* factor) {
  const int per = experts / 64;
  float v[1024];
  uint32_t key[1024];
  for (int r = 0; r < rows; ++r) {
    const uint16_t* in = logits + (int64_t)r * logit_stride;
    float mx = bf(in[0]);
    for (int e = 0; e < experts; ++e) {
      v[e] = bf(in[e]);
      if (v[e] > mx) mx = v[e];
    }
    float lanes[64];
    for (int l = 0; l < 64; ++l) {
      float s = 0.0f;
      for (int i = 0; i < per; ++i) {
        v[l * per + i] = mxo_expf(v[l * per + i] - mx);
        s = s + v[l * per + i];
      }
      lanes[l] = s;
    }
    const float inv = 1.0f / butterfly(lanes, 64);
    for (int e = 0; e < experts; ++e) {
      const uint32_t g = mxo_f32_to_bf16(v[e] * inv);
      const uint32_t k16 = (g & 0x8000u) ? (~g & 0xffffu) : (g | 0x8000u);
      key[e] = (k16 << 16) | (uint32_t)e;
    }
    float picked[64];
    for (int s = 0; s < top_k; ++s) {
      int bi = 0;
      for (int e = 1; e < experts; ++e)
        if (key[e] > key[bi]) bi = e;
      const uint32_t k16 = key[bi] >> 16;
      const uint32_t g = (k16 & 0x8000u) ? (k16 & 0x7fffu) : (~k16 & 0xffffu);
      picked[top_k - 1 - s] = bf((uint16_t)g);
      ids[(int64_t)r * top_k + top_k - 1 - s] = (uint32_t)bi;
      key[bi] = 0u;
    }
    float total = 0.0f;
    for (int j = 0; j < top_k; ++j) total = rbf(picked[j] + total);
    for (int j = 0; j < top_k; ++j) scores[(int64_t)r * top_k + j] = mxo_f32_to_bf16(picked[j] / total);
    factor[r] = mxo_f32_to_bf16(mxo_sigmoid_bf16(bf(shared_logit[(int64_t)r * shared_stride])));
  }
}

static const uint32_t* qw_row_codes(const mxo_qw* w, int64_t row) {
  return w->codes + row * (((int64_t)w->k * w->bits) >> 5);
}
static const uint16_t* qw_row_s(const mxo_qw* w, int64_t row) { return w->scales + row * (w->k / w->gs); }
static const uint16_t* qw_row_b(const mxo_qw* w, int64_t row) { return w->biases + row * (w->k / w->gs); }
static float qw_dot(const mxo_qw* w, int64_t row, const uint16_t* x) {
  if (w->mode == 1)
    return mxo_xq_row(qw_row_codes(w, row), qw_row_s(w, row), qw_row_b(w, row), w->k, w->bits, x);
  return mxo_qmv_row(qw_row_codes(w, row), qw_row_s(w, row), qw_row_b(w, row), w->k, w->bits, w->gs, x);
}
static mxo_qw bank_expert(const mxo_qbank* b, int e) {
  const int64_t cs = (int64_t)b->n * b->k * b->bits / 32;
  const int64_t ss = (int64_t)b->n * (b->k / b->gs);
  mxo_qw w = {b->codes + cs * e, b->scales + ss * e, b->biases + ss * e, b->n, b->k, b->bits, b->gs,
              b->mode};
  return w;
}

/* Expert MLPs (MoE::parts, reference src/hybrid.rs:192-287; gather_qmm per
 * route, swiglu compiled.rs:10-12, down_tail score product moe_down_tail.metal:81-83):
 *   h = bf16(bf16(bf16(g) * sigmoid_bf16(bf16(g))) * bf16(u))
 *   p[row][slot] = bf16(bf16(down(h)) * score)   (slot == top_k: the shared
 *   expert, unweighted: bf16(down(h))).
 * p is [rows, top_k + 1, hidden]. */
void mxo_moe_experts(const uint16_t* x, const uint32_t* ids, const uint16_t* scores, int rows,
                     int top_k, const mxo_qbank* gate, const mxo_qbank* up, const mxo_qbank* down,
                     const mxo_qw* sgate, const mxo_qw* sup, const mxo_qw* sdown, uint16_t* p) {
  const int hidden = gate->k;
  const int routes = rows * (top_k + 1);
#pragma omp parallel for schedule(dynamic)
  for (int t = 0; t < routes; ++t) {
    const int r = t / (top_k + 1), slot = t % (top_k + 1);
    mxo_qw g, u, d;
    if (slot < top_k) {
      const int e = (int)ids[(int64_t)r * top_k + slot];
      g = bank_expert(gate, e);
      u = bank_expert(up, e);
      d = bank_expert(down, e);
    } else {
      g = *sgate;
      u = *sup;
      d = *sdown;
    }
    const int inter = g.n;
    uint16_t h[4096];
    const uint16_t* xr = x + (int64_t)r * hidden;
    for (int i = 0; i < inter; ++i) {
      const float gv = rbf(qw_dot(&g, i, xr));
      const float uv = rbf(qw_dot(&u, i, xr));
      const float silu = rbf(gv * mxo_sigmoid_bf16(gv));
      h[i] = mxo_f32_to_bf16(silu * uv);
    }
    const float sc = slot < top_k ? bf(scores[(int64_t)r * top_k + slot]) : 1.0f;
    uint16_t* out = p + ((int64_t)r * (top_k + 1) + slot) * d.n;
    for (int c = 0; c < d.n; ++c) {
      const float dv = rbf(qw_dot(&d, c, h));
      out[c] = mxo_f32_to_bf16(slot < top_k ? dv * sc : dv);
    }
  }
}

/* Slot reduction in the reference order (kernels/moe_down_tail.h:20,
 * moe_down_tail.metal:83-99): slot i accumulates into lane i % 8 (one bf16 add
 * per later slot), then lanes 1..7 are added to lane 0 one by one. */
static float slot_sum(const uint16_t* pr, int top_k, int64_t stride) {
  float acc[8] = {0.0f};
  const int lanes = top_k < 8 ? top_k : 8;
  for (int a = 0; a < lanes; ++a) {
    float v = bf(pr[a * stride]);
    for (int s = a + 8; s < top_k; s += 8) v = rbf(v + bf(pr[s * stride]));
    acc[a] = v;
  }
  float routed = acc[0];
  for (int a = 1; a < lanes; ++a) routed = rbf(acc[a] + routed);
  return routed;
}

void mxo_moe_reduce(const uint16_t* p, int rows, int top_k, int hidden, uint16_t* routed) {
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < hidden; ++c)
      routed[(int64_t)r * hidden + c] =
          mxo_f32_to_bf16(slot_sum(p + (int64_t)r * (top_k + 1) * hidden + c, top_k, hidden));
}

/* HC write of the MoE output (kernels/moe_hc_epilogue.metal:8-11). */
void mxo_moe_hc_epilogue(const uint16_t* routed, const uint16_t* shared, const uint16_t* factor,
                         const uint16_t* residual, const uint16_t* gate, int rows, int hc,
                         int hidden, uint16_t* out) {
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < hidden; ++c) {
      const float weighted = rbf(bf(shared[(int64_t)r * hidden + c]) * bf(factor[r]));
      const float combined = rbf(bf(routed[(int64_t)r * hidden + c]) + weighted);
      for (int s = 0; s < hc; ++s) {
        const int64_t o = ((int64_t)r * hc + s) * hidden + c;
        const float inj = rbf(combined * bf(gate[(int64_t)r * hc + s]));
        out[o] = mxo_f32_to_bf16(bf(residual[o]) + inj);
      }
    }
}

/* ---------------------------------------------------------------- GDN ---- */

/* Causal depthwise conv + SiLU over the cached window (compiled::decode_conv,
 * reference src/compiled.rs:88-95, applied per position as in verify mode,
 * src/hybrid.rs:385-396): acc = sum_j fl(x_j * w_j) in tap order, v = bf16(acc),
 * out = bf16(v * sigmoid_bf16(v)).  Updates conv_state [slots, K-1, C] and,
 * when window_history is non-null, stores the window [g, K-1+t, C]. */
void mxo_gdn_conv(const uint16_t* qkv, int64_t row_stride, int groups, int t, const int32_t* slots,
                  uint16_t* conv_state, const float* w, int channels, int taps, uint16_t* out,
                  int64_t out_stride, uint16_t* window_history) {
  for (int g = 0; g < groups; ++g) {
    uint16_t* st = conv_state + (int64_t)slots[g] * (taps - 1) * channels;
    for (int c = 0; c < channels; ++c) {
      float win[8];
      for (int j = 0; j < taps - 1; ++j) win[j] = bf(st[(int64_t)j * channels + c]);
      uint16_t* hist = window_history ? window_history + (int64_t)g * (taps - 1 + t) * channels + c : 0;
      if (hist)
        for (int j = 0; j < taps - 1; ++j) hist[(int64_t)j * channels] = mxo_f32_to_bf16(win[j]);
      for (int i = 0; i < t; ++i) {
        const int64_t row = (int64_t)g * t + i;
        const uint16_t xr = qkv[row * row_stride + c];
        win[taps - 1] = bf(xr);
        if (hist) hist[(int64_t)(taps - 1 + i) * channels] = xr;
        float acc = 0.0f;
        for (int j = 0; j < taps; ++j) acc = acc + win[j] * w[(int64_t)j * channels + c];
        const float v = rbf(acc);
        out[row * out_stride + c] = mxo_f32_to_bf16(v * mxo_sigmoid_bf16(v));
        for (int j = 0; j < taps - 1; ++j) win[j] = win[j + 1];
      }
      for (int j = 0; j < taps - 1; ++j) st[(int64_t)j * channels + c] = mxo_f32_to_bf16(win[j]);
    }
  }
}

/* Sum of 128 values: xor butterfly over each half (64 lanes), then
 * half 0 + half 1. */
static float sum128(const float* v) {
  float a[64], b[64];
  memcpy(a, v, sizeof a);
  memcpy(b, v + 64, sizeof b);
  const float sa = butterfly(a, 64);
  const float sb = butterfly(b, 64);
  return sa + sb;
}

/* Delta rule for one token of one value head (reference kernels/gated_delta.metal,
 * gdn_reference src/hybrid.rs:457-498): s *= g; kv = s.k; delta = (v - kv) * beta;
 * s += k delta; y = bf16(s.q).  Dot products as four interleaved fma chains
 * (d mod 4), then (c0+c1)+(c2+c3).  State [Dk][Dv] (dk-major). */
static void scan_token(float* sp, const float* q, const float* k, const float* v, float beta,
                       float gd, float* yo) {
  enum { D = 128 };
  for (int i = 0; i < D; ++i) {
    float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int d = 0; d < D; ++d) {
      float* s = &sp[(int64_t)d * D + i];
      *s = *s * gd;
      c[d & 3] = fmaf(*s, k[d], c[d & 3]);
    }
    const float kv = (c[0] + c[1]) + (c[2] + c[3]);
    const float delta = (v[i] - kv) * beta;
    float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int d = 0; d < D; ++d) {
      float* s = &sp[(int64_t)d * D + i];
      *s = fmaf(k[d], delta, *s);
      o[d & 3] = fmaf(*s, q[d], o[d & 3]);
    }
    yo[i] = rbf((o[0] + o[1]) + (o[2] + o[3]));
  }
}

/* The reference's recurrent-kernel interface: normalised q, k [rows, hk, 128],
 * v [rows, hv, 128], g f32 [rows, hv], beta bf16 [rows, hv] -> y bf16
 * [rows, hv, 128].  State [slots, hv, Dk, Dv]; history [rows, hv, Dk, Dv]. */
void mxo_gdn_scan(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                  const uint16_t* beta, int hk_heads, int hv_heads, int groups, int t,
                  const int32_t* slots, float* state, float* history, uint16_t* y) {
  enum { D = 128 };
#pragma omp parallel for collapse(2) schedule(static)
  for (int gi = 0; gi < groups; ++gi)
    for (int hv = 0; hv < hv_heads; ++hv) {
      const int hk = hv / (hv_heads / hk_heads);
      float* sp = state + ((int64_t)slots[gi] * hv_heads + hv) * D * D;
      for (int step = 0; step < t; ++step) {
        const int64_t row = (int64_t)gi * t + step;
        float qf[D], kf[D], vf[D], yo[D];
        for (int i = 0; i < D; ++i) {
          qf[i] = bf(q[(row * hk_heads + hk) * D + i]);
          kf[i] = bf(k[(row * hk_heads + hk) * D + i]);
          vf[i] = bf(v[(row * hv_heads + hv) * D + i]);
        }
        scan_token(sp, qf, kf, vf, bf(beta[row * hv_heads + hv]), g[row * hv_heads + hv], yo);
        if (history) memcpy(history + ((row * hv_heads + hv) * D) * D, sp, sizeof(float) * D * D);
        for (int i = 0; i < D; ++i) y[(row * hv_heads + hv) * D + i] = mxo_f32_to_bf16(yo[i]);
      }
    }
}

/* The GDN sublayer between the conv and out_proj (reference
 * Gdn::forward_reference src/hybrid.rs:401-453):
 *   q = bf16(bf16(q * bf16(rsqrt(bf16(bf16(sum bf16(q^2)) + bf16(1e-6))))) * bf16(Dk^-1/2))
 *   k likewise without the scale; beta = sigmoid_bf16(b);
 *   g = exp(-exp(A_log) * softplus_bf16(bf16(a + dt)))              (f32)
 *   delta rule (scan_token); y = bf16(bf16(w * bf16(y * rsqrt(mean(y^2) + eps))) * sigmoid(z)).
 * Sums over 128 values: xor butterfly over each half of 64, then half0 + half1.
 * Requires Dk == Dv == 128. */
void mxo_gdn_recurrence(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                        const uint16_t* a, const uint16_t* b, int64_t zab_stride,
                        const float* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                        float eps, int hk_heads, int hv_heads, int groups, int t,
                        const int32_t* slots, float* state, float* history, uint16_t* y) {
  enum { D = 128 };
  const float eps_l2 = rbf(1e-6f);
  const float qscale = rbf(0.08838834764831845f);
#pragma omp parallel for collapse(2) schedule(static)
  for (int g = 0; g < groups; ++g)
    for (int hv = 0; hv < hv_heads; ++hv) {
      const int hk = hv / (hv_heads / hk_heads);
      float* sp = state + ((int64_t)slots[g] * hv_heads + hv) * D * D;
      const float neg_a = -mxo_expf(a_log[hv]);
      const float dt = bf(dt_bias[hv]);
      for (int step = 0; step < t; ++step) {
        const int64_t row = (int64_t)g * t + step;
        const uint16_t* cr = conv_out + row * conv_stride;
        float q[D], k[D], v[D], tq[D], tk[D], yo[D];
        for (int i = 0; i < D; ++i) {
          q[i] = bf(cr[hk * D + i]);
          k[i] = bf(cr[(hk_heads + hk) * D + i]);
          v[i] = bf(cr[2 * hk_heads * D + hv * D + i]);
          tq[i] = rbf(q[i] * q[i]);
          tk[i] = rbf(k[i] * k[i]);
        }
        const float qss = rbf(sum128(tq));
        const float kss = rbf(sum128(tk));
        const float rq = rbf(1.0f / sqrtf(rbf(qss + eps_l2)));
        const float rk = rbf(1.0f / sqrtf(rbf(kss + eps_l2)));
        for (int i = 0; i < D; ++i) {
          q[i] = rbf(rbf(q[i] * rq) * qscale);
          k[i] = rbf(k[i] * rk);
        }
        const float beta = mxo_sigmoid_bf16(bf(b[row * zab_stride + hv]));
        const float x = rbf(bf(a[row * zab_stride + hv]) + dt);
        const float gd = mxo_expf(neg_a * mxo_softplus_bf16(x));
        scan_token(sp, q, k, v, beta, gd, yo);
        if (history)
          memcpy(history + ((row * hv_heads + hv) * D) * D, sp, sizeof(float) * D * D);
        float sq[D];
        for (int i = 0; i < D; ++i) sq[i] = yo[i] * yo[i];
        const float ss = sum128(sq);
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
        for (int i = 0; i < D; ++i) {
          const float normed = rbf(bf(norm_w[i]) * rbf(yo[i] * inv));
          const float zi = bf(z[row * zab_stride + hv * D + i]);
          y[row * ((int64_t)hv_heads * D) + hv * D + i] = mxo_f32_to_bf16(normed * mxo_sigmoidf(zi));
        }
      }
    }
}

/* -------------------------------------------------------------- head ---- */

/* Greedy selection over bf16 values (reference kernels/greedy_reduce.metal,
 * MLX argmax): the largest value, lowest id among equals; NaN never wins; 0
 * when no value exceeds -inf. */
static uint32_t select_best(const float* v, int64_t n) {
  float best = -INFINITY;
  uint32_t id = 0;
  for (int64_t i = 0; i < n; ++i)
    if (v[i] > best) {
      best = v[i];
      id = (uint32_t)i;
    }
  return id;
}

void mxo_argmax_bf16(const uint16_t* logits, int rows, int n, uint32_t* tokens) {
  for (int r = 0; r < rows; ++r) {
    float best = -INFINITY;
    uint32_t id = 0;
    for (int i = 0; i < n; ++i) {
      const float x = bf(logits[(int64_t)r * n + i]);
      if (x > best) {
        best = x;
        id = (uint32_t)i;
      }
    }
    tokens[r] = id;
  }
}

/* Greedy head: bf16(qmv row) for every vocabulary row, then select_best. */
void mxo_head_argmax(const mxo_qw* w, const uint16_t* x, int m, uint32_t* tokens, float* scratch) {
  for (int mm = 0; mm < m; ++mm) {
#pragma omp parallel for schedule(static)
    for (int row = 0; row < w->n; ++row)
      scratch[row] = rbf(qw_dot(w, row, x + (int64_t)mm * w->k));
    tokens[mm] = select_best(scratch, w->n);
  }
}

/* Unquantised bf16 GEMV for 1..8 rows (reference src/gemv_kernel.rs:30-90,
 * kernels/shared_gemv.metal): per output column, 32 lanes; lane l accumulates,
 * over k-blocks of 128 in order, values k0 + 4l + c (c = 0..3) as
 * acc = fma(w, x, acc); then a shuffle-down tree over lanes with offsets 16, 8,
 * 4, 2, 1 (lane l += lane l + d); lane 0's sum is rounded to bf16.  Every row
 * uses the same order, so a row's result does not depend on the others. */
void mxo_gemv_bf16(const uint16_t* w, int n, int k, const uint16_t* x, int rows, uint16_t* y) {
#pragma omp parallel for schedule(static)
  for (int o = 0; o < n; ++o) {
    for (int r = 0; r < rows; ++r) {
      float acc[32];
      for (int l = 0; l < 32; ++l) {
        float a = 0.0f;
        for (int k0 = 0; k0 < k; k0 += 128)
          for (int c = 0; c < 4; ++c) {
            const int kk = k0 + 4 * l + c;
            a = fmaf(bf(w[(int64_t)o * k + kk]), bf(x[(int64_t)r * k + kk]), a);
          }
        acc[l] = a;
      }
      for (int d = 16; d >= 1; d >>= 1)
        for (int l = 0; l < d; ++l) acc[l] = acc[l] + acc[l + d];
      y[(int64_t)r * n + o] = mxo_f32_to_bf16(acc[0]);
    }
  }
}
