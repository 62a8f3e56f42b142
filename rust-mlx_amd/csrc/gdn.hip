// GatedDeltaNet decode / verify kernels for gfx950.
//
// Reference: Gdn::forward_reference (src/hybrid.rs:369-455) with the compiled
// graphs decode_conv / decay / silu (src/compiled.rs:13-21, 88-95) and the
// recurrence kernel gdn_kernel::recurrent{,_with_history} (src/gdn_kernel.rs:7-142,
// kernels/gated_delta{,_history}.metal).
//
// Rows are organised as `groups` independent sequences of `t` consecutive
// tokens each (row = g * t + i): decode of B slots is groups = B, t = 1; an
// MTP verify block or a prefill chunk of one slot is groups = 1, t = T.
// `slots[g]` selects the recurrent state of group g.
//
// State layout (HBM): fp32 [slots, Hv, Dk, Dv] — dk-major, so the 128 lanes
// that own the 128 value rows of a head read and write it fully coalesced.
// (MLX keeps [B, Hv, Dv, Dk]; the C ABI documents the transposition.)
#include "common.hpp"
#include "kernels.hpp"
#include "xq_core.hpp"

namespace mx {

namespace {

// logaddexp(x, 0) at bfloat (MLX LogAddExp with per-operation bf16 rounding).
__device__ __forceinline__ float softplus_bf16(float x) {
  if (x != x) return x;
  const float hi = x > 0.0f ? x : 0.0f;
  const float lo = x > 0.0f ? 0.0f : x;
  if (hi == u2f(0x7f800000u) || lo == u2f(0xff800000u)) return hi;
  const float d = round_bf16(lo - hi);
  const float e = round_bf16(expf_(d));
  const float l = round_bf16(log1pf_(e));
  return round_bf16(hi + l);
}

// ---------------------------------------------------------------------------
// Causal depthwise conv over the cached window + SiLU, and the conv-state
// update.  One thread owns one channel of one group, so the in-place state
// update never races.  Per token: acc = sum_j fl(x_j * w_j) in j order (f32),
// out = bf16(acc); silu = bf16(out * sigmoid_bf16(out)).
__global__ __launch_bounds__(256) void conv_kernel(const uint16_t* __restrict__ qkv,
                                                   int64_t row_stride, int t,
                                                   const int32_t* __restrict__ slots,
                                                   uint16_t* __restrict__ conv_state,
                                                   const float* __restrict__ w, int channels,
                                                   int taps, uint16_t* __restrict__ out,
                                                   int64_t out_stride,
                                                   uint16_t* __restrict__ window_history) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const int g = blockIdx.y;
  if (c >= channels) return;
  uint16_t* st = conv_state + size_t(slots[g]) * (taps - 1) * channels + c;
  // fixed-size arrays indexed by unrolled loops (taps <= kMaxTaps, checked
  // on the host), so they stay in registers
  constexpr int kMaxTaps = 8;
  constexpr int kBlock = 8;  // tokens whose inputs are requested together
  float win[kMaxTaps];
  float wj[kMaxTaps];
#pragma unroll
  for (int j = 0; j < kMaxTaps; ++j) {
    win[j] = j < taps - 1 ? bf16_to_f32(st[size_t(j) * channels]) : 0.0f;
    wj[j] = j < taps ? w[size_t(j) * channels + c] : 0.0f;
  }
  uint16_t* hist = window_history
                       ? window_history + size_t(g) * (taps - 1 + t) * channels + c
                       : nullptr;
  if (hist)
    for (int j = 0; j < taps - 1; ++j) hist[size_t(j) * channels] = f32_to_bf16(win[j]);
  for (int i0 = 0; i0 < t; i0 += kBlock) {
    const int n = t - i0 < kBlock ? t - i0 : kBlock;
    uint16_t xs[kBlock];
#pragma unroll
    for (int i = 0; i < kBlock; ++i)
      xs[i] = i < n ? qkv[(size_t(g) * t + i0 + i) * row_stride + c] : uint16_t(0);
#pragma unroll
    for (int i = 0; i < kBlock; ++i) {
      if (i >= n) continue;  // uniform
      const size_t row = size_t(g) * t + i0 + i;
      // the new input sits at tap taps - 1
#pragma unroll
      for (int j = 0; j < kMaxTaps; ++j)
        if (j == taps - 1) win[j] = bf16_to_f32(xs[i]);
      if (hist) hist[size_t(taps - 1 + i0 + i) * channels] = xs[i];
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxTaps; ++j)
        if (j < taps) acc = acc + win[j] * wj[j];
      const float v = round_bf16(acc);
      out[row * out_stride + c] = f32_to_bf16(v * sigmoid_bf16(v));
#pragma unroll
      for (int j = 0; j < kMaxTaps - 1; ++j)
        if (j < taps - 1) win[j] = win[j + 1];
    }
  }
#pragma unroll
  for (int j = 0; j < kMaxTaps; ++j)
    if (j < taps - 1) st[size_t(j) * channels] = f32_to_bf16(win[j]);
}

// The same causal conv for long runs of tokens without a window history (a
// prefill chunk): the conv has no recurrence, so each thread takes one
// channel and kConvTok consecutive tokens of one group (grid.y), reading its
// window from the inputs (and, for the first block, from the cached window).
// Same arithmetic as conv_kernel, bit for bit.  Block 0 of each group alone
// reads and rewrites the cached window, so no block reads it after its update.
constexpr int kConvTok = 16;  // >= taps - 1

__global__ __launch_bounds__(256) void conv_tokens_kernel(const uint16_t* __restrict__ qkv,
                                                          int64_t row_stride, int t,
                                                          const int32_t* __restrict__ slots,
                                                          uint16_t* __restrict__ conv_state,
                                                          const float* __restrict__ w,
                                                          int channels, int taps,
                                                          uint16_t* __restrict__ out,
                                                          int64_t out_stride) {
  constexpr int kMaxTaps = 8;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const int t0 = blockIdx.y * kConvTok, g = blockIdx.z;
  if (c >= channels) return;
  uint16_t* st = conv_state + size_t(slots[g]) * (taps - 1) * channels + c;
  const uint16_t* xg = qkv + size_t(g) * t * row_stride + c;
  const int n = t - t0 < kConvTok ? t - t0 : kConvTok;
  // window: inputs t0 - (taps - 1) .. t0 + n - 1 (negative: the cached window)
  float x[kConvTok + kMaxTaps - 1];
#pragma unroll
  for (int j = 0; j < kConvTok + kMaxTaps - 1; ++j) {
    const int i = t0 - (taps - 1) + j;  // input index
    float v = 0.0f;
    if (j < n + taps - 1) {
      if (i >= 0)
        v = bf16_to_f32(xg[size_t(i) * row_stride]);
      else
        v = bf16_to_f32(st[size_t(i + taps - 1) * channels]);
    }
    x[j] = v;
  }
  float wj[kMaxTaps];
#pragma unroll
  for (int j = 0; j < kMaxTaps; ++j) wj[j] = j < taps ? w[size_t(j) * channels + c] : 0.0f;
#pragma unroll
  for (int k = 0; k < kConvTok; ++k) {
    if (k >= n) break;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxTaps; ++j)
      if (j < taps) acc = acc + x[k + j] * wj[j];
    const float v = round_bf16(acc);
    out[(size_t(g) * t + t0 + k) * out_stride + c] = f32_to_bf16(v * sigmoid_bf16(v));
  }
  if (blockIdx.y == 0) {
    // the cached window after the last token: inputs t - (taps - 1) .. t - 1
    for (int j = 0; j < taps - 1; ++j) {
      const int i = t - (taps - 1) + j;
      const float v = i >= 0 ? bf16_to_f32(xg[size_t(i) * row_stride])
                             : x[i - t0 + taps - 1];  // an old cached value (t0 == 0)
      st[size_t(j) * channels] = f32_to_bf16(v);
    }
  }
}

constexpr int kD = 128;  // head dim handled by the recurrence kernel (Dk == Dv == 128)

// Inputs of the delta rule for one token: either computed from the conv
// output and the z/a/b projections (FUSED: L2 norms, beta, decay; the gated
// RMS norm follows the scan) or read as given (the reference's recurrent
// kernel interface: normalised q/k, v, fp32 g, bf16 beta).
struct ScanArgs {
  // fused form
  const uint16_t* conv_out;
  int64_t conv_stride;
  const uint16_t* z;
  const uint16_t* a;
  const uint16_t* b;
  int64_t zab_stride;
  const float* a_log;
  const uint16_t* dt_bias;
  const uint16_t* norm_w;
  float eps;
  // raw form: q, k [rows, hk, 128]; v, y [rows, hv, 128]; g, beta [rows, hv]
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const float* g;
  const uint16_t* beta;
  // common
  int hk_heads, hv_heads, t;
  const int32_t* slots;
  float* state;
  float* history;
  uint16_t* y;
  char* plane;  // nullable: the exact-integer operand plane of y (rows <= 8)
};

// ---------------------------------------------------------------------------
// Delta-rule scan for one (group, value head), in the fixed order of the CPU
// oracle: per value column i, the key-row dot products are four fma chains
// c_r over the key rows d = r mod 4 (ascending), joined as (c0 + c1) +
// (c2 + c3).  512 threads: wave w owns value columns 16 w .. 16 w + 15, lane
// l = 16 r + c column 16 w + c over the key rows d = 4 m + r, m = 0 .. 31
// (chain r), so each thread holds 32 state values and the two joins are the
// lane exchanges l ^ 16 then l ^ 32 (fp32 addition commutes, so all four
// parts end with the oracle's bits).  Sums over 128 values (the q / k L2
// norms, the gated norm) are the oracle's two 64-lane xor butterflies, over
// values 0 .. 63 and 64 .. 127, added.  State loads stay coalesced in 64-byte
// runs (four key rows of 16 columns per wave load).
constexpr int kExactParts = 4;
constexpr int kExactRows = kD / kExactParts;  // key rows per thread
constexpr int kExactThreads = kD * kExactParts;

__device__ __forceinline__ float xor_butterfly64(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

// Tokens are taken in chunks of up to CH (1 for a decode step, kExactChunk
// for verify and prefill blocks).  Before a chunk's
// recurrence, wave w normalises token w's q and k into LDS and every thread
// holds its column's v, z and the token's gates in registers, so the
// recurrence itself runs the chunk's tokens with no barrier; the gated norm
// and the output plane of the chunk's tokens follow it, one wave per token.
// Every value is computed as in the one-token-at-a-time order (the same
// butterflies, chains and roundings), only the schedule differs.
constexpr int kExactChunk = 8;

template <bool FUSED, int CH>
__global__ __launch_bounds__(kExactThreads) void recurrence_kernel(ScanArgs p) {
  static_assert(kExactThreads / 64 >= CH, "a wave per token of a chunk");
  const int hv = blockIdx.x;
  const int g = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, part = lane >> 4;
  const int i = wave * 16 + c;  // value column
  const int hv_heads = p.hv_heads, hk_heads = p.hk_heads;
  const int hk = hv / (hv_heads / hk_heads);
  __shared__ float qs[CH][kD], ks[CH][kD], ys[CH][kD];
  __shared__ float red[CH];
  __shared__ __align__(16) uint16_t yb[CH][kD];  // y rows (plane only)

  // a token's per-column inputs as raw bits: v of column i, b / a (or beta,
  // g) and z
  struct In {
    uint16_t v, b, a, z;
    float g;
  };
  auto load_in = [&](size_t row) {
    In r{};
    if constexpr (FUSED) {
      const uint16_t* cr = p.conv_out + row * p.conv_stride;
      r.v = cr[2 * hk_heads * kD + hv * kD + i];
      r.b = p.b[row * p.zab_stride + hv];
      r.a = p.a[row * p.zab_stride + hv];
      r.z = p.z[row * p.zab_stride + hv * kD + i];
    } else {
      r.v = p.v[(row * hv_heads + hv) * kD + i];
      r.b = p.beta[row * hv_heads + hv];
      r.g = p.g[row * hv_heads + hv];
    }
    return r;
  };
  // wave w's raw q / k of chunk token w: lanes hold values lane, 64 + lane
  auto load_qk = [&](size_t row, uint16_t (&qk)[4]) {
    if constexpr (FUSED) {
      const uint16_t* cr = p.conv_out + row * p.conv_stride;
      qk[0] = cr[hk * kD + lane];
      qk[1] = cr[hk * kD + 64 + lane];
      qk[2] = cr[(hk_heads + hk) * kD + lane];
      qk[3] = cr[(hk_heads + hk) * kD + 64 + lane];
    } else {
      const uint16_t* qr = p.q + (row * hk_heads + hk) * kD;
      const uint16_t* kr = p.k + (row * hk_heads + hk) * kD;
      qk[0] = qr[lane];
      qk[1] = qr[64 + lane];
      qk[2] = kr[lane];
      qk[3] = kr[64 + lane];
    }
  };
  const size_t row0 = size_t(g) * p.t;
  // the first chunk's inputs are requested before the state, so the q / k
  // norms run while the state streams in
  In in[CH];
  uint16_t qk[4] = {0, 0, 0, 0};
  {
    const int n0 = p.t < CH ? p.t : CH;
    if (wave < n0) load_qk(row0 + wave, qk);
#pragma unroll
    for (int k = 0; k < CH; ++k)
      if (k < n0) in[k] = load_in(row0 + k);
  }

  const size_t my_off = size_t(part) * kD + i;
  float* sp = p.state + (size_t(p.slots[g]) * hv_heads + hv) * kD * kD + my_off;
  float s[kExactRows];  // s[m]: key row 4 m + part of column i
#pragma unroll
  for (int m = 0; m < kExactRows; ++m) s[m] = sp[size_t(m) * kExactParts * kD];

  const float eps_l2 = round_bf16(1e-6f);
  const float qscale = round_bf16(0.08838834764831845f);  // bf16(Dk^-1/2), Dk = 128
  float neg_a = 0.0f, dt = 0.0f, nw = 0.0f;
  if constexpr (FUSED) {
    neg_a = -expf_(p.a_log[hv]);
    dt = bf16_to_f32(p.dt_bias[hv]);
    nw = bf16_to_f32(p.norm_w[i]);
  }

  for (int c0 = 0; c0 < p.t; c0 += CH) {
    const int n = p.t - c0 < CH ? p.t - c0 : CH;
    // LDS of the previous chunk (qs, ks, ys, red, yb) is read by every wave
    // before this barrier
    if (c0 > 0) {
      __syncthreads();
      if (wave < n) load_qk(row0 + c0 + wave, qk);
#pragma unroll
      for (int k = 0; k < CH; ++k)
        if (k < n) in[k] = load_in(row0 + c0 + k);
    }
    if (wave < n) {
      const float q0 = bf16_to_f32(qk[0]), q1 = bf16_to_f32(qk[1]);
      const float k0 = bf16_to_f32(qk[2]), k1 = bf16_to_f32(qk[3]);
      if constexpr (FUSED) {
        // x * rsqrt(sum(x^2) + eps) with bf16 operations (hybrid.rs:409-413)
        const float qss = round_bf16(xor_butterfly64(round_bf16(q0 * q0)) +
                                     xor_butterfly64(round_bf16(q1 * q1)));
        const float kss = round_bf16(xor_butterfly64(round_bf16(k0 * k0)) +
                                     xor_butterfly64(round_bf16(k1 * k1)));
        const float rq = round_bf16(1.0f / __builtin_sqrtf(round_bf16(qss + eps_l2)));
        const float rk = round_bf16(1.0f / __builtin_sqrtf(round_bf16(kss + eps_l2)));
        qs[wave][lane] = round_bf16(round_bf16(q0 * rq) * qscale);
        qs[wave][64 + lane] = round_bf16(round_bf16(q1 * rq) * qscale);
        ks[wave][lane] = round_bf16(k0 * rk);
        ks[wave][64 + lane] = round_bf16(k1 * rk);
      } else {
        qs[wave][lane] = q0;
        qs[wave][64 + lane] = q1;
        ks[wave][lane] = k0;
        ks[wave][64 + lane] = k1;
      }
    }
    __syncthreads();

    float yo[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      yo[k] = 0.0f;
      if (k >= n) continue;  // uniform
      const size_t row = row0 + c0 + k;
      float vi, beta, gdecay;
      if constexpr (FUSED) {
        vi = bf16_to_f32(in[k].v);
        beta = sigmoid_bf16(bf16_to_f32(in[k].b));
        const float x = round_bf16(bf16_to_f32(in[k].a) + dt);
        gdecay = expf_(neg_a * softplus_bf16(x));
      } else {
        vi = bf16_to_f32(in[k].v);
        beta = bf16_to_f32(in[k].b);
        gdecay = in[k].g;
      }
      // state *= g; chain `part` of kv = sum_d s[d] k[d]
      float cp = 0.0f;
#pragma unroll
      for (int m = 0; m < kExactRows; ++m) {
        s[m] = s[m] * gdecay;
        cp = fmaf_(s[m], ks[k][kExactParts * m + part], cp);
      }
      float kv = cp + __shfl_xor(cp, 16, 64);  // c0 + c1 (parts 0, 1), c2 + c3 (parts 2, 3)
      kv = kv + __shfl_xor(kv, 32, 64);        // (c0 + c1) + (c2 + c3)
      const float delta = (vi - kv) * beta;
      float op = 0.0f;
#pragma unroll
      for (int m = 0; m < kExactRows; ++m) {
        s[m] = fmaf_(ks[k][kExactParts * m + part], delta, s[m]);
        op = fmaf_(s[m], qs[k][kExactParts * m + part], op);
      }
      float os = op + __shfl_xor(op, 16, 64);
      os = os + __shfl_xor(os, 32, 64);
      yo[k] = round_bf16(os);
      if (p.history) {
        float* hp = p.history + ((row * hv_heads + hv) * kD) * kD + my_off;
#pragma unroll
        for (int m = 0; m < kExactRows; ++m) hp[size_t(m) * kExactParts * kD] = s[m];
      }
      if constexpr (FUSED) {
        if (part == 0) ys[k][i] = yo[k];
      } else {
        if (part == 0) p.y[row * (size_t(hv_heads) * kD) + hv * kD + i] = f32_to_bf16(yo[k]);
      }
    }
    if constexpr (FUSED) {
      // fast::rms_norm(y, w, eps) then * sigmoid(z) in f32 (hybrid.rs:447-452):
      // wave w sums token w's squares, then every column normalises
      __syncthreads();
      if (wave < n) {
        const float y0 = ys[wave][lane], y1 = ys[wave][64 + lane];
        const float ss = xor_butterfly64(y0 * y0) + xor_butterfly64(y1 * y1);
        if (lane == 0) red[wave] = ss;
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        if (k >= n) continue;
        const size_t row = row0 + c0 + k;
        const float inv = 1.0f / __builtin_sqrtf(red[k] / float(kD) + p.eps);
        const float normed = round_bf16(nw * round_bf16(yo[k] * inv));
        const float zi = bf16_to_f32(in[k].z);
        const uint16_t yv = f32_to_bf16(normed * sigmoidf_(zi));
        if (part == 0) {
          p.y[row * (size_t(hv_heads) * kD) + hv * kD + i] = yv;
          yb[k][i] = yv;
        }
      }
      if (p.plane) {
        // each token's two 64-value groups of this head, digitised by wave
        // `token` (lanes 16 kb + gl, gl < 2), for the output projection
        __syncthreads();
        if (wave < n) {
          const int kb = lane >> 4, gl = lane & 15;
          float f[16];
          const bool unit = gl < kD / xq::kGroup;
#pragma unroll
          for (int q = 0; q < 16; ++q)
            f[q] = unit ? bf16_to_f32(yb[wave][gl * xq::kGroup + 16 * kb + q]) : 0.0f;
          xq::digitize_unit(f, int(row0 + c0 + wave), hv * (kD / xq::kGroup) + (unit ? gl : 0), kb,
                            unit, p.plane, hv_heads * (kD / xq::kGroup));
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kExactRows; ++m) sp[size_t(m) * kExactParts * kD] = s[m];
}

// ---------------------------------------------------------------------------
// Fast-mode step, same inputs and outputs as recurrence_kernel<true> (t tokens
// per group, optional per-token history; each token's arithmetic is the same
// whatever t is, so a verify block matches one-token decode steps bit for
// bit): wave 0 forms the q / k L2 norms with lane shuffles, q and k reach the
// threads through LDS as float4, the state's key
// rows are split four ways among lanes (fp32 dot products summed in another
// order than the exact step), and the scalar functions use the hardware exp2 /
// log2 / reciprocal / rsqrt.  The bf16 rounding points of the exact step (the
// reference's bf16 operations) are kept, so the step stays within the north
// star's tolerances of the exact one layer after layer.
__device__ __forceinline__ float exp_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + exp_fast(-x));
}
// The bf16-rounded logistic and softplus of the exact step (the reference's
// bf16 operations), with the hardware exp2 / log2 / reciprocal inside.
__device__ __forceinline__ float sigmoid_bf16_fast(float x) {
  const float e = round_bf16(exp_fast(__builtin_fabsf(x)));
  const float d = round_bf16(1.0f + e);
  const float y = round_bf16(__builtin_amdgcn_rcpf(d));
  return x < 0.0f ? y : round_bf16(1.0f - y);
}
__device__ __forceinline__ float softplus_bf16_fast(float x) {
  const float hi = x > 0.0f ? x : 0.0f;
  const float lo = x > 0.0f ? 0.0f : x;
  const float e = round_bf16(exp_fast(round_bf16(lo - hi)));
  // log1p(e): series below 2^-10, where log2(1 + e) would lose the low bits
  const float l = e < 0x1p-10f ? e - 0.5f * e * e
                               : __builtin_amdgcn_logf(1.0f + e) * 0.6931471805599453f;
  return round_bf16(hi + round_bf16(l));
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

// 512 threads per (value head, row): wave w owns value columns 16 w .. 16 w
// + 15, lane l = 16 part + c column 16 w + c over the key rows 32 part .. 32
// part + 31, so a thread holds 32 state values and every key-row dot product
// ends in an exchange over the four parts (lanes l ^ 16, l ^ 32).  State
// loads stay coalesced in 64-byte runs per part.
constexpr int kFastParts = 4;
constexpr int kFastRows = kD / kFastParts;  // key rows per thread
constexpr int kFastThreads = kD * kFastParts;

// Wave 0: the key head's q and k, L2-normalised (q also scaled by
// bf16(dk^-1/2)) at the exact step's bf16 rounding points, into LDS as
// float4.  q0 / q1 are q[lane] / q[64 + lane], k likewise.
// The fast step's L2 norms of one token's q and k (one key head, one wave:
// lane l holds dims l and 64 + l of each): qk = {q_l, q_64+l, k_l, k_64+l},
// bf16 values.
__device__ __forceinline__ void fast_qk_values(float q0, float q1, float k0, float k1,
                                               float (&qk)[4]) {
  const float eps_l2 = round_bf16(1e-6f);
  const float qscale = round_bf16(0.08838834764831845f);  // bf16(Dk^-1/2), Dk = 128
  const float qss = round_bf16(wave_sum(round_bf16(q0 * q0) + round_bf16(q1 * q1)));
  const float kss = round_bf16(wave_sum(round_bf16(k0 * k0) + round_bf16(k1 * k1)));
  const float rq = round_bf16(__builtin_amdgcn_rsqf(round_bf16(qss + eps_l2)));
  const float rk = round_bf16(__builtin_amdgcn_rsqf(round_bf16(kss + eps_l2)));
  qk[0] = round_bf16(round_bf16(q0 * rq) * qscale);
  qk[1] = round_bf16(round_bf16(q1 * rq) * qscale);
  qk[2] = round_bf16(k0 * rk);
  qk[3] = round_bf16(k1 * rk);
}

__device__ __forceinline__ void fast_qk_norm(float q0, float q1, float k0, float k1, float4* qs4,
                                             float4* ks4) {
  const int lane = threadIdx.x & 63;
  float qk[4];
  fast_qk_values(q0, q1, k0, k1, qk);
  float* qs = reinterpret_cast<float*>(qs4);
  float* ks = reinterpret_cast<float*>(ks4);
  qs[lane] = qk[0];
  qs[64 + lane] = qk[1];
  ks[lane] = qk[2];
  ks[64 + lane] = qk[3];
}

// The decay gate exp(-exp(a_log) softplus(bf16(a + dt_bias))) and beta =
// sigmoid(b) of value head hv, row `row`.
__device__ __forceinline__ void fast_gates(const ScanArgs& p, int hv, int row, float& beta,
                                           float& gdecay) {
  const float bv = bf16_to_f32(p.b[size_t(row) * p.zab_stride + hv]);
  const float av = bf16_to_f32(p.a[size_t(row) * p.zab_stride + hv]);
  beta = sigmoid_bf16_fast(bv);
  const float x = round_bf16(av + bf16_to_f32(p.dt_bias[hv]));
  gdecay = exp_fast(-exp_fast(p.a_log[hv]) * softplus_bf16_fast(x));
}

// One thread's share of the delta rule: its 32 state values s (key rows
// 32 part .. of value column i) are decayed, their k dot product is summed
// over the four parts, the column's delta applied, the new values stored
// through sp when it is not null; returns the column's q dot product (summed
// over the parts).
__device__ __forceinline__ float fast_delta(float (&s)[kFastRows], float* sp, const float4* ks4,
                                            const float4* qs4, int part, float gdecay,
                                            float beta, float vi) {
  const float4* kp = ks4 + part * (kFastRows / 4);
  const float4* qp = qs4 + part * (kFastRows / 4);
  float c0 = 0.0f, c1 = 0.0f, c2 = 0.0f, c3 = 0.0f;
#pragma unroll
  for (int d4 = 0; d4 < kFastRows / 4; ++d4) {
    const float4 kv4 = kp[d4];
    const int d = 4 * d4;
    s[d] = s[d] * gdecay;
    s[d + 1] = s[d + 1] * gdecay;
    s[d + 2] = s[d + 2] * gdecay;
    s[d + 3] = s[d + 3] * gdecay;
    c0 = fmaf_(s[d], kv4.x, c0);
    c1 = fmaf_(s[d + 1], kv4.y, c1);
    c2 = fmaf_(s[d + 2], kv4.z, c2);
    c3 = fmaf_(s[d + 3], kv4.w, c3);
  }
  float cs = (c0 + c1) + (c2 + c3);
  cs = cs + __shfl_xor(cs, 16, 64);
  cs = cs + __shfl_xor(cs, 32, 64);
  const float delta = (vi - cs) * beta;
  float o0 = 0.0f, o1 = 0.0f, o2 = 0.0f, o3 = 0.0f;
#pragma unroll
  for (int d4 = 0; d4 < kFastRows / 4; ++d4) {
    const float4 kv4 = kp[d4], qv4 = qp[d4];
    const int d = 4 * d4;
    s[d] = fmaf_(kv4.x, delta, s[d]);
    s[d + 1] = fmaf_(kv4.y, delta, s[d + 1]);
    s[d + 2] = fmaf_(kv4.z, delta, s[d + 2]);
    s[d + 3] = fmaf_(kv4.w, delta, s[d + 3]);
    o0 = fmaf_(s[d], qv4.x, o0);
    o1 = fmaf_(s[d + 1], qv4.y, o1);
    o2 = fmaf_(s[d + 2], qv4.z, o2);
    o3 = fmaf_(s[d + 3], qv4.w, o3);
  }
  if (sp) {
#pragma unroll
    for (int d = 0; d < kFastRows; ++d) sp[size_t(d) * kD] = s[d];
  }
  float os = (o0 + o1) + (o2 + o3);
  os = os + __shfl_xor(os, 16, 64);
  os = os + __shfl_xor(os, 32, 64);
  return os;
}

// Wave w's share of a value head's output sum of squares (part 0 of each
// column enters: the four parts hold the same value).
__device__ __forceinline__ float fast_sq_part(float yo, int part) {
  return wave_sum(part == 0 ? yo * yo : 0.0f);
}

// BLOCK = false: the one-token decode form (t = 1, no history), with no token
// loop in the code; BLOCK = true: t tokens per group and optional history.
// Both run the same per-token arithmetic, so their bits agree.
template <bool BLOCK>
__global__ __launch_bounds__(kFastThreads) void recurrence_fast_kernel(ScanArgs p) {
  const int hv = blockIdx.x;
  const int g = blockIdx.y;  // group: p.t consecutive tokens of one slot
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 15, part = lane >> 4;
  const int i = wave * 16 + c;  // value column
  const int hv_heads = p.hv_heads, hk_heads = p.hk_heads;
  const int hk = hv / (hv_heads / hk_heads);
  __shared__ float4 qs4[kD / 4], ks4[kD / 4];
  __shared__ float red[kFastThreads / 64];
  const size_t my_off = size_t(part * kFastRows) * kD + i;
  float* sp = p.state + (size_t(p.slots[g]) * hv_heads + hv) * kD * kD + my_off;
  float s[kFastRows];
#pragma unroll
  for (int d = 0; d < kFastRows; ++d) s[d] = sp[size_t(d) * kD];
  const float nw = bf16_to_f32(p.norm_w[i]);
  // Every token runs the single-token step's arithmetic on the registers'
  // state, so a block of t tokens gives the bits of t one-token launches.
  // LDS reuse across tokens: qs4 / ks4 are rewritten only after the barrier
  // that follows every wave's reads of them, red only after the next
  // token's first barrier, which every wave reaches after reading it.
  const int T = BLOCK ? p.t : 1;
  float* const history = BLOCK ? p.history : nullptr;
  for (int step = 0; step < T; ++step) {
    const size_t row = size_t(g) * T + step;
    const uint16_t* cr = p.conv_out + row * p.conv_stride;
    const float vi = bf16_to_f32(cr[2 * hk_heads * kD + hv * kD + i]);
    const float zi = bf16_to_f32(p.z[row * p.zab_stride + hv * kD + i]);
    if (wave == 0)
      fast_qk_norm(bf16_to_f32(cr[hk * kD + lane]), bf16_to_f32(cr[hk * kD + 64 + lane]),
                   bf16_to_f32(cr[(hk_heads + hk) * kD + lane]),
                   bf16_to_f32(cr[(hk_heads + hk) * kD + 64 + lane]), qs4, ks4);
    float beta, gdecay;
    fast_gates(p, hv, int(row), beta, gdecay);
    __syncthreads();
    // the state after this token: into the history row when there is one,
    // else into the cache after the last token
    float* dst = history ? history + (row * hv_heads + hv) * kD * kD + my_off
                         : (step == T - 1 ? sp : nullptr);
    const float yo = round_bf16(fast_delta(s, dst, ks4, qs4, part, gdecay, beta, vi));
    const float ws = fast_sq_part(yo, part);
    if (lane == 0) red[wave] = ws;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < kFastThreads / 64; ++w) tot = tot + red[w];
    const float inv = __builtin_amdgcn_rsqf(tot * (1.0f / kD) + p.eps);
    if (part == 0) {
      const float normed = round_bf16(nw * round_bf16(yo * inv));
      p.y[row * (size_t(hv_heads) * kD) + hv * kD + i] = f32_to_bf16(normed * sigmoid_fast(zi));
    }
  }
  if (history) {
#pragma unroll
    for (int d = 0; d < kFastRows; ++d) sp[size_t(d) * kD] = s[d];
  }
}

// ---------------------------------------------------------------------------
// A prefill chunk's fast GDN step through the chunked scan (gdn_chunk.hip).
// Inputs per token row: normalised q / k of every key head (fast_qk_values)
// and the decay and beta of every value head (fast_gates); the scan's output
// then takes the gated RMS norm of the fast step.
struct ChunkIo {
  uint16_t* q;     // [rows][hk][kD] bf16
  uint16_t* k;     // [rows][hk][kD] bf16
  float* g;        // [rows][hv]
  uint16_t* beta;  // [rows][hv] bf16
};

__host__ __device__ inline size_t chunk_io_align(size_t b) { return (b + 255) / 256 * 256; }

__host__ __device__ inline ChunkIo chunk_io(void* io, int rows, int hk, int hv) {
  char* p = static_cast<char*>(io);
  ChunkIo c;
  const size_t qk = chunk_io_align(size_t(rows) * hk * kD * 2);
  c.q = reinterpret_cast<uint16_t*>(p);
  c.k = reinterpret_cast<uint16_t*>(p + qk);
  c.g = reinterpret_cast<float*>(p + 2 * qk);
  c.beta = reinterpret_cast<uint16_t*>(p + 2 * qk + chunk_io_align(size_t(rows) * hv * 4));
  return c;
}

// One workgroup per token row: wave w normalises key heads w, w + 4, ...;
// threads below hv give the value heads' gates.
__global__ __launch_bounds__(256) void chunk_inputs_kernel(ScanArgs p, ChunkIo io) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint16_t* cr = p.conv_out + size_t(row) * p.conv_stride;
  for (int kh = wave; kh < p.hk_heads; kh += 4) {
    float qk[4];
    fast_qk_values(bf16_to_f32(cr[kh * kD + lane]), bf16_to_f32(cr[kh * kD + 64 + lane]),
                   bf16_to_f32(cr[(p.hk_heads + kh) * kD + lane]),
                   bf16_to_f32(cr[(p.hk_heads + kh) * kD + 64 + lane]), qk);
    uint16_t* qo = io.q + (size_t(row) * p.hk_heads + kh) * kD;
    uint16_t* ko = io.k + (size_t(row) * p.hk_heads + kh) * kD;
    qo[lane] = f32_to_bf16(qk[0]);
    qo[64 + lane] = f32_to_bf16(qk[1]);
    ko[lane] = f32_to_bf16(qk[2]);
    ko[64 + lane] = f32_to_bf16(qk[3]);
  }
  for (int hv = threadIdx.x; hv < p.hv_heads; hv += 256) {
    float beta, gdecay;
    fast_gates(p, hv, row, beta, gdecay);
    io.g[size_t(row) * p.hv_heads + hv] = gdecay;
    io.beta[size_t(row) * p.hv_heads + hv] = f32_to_bf16(beta);
  }
}

// Gated RMS norm of the scan's output, in place: one wave per (value head,
// row), lane l holding values l and 64 + l.
__global__ __launch_bounds__(64) void chunk_norm_kernel(ScanArgs p) {
  const int hv = blockIdx.x, row = blockIdx.y, lane = threadIdx.x;
  uint16_t* yr = p.y + (size_t(row) * p.hv_heads + hv) * kD;
  const float y0 = bf16_to_f32(yr[lane]), y1 = bf16_to_f32(yr[64 + lane]);
  const float tot = wave_sum(y0 * y0 + y1 * y1);
  const float inv = __builtin_amdgcn_rsqf(tot * (1.0f / kD) + p.eps);
  const uint16_t* zr = p.z + size_t(row) * p.zab_stride + hv * kD;
  const float o0 = round_bf16(bf16_to_f32(p.norm_w[lane]) * round_bf16(y0 * inv));
  const float o1 = round_bf16(bf16_to_f32(p.norm_w[64 + lane]) * round_bf16(y1 * inv));
  yr[lane] = f32_to_bf16(o0 * sigmoid_fast(bf16_to_f32(zr[lane])));
  yr[64 + lane] = f32_to_bf16(o1 * sigmoid_fast(bf16_to_f32(zr[64 + lane])));
}

}  // namespace

int gdn_recurrence_fast(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                        const uint16_t* a, const uint16_t* b, int64_t zab_stride,
                        const float* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                        float eps, GdnDims d, int groups, int t, const int32_t* slots,
                        float* state, float* history, uint16_t* y, hipStream_t s) {
  if (d.dk != kD || d.dv != kD || d.hk <= 0 || d.hv % d.hk != 0) return MX_EUNSUPPORTED;
  if (groups <= 0) return MX_OK;
  if (t < 1) return MX_EINVAL;
  ScanArgs p{};
  p.conv_out = conv_out; p.conv_stride = conv_stride; p.z = z; p.a = a; p.b = b;
  p.zab_stride = zab_stride; p.a_log = a_log; p.dt_bias = dt_bias; p.norm_w = norm_w; p.eps = eps;
  p.hk_heads = d.hk; p.hv_heads = d.hv; p.t = t; p.slots = slots; p.state = state;
  p.history = history; p.y = y;
  if (t == 1 && !history)
    hipLaunchKernelGGL(recurrence_fast_kernel<false>, dim3(d.hv, groups), dim3(kFastThreads), 0, s,
                       p);
  else
    hipLaunchKernelGGL(recurrence_fast_kernel<true>, dim3(d.hv, groups), dim3(kFastThreads), 0, s,
                       p);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

size_t gdn_chunk_io_bytes(int rows, GdnDims d) {
  return 2 * chunk_io_align(size_t(rows) * d.hk * kD * 2) +
         chunk_io_align(size_t(rows) * d.hv * 4) + chunk_io_align(size_t(rows) * d.hv * 2);
}

int gdn_chunk_fast(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                   const uint16_t* a, const uint16_t* b, int64_t zab_stride, const float* a_log,
                   const uint16_t* dt_bias, const uint16_t* norm_w, float eps, GdnDims d,
                   int groups, int t, const int32_t* slots, float* state, uint16_t* y, void* io,
                   float* workspace, hipStream_t s) {
  if (d.dk != kD || d.dv != kD || d.hk <= 0 || d.hv % d.hk != 0) return MX_EUNSUPPORTED;
  if (groups <= 0) return MX_OK;
  if (t < 1) return MX_EINVAL;
  const int rows = groups * t;
  ScanArgs p{};
  p.conv_out = conv_out; p.conv_stride = conv_stride; p.z = z; p.a = a; p.b = b;
  p.zab_stride = zab_stride; p.a_log = a_log; p.dt_bias = dt_bias; p.norm_w = norm_w; p.eps = eps;
  p.hk_heads = d.hk; p.hv_heads = d.hv; p.t = t; p.slots = slots; p.state = state; p.y = y;
  const ChunkIo c = chunk_io(io, rows, d.hk, d.hv);
  hipLaunchKernelGGL(chunk_inputs_kernel, dim3(rows), dim3(256), 0, s, p, c);
  // v: the conv output's value channels, row stride conv_stride
  if (int rc = gdn_prefill_chunked(c.q, c.k, conv_out + 2 * d.hk * kD, c.g, c.beta, d, groups, t,
                                   slots, state, y, workspace, s, conv_stride);
      rc != MX_OK)
    return rc;
  hipLaunchKernelGGL(chunk_norm_kernel, dim3(d.hv, rows), dim3(64), 0, s, p);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int gdn_conv(const uint16_t* qkv, int64_t row_stride, int groups, int t, const int32_t* slots,
             uint16_t* conv_state, const float* conv_w, int channels, int conv_k, uint16_t* out,
             int64_t out_stride, uint16_t* window_history, hipStream_t s) {
  if (conv_k < 2 || conv_k > 8) return MX_EUNSUPPORTED;
  if (groups <= 0) return MX_OK;
  if (!window_history && t > kConvTok) {  // long runs: tokens spread over workgroups
    const dim3 grid((channels + 255) / 256, (t + kConvTok - 1) / kConvTok, groups);
    hipLaunchKernelGGL(conv_tokens_kernel, grid, dim3(256), 0, s, qkv, row_stride, t, slots,
                       conv_state, conv_w, channels, conv_k, out, out_stride);
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
  }
  const dim3 grid((channels + 255) / 256, groups);
  hipLaunchKernelGGL(conv_kernel, grid, dim3(256), 0, s, qkv, row_stride, t, slots, conv_state,
                     conv_w, channels, conv_k, out, out_stride, window_history);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int gdn_recurrence(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                   const uint16_t* a, const uint16_t* b, int64_t zab_stride, const float* a_log,
                   const uint16_t* dt_bias, const uint16_t* norm_w, float eps, GdnDims d,
                   int groups, int t, const int32_t* slots, float* state, float* history,
                   uint16_t* y, hipStream_t s, char* plane) {
  if (d.dk != kD || d.dv != kD || d.hk <= 0 || d.hv % d.hk != 0) return MX_EUNSUPPORTED;
  ScanArgs p{};
  p.conv_out = conv_out; p.conv_stride = conv_stride; p.z = z; p.a = a; p.b = b;
  p.zab_stride = zab_stride; p.a_log = a_log; p.dt_bias = dt_bias; p.norm_w = norm_w; p.eps = eps;
  p.hk_heads = d.hk; p.hv_heads = d.hv; p.t = t; p.slots = slots; p.state = state;
  p.history = history; p.y = y;
  p.plane = groups * t <= 8 ? plane : nullptr;
  if (t == 1)
    hipLaunchKernelGGL((recurrence_kernel<true, 1>), dim3(d.hv, groups), dim3(kExactThreads), 0,
                       s, p);
  else
    hipLaunchKernelGGL((recurrence_kernel<true, kExactChunk>), dim3(d.hv, groups),
                       dim3(kExactThreads), 0, s, p);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

int gdn_scan(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
             const uint16_t* beta, GdnDims d, int groups, int t, const int32_t* slots,
             float* state, float* history, uint16_t* y, hipStream_t s) {
  if (d.dk != kD || d.dv != kD || d.hk <= 0 || d.hv % d.hk != 0) return MX_EUNSUPPORTED;
  ScanArgs p{};
  p.q = q; p.k = k; p.v = v; p.g = g; p.beta = beta;
  p.hk_heads = d.hk; p.hv_heads = d.hv; p.t = t; p.slots = slots; p.state = state;
  p.history = history; p.y = y;
  if (t == 1)
    hipLaunchKernelGGL((recurrence_kernel<false, 1>), dim3(d.hv, groups), dim3(kExactThreads), 0,
                       s, p);
  else
    hipLaunchKernelGGL((recurrence_kernel<false, kExactChunk>), dim3(d.hv, groups),
                       dim3(kExactThreads), 0, s, p);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
