// Epilogues of the 1..8-row projection kernels (the ProjEpilogue modes),
// shared by the bf16 matrix-core kernels (skinny.hip) and the exact-integer
// kernels (xq.hip).  A workgroup owns NC output columns (rows of the weight
// matrix) of all activation rows; its fp32 projection values sit in LDS as
// yt[m][c] (m < 8, c < NC) when finish() runs, and every arithmetic step
// after that value is the same in both families:
//   kPlain   y = bf16(v)
//   kHcDown  t = bf16(bf16(v) / hc); rows < rank: bf16(t silu-gated), the
//            hc inject rows: bf16(2 sigmoid(t))
//   kHcUpMix out = bf16(bf16(sum_s bf16(sigmoid(bf16(v_s)) xn_s)) / 4)
//   kHcWrite residual_s += bf16(bf16(v) inj_s)  (one stream per thread)
//   kConv    the causal conv of the column's cached window and bf16(v),
//            bf16(silu(bf16(conv))), window shifted in place
// (reference src/hybrid.rs:78-105, src/compiled.rs:22-95).
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace mx {

template <int MODE, int NC, int NT>
struct ProjFinish {
  // kConv with one output per thread: the thread's slot is read before the
  // weight stream, its window and conv weights right after it
  static constexpr bool kConvPre = MODE == kConv && 8 * NC <= NT;
  // activation rows this workgroup writes: [m_lo, min(m_hi, M))
  int m_lo = 0, m_hi = 8;
  int cm = 0, cr = 0, cslot = 0;
  bool conv_item = false;
  uint16_t cwin[kConvMaxTaps - 1] = {};
  float cw[kConvMaxTaps] = {};

  // window taps and weights at indices clamped to the last real one, so the
  // loads stay unconditional within the item
  __device__ __forceinline__ static void conv_fetch(const ProjEpilogue& e, int slot, int r,
                                                    uint16_t (&win)[kConvMaxTaps - 1],
                                                    float (&wt)[kConvMaxTaps]) {
    const uint16_t* stp = e.conv_state + size_t(slot) * (e.taps - 1) * e.conv_ch + r;
#pragma unroll
    for (int j = 0; j < kConvMaxTaps - 1; ++j) win[j] = stp[size_t(min(j, e.taps - 2)) * e.conv_ch];
#pragma unroll
    for (int j = 0; j < kConvMaxTaps; ++j) wt[j] = e.conv_w[size_t(min(j, e.taps - 1)) * e.conv_ch + r];
  }

  __device__ __forceinline__ void begin(const ProjEpilogue& e, int tg, int M, int n) {
    if constexpr (kConvPre) {
      cm = threadIdx.x / NC;
      cr = tg * NC + threadIdx.x % NC;
      conv_item = cm >= m_lo && cm < min(M, m_hi) && cr < min(n, e.conv_ch);
      if (conv_item) cslot = e.slots[cm];
    }
  }

  __device__ __forceinline__ void prefetch(const ProjEpilogue& e) {
    if constexpr (kConvPre)
      if (conv_item) conv_fetch(e, cslot, cr, cwin, cw);
  }

  // tg: the workgroup's column block (kHcUpMix: columns tg*16 .. +15 of the
  // four streams, tile s at yt column s*16 + j).
  __device__ __forceinline__ void finish(const float* yt, const ProjEpilogue& e, int tg, int M,
                                         int n) {
    if constexpr (MODE == kHcUpMix) {
      // 8 rows x 16 columns; each output mixes the four streams of its column
      if (threadIdx.x >= 128) return;
      const int m = threadIdx.x >> 4, cj = threadIdx.x & 15;
      const int c = tg * 16 + cj;
      if (m < m_lo || m >= min(M, m_hi) || c >= e.hidden) return;
      float sum = 0.0f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float p = round_bf16(yt[m * NC + s * 16 + cj]);
        const float xn = bf16_to_f32(e.xn[size_t(m) * e.xn_stride + size_t(s) * e.hidden + c]);
        sum = sum + round_bf16(sigmoid_bf16(p) * xn);
      }
      e.y[size_t(m) * e.y_stride + c] = f32_to_bf16(round_bf16(sum) / 4.0f);
    } else if constexpr (MODE == kConv) {
      for (int i = threadIdx.x; i < 8 * NC; i += NT) {
        const int m = i / NC, c = i - m * NC;
        const int r = tg * NC + c;
        if (m < m_lo || m >= min(M, m_hi) || r >= n) continue;
        const uint16_t xb = f32_to_bf16(yt[i]);
        if (r >= e.conv_ch) {
          e.y[size_t(m) * e.y_stride + r] = xb;
          continue;
        }
        uint16_t win[kConvMaxTaps - 1];
        float wt[kConvMaxTaps];
        const int slot = kConvPre ? cslot : e.slots[m];
        if constexpr (kConvPre) {
#pragma unroll
          for (int j = 0; j < kConvMaxTaps - 1; ++j) win[j] = cwin[j];
#pragma unroll
          for (int j = 0; j < kConvMaxTaps; ++j) wt[j] = cw[j];
        } else {
          conv_fetch(e, slot, r, win, wt);
        }
        // acc = sum_j fl(x_j * w_j) over the window then the new value
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kConvMaxTaps - 1; ++j)
          if (j < e.taps - 1) acc = acc + bf16_to_f32(win[j]) * wt[j];
        acc = acc + bf16_to_f32(xb) * wt[kConvMaxTaps - 1];
        const float v = round_bf16(acc);
        e.conv_out[size_t(m) * e.conv_stride + r] = f32_to_bf16(v * sigmoid_bf16(v));
        uint16_t* stp = e.conv_state + size_t(slot) * (e.taps - 1) * e.conv_ch + r;
#pragma unroll
        for (int j = 0; j < kConvMaxTaps - 2; ++j)
          if (j < e.taps - 2) stp[size_t(j) * e.conv_ch] = win[j + 1];
        stp[size_t(e.taps - 2) * e.conv_ch] = xb;
      }
    } else if constexpr (MODE == kHcWrite) {
      // one residual stream per thread: the read-modify-writes of a column's
      // streams are independent, so none waits on another's load
      for (int i = threadIdx.x; i < 8 * NC * e.hc; i += NT) {
        const int s = i / (8 * NC), mc = i - s * (8 * NC);
        const int m = mc / NC, c = mc - m * NC;
        const int r = tg * NC + c;
        if (m < m_lo || m >= min(M, m_hi) || r >= n) continue;
        const float vb = round_bf16(yt[mc]);
        uint16_t* res = e.y + size_t(m) * e.y_stride + size_t(s) * n + r;
        const float inj = round_bf16(vb * bf16_to_f32(e.aux[size_t(m) * e.aux_stride + s]));
        *res = f32_to_bf16(bf16_to_f32(*res) + inj);
      }
    } else {
      for (int i = threadIdx.x; i < 8 * NC; i += NT) {
        const int m = i / NC, c = i - m * NC;
        const int r = tg * NC + c;
        if (m < m_lo || m >= min(M, m_hi) || r >= n) continue;
        const float v = yt[i];
        if constexpr (MODE == kPlain) {
          e.y[size_t(m) * e.y_stride + r] = f32_to_bf16(v);
        } else {  // kHcDown
          const float tt = round_bf16(round_bf16(v) / float(e.hc));
          if (r < e.rank)
            e.y[size_t(m) * e.y_stride + r] = f32_to_bf16(tt * sigmoid_bf16(tt));
          else
            e.aux[size_t(m) * e.aux_stride + (r - e.rank)] = f32_to_bf16(sigmoid_bf16(tt) * 2.0f);
        }
      }
    }
  }
};

}  // namespace mx
