// Gated full attention for decode / verify rows (gfx950).
//
// Reference: Attention::forward_selection with gated = true (src/dense.rs:139-270):
// q/gate projection split per head, zero-centred q/k norms (compiled::norm,
// src/compiled.rs:22-28), partial text RoPE (src/rope.rs:8-57,
// kernels/text_rope.metal), KV append (KvCache::update, src/dense.rs:46-110),
// scaled dot-product attention over the cached positions (MLX
// fast::scaled_dot_product_attention), output * sigmoid(gate).
//
// Every row carries its own (slot, position): rows of one decode step may sit
// at different offsets, and rows of one verify block attend causally (row r
// sees positions <= pos[r]).  The cache holds K and V as bf16
// [slot][layer][kv_head][position][head_dim].
//
// Decoding splits each row's positions into chunks of kAttnChunk; a workgroup
// handles one (chunk, kv head, row) for all q heads sharing the kv head, so K
// and V stream once per group.  A second pass combines the chunks.
#include <type_traits>
#include <utility>

#include "common.hpp"
#include "kernels.hpp"
#include "skinny_core.hpp"
#include "xq_core.hpp"

namespace mx {

namespace {

constexpr int kMaxHd = 256;
constexpr int kMaxGroup = 16;  // q heads per kv head

// ---------------------------------------------------------------------------
// One wave per (row, head): zero-centred RMS norm over head_dim, then RoPE on
// the first rotary_dim values (halves rotated), written to q_out (q heads) or
// appended to the cache (k heads; v heads are appended unchanged).
// Norm: lane l sums x^2 over l, l+64, ... in order, xor butterfly;
// y = bf16((x * rsqrt(mean + eps)) * (w + 1)).
// RoPE: out[i] = bf16(x1 c - x2 s), out[i+h] = bf16(x2 c + x1 s), c/s from the
// fp32 table of the row's position.
__global__ __launch_bounds__(64) void prep_kernel(const uint16_t* __restrict__ qkv,
                                                  int64_t qkv_stride,
                                                  const int32_t* __restrict__ slots,
                                                  const int32_t* __restrict__ pos,
                                                  const uint16_t* __restrict__ q_norm,
                                                  const uint16_t* __restrict__ k_norm, float eps,
                                                  const float* __restrict__ rope_cos,
                                                  const float* __restrict__ rope_sin,
                                                  AttnDims d, uint16_t* __restrict__ q_out,
                                                  uint16_t* __restrict__ k_cache,
                                                  uint16_t* __restrict__ v_cache) {
  __shared__ float buf[kMaxHd];
  const int head = blockIdx.x;  // [0, heads) q, [heads, heads + kv) k, then v
  const int row = blockIdx.y;
  const int lane = threadIdx.x;
  const int hd = d.head_dim;
  const uint16_t* xr = qkv + size_t(row) * qkv_stride;
  const int p = pos[row];
  const size_t cache_off =
      size_t(slots[row]) * d.slot_stride;  // + (kvh * max_ctx + p) * hd below
  if (head >= d.heads + d.kv_heads) {
    const int kvh = head - d.heads - d.kv_heads;
    const uint16_t* src = xr + size_t(d.heads) * 2 * hd + size_t(d.kv_heads) * hd + size_t(kvh) * hd;
    uint16_t* dst = v_cache + cache_off + (size_t(kvh) * d.max_ctx + p) * hd;
    for (int c = lane; c < hd; c += 64) dst[c] = src[c];
    return;
  }
  const bool is_q = head < d.heads;
  const int h = is_q ? head : head - d.heads;
  const uint16_t* src = is_q ? xr + size_t(h) * 2 * hd  // [heads, 2, hd]: q then gate
                             : xr + size_t(d.heads) * 2 * hd + size_t(h) * hd;
  const uint16_t* w = is_q ? q_norm : k_norm;
  float acc = 0.0f;
  for (int c = lane; c < hd; c += 64) {
    const float v = bf16_to_f32(src[c]);
    acc = acc + v * v;
  }
  for (int o = 32; o > 0; o >>= 1) acc = acc + __shfl_xor(acc, o, 64);
  const float inv = 1.0f / __builtin_sqrtf(acc / float(hd) + eps);
  for (int c = lane; c < hd; c += 64)
    buf[c] = round_bf16((bf16_to_f32(src[c]) * inv) * (bf16_to_f32(w[c]) + 1.0f));
  __syncthreads();
  uint16_t* dst = is_q ? q_out + (size_t(row) * d.heads + h) * hd
                       : k_cache + cache_off + (size_t(h) * d.max_ctx + p) * hd;
  const int half = d.rotary_dim / 2;
  const float* cs = rope_cos + size_t(p) * half;
  const float* sn = rope_sin + size_t(p) * half;
  for (int c = lane; c < hd; c += 64) {
    float v;
    if (c < half) {
      v = buf[c] * cs[c] - buf[c + half] * sn[c];
    } else if (c < 2 * half) {
      const int i = c - half;
      v = buf[c] * cs[i] + buf[i] * sn[i];
    } else {
      v = buf[c];
    }
    dst[c] = f32_to_bf16(v);
  }
}

// ---------------------------------------------------------------------------
// Partial attention of one chunk for the G q heads of one kv head.
// Scores: thread t owns position j = chunk*C + t; s = (q . k_j) * scale, the dot
// as four interleaved fma chains over d (d mod 4), then (c0+c1)+(c2+c3).
// m = max_t s; p = e^(s - m); l = sum_t p (xor butterfly per wave, waves in
// order).  Values: wave w takes the chunk's positions 64 w .. 64 w + 63 and
// lane l the dims DPL l .. DPL l + DPL - 1 (DPL = head_dim / 64); per (head,
// dim) one fma chain over the wave's positions ascending, then the four
// waves' sums added in wave order, ((o0 + o1) + o2) + o3.  Writes (m, l) and
// o (fp32) per (row, head, chunk).  A workgroup takes G of the kv head's q
// heads (`splits` workgroups per kv head), so short contexts still spread
// over many workgroups.
template <int G, int DPL>
__global__ __launch_bounds__(kAttnChunk) void decode_kernel(
    const uint16_t* __restrict__ q, const int32_t* __restrict__ slots,
    const int32_t* __restrict__ pos, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, AttnDims d, int max_chunks, float scale,
    float* __restrict__ o_part, float* __restrict__ ml_part, int chunks, int rows) {
  static_assert(kAttnChunk == 256, "four waves of 64 positions");
  __shared__ float qs[G][kMaxHd];
  __shared__ float ps[G][kAttnChunk];
  __shared__ float red[G][4];
  __shared__ float ow[4][G][64 * DPL];
  // one-dimensional grid placed by XCD: workgroups go to the eight XCDs in
  // turn (id mod 8), so the `splits` workgroups of one (chunk, kv head, row)
  // -- which read the same K and V rows -- take ids congruent mod 8 and
  // share one L2
  const int splits = d.heads / d.kv_heads / G;
  const int b = blockIdx.x, xcd = b & 7, k8 = b >> 3;
  const int group = (k8 / splits) * 8 + xcd;  // (chunk, kv head, row)
  const int split = k8 - (k8 / splits) * splits;
  if (group >= chunks * d.kv_heads * rows) return;  // padding (uniform)
  const int chunk = group % chunks;
  const int kvh = (group / chunks) % d.kv_heads;
  const int h0 = kvh * (G * splits) + split * G;  // first q head
  const int row = group / (chunks * d.kv_heads);
  const int t = threadIdx.x;
  const int n_pos = pos[row] + 1;
  const int j0 = chunk * kAttnChunk;
  if (j0 >= n_pos) return;  // uniform per workgroup
  const int hd = d.head_dim;  // 64 DPL (checked on the host)
  const size_t base = size_t(slots[row]) * d.slot_stride + size_t(kvh) * d.max_ctx * hd;
  const int j = j0 + t;
  const bool valid = j < n_pos;
  const int wave = t >> 6, lane = t & 63;
  // the position's whole K row is requested before the q heads are staged
  // (one memory round trip); a position past the row's end reads the chunk's
  // first row, which is in bounds, and ignores it
  constexpr int N8 = 8 * DPL;  // 16-byte pieces per row
  uint4 raw[N8];
  {
    const uint4* kr = reinterpret_cast<const uint4*>(k_cache + base + size_t(valid ? j : j0) * hd);
#pragma unroll
    for (int b = 0; b < N8; ++b) raw[b] = kr[b];
  }
  for (int i = t; i < G * hd; i += kAttnChunk) {
    const int g = i / hd, c = i - g * hd;
    qs[g][c] = bf16_to_f32(q[(size_t(row) * d.heads + h0 + g) * hd + c]);
  }
  __syncthreads();
  if (valid) {
    // fma order: chain d mod 4, dims ascending
    float c0[G], c1[G], c2[G], c3[G];
    for (int g = 0; g < G; ++g) c0[g] = c1[g] = c2[g] = c3[g] = 0.0f;
#pragma unroll
    for (int b = 0; b < N8; ++b) {
      const int c = b * 8;
      const float kv[8] = {u2f(raw[b].x << 16), u2f(raw[b].x & 0xffff0000u),
                           u2f(raw[b].y << 16), u2f(raw[b].y & 0xffff0000u),
                           u2f(raw[b].z << 16), u2f(raw[b].z & 0xffff0000u),
                           u2f(raw[b].w << 16), u2f(raw[b].w & 0xffff0000u)};
      for (int g = 0; g < G; ++g) {
        c0[g] = fmaf_(qs[g][c + 0], kv[0], c0[g]);
        c1[g] = fmaf_(qs[g][c + 1], kv[1], c1[g]);
        c2[g] = fmaf_(qs[g][c + 2], kv[2], c2[g]);
        c3[g] = fmaf_(qs[g][c + 3], kv[3], c3[g]);
        c0[g] = fmaf_(qs[g][c + 4], kv[4], c0[g]);
        c1[g] = fmaf_(qs[g][c + 5], kv[5], c1[g]);
        c2[g] = fmaf_(qs[g][c + 6], kv[6], c2[g]);
        c3[g] = fmaf_(qs[g][c + 7], kv[7], c3[g]);
      }
    }
    for (int g = 0; g < G; ++g) ps[g][t] = ((c0[g] + c1[g]) + (c2[g] + c3[g])) * scale;
  } else {
    for (int g = 0; g < G; ++g) ps[g][t] = u2f(0xff800000u);
  }
  // the wave's V rows (positions 64 wave .. +63 before the row's end; lane:
  // DPL dims) are requested now and arrive during the softmax
  using VT = typename std::conditional<DPL == 4, uint2,
             typename std::conditional<DPL == 2, uint32_t, uint16_t>::type>::type;
  const int jend = min(n_pos - j0, kAttnChunk);
  const int ja = wave * 64, jb = min(jend, ja + 64);
  const int nv = jb > ja ? jb - ja : 0;  // uniform per wave
  VT vraw[64];
  {
    // positions past the wave's last one reload that one (in bounds, unused)
    const VT* vr = reinterpret_cast<const VT*>(v_cache + base + size_t(j0) * hd) + lane;
    const size_t vstride = size_t(hd) / DPL;  // VT elements per position
    const int last = nv > 0 ? jb - 1 : 0;
#pragma unroll
    for (int b = 0; b < 64; ++b) vraw[b] = vr[size_t(min(ja + b, last)) * vstride];
  }
  __syncthreads();
  // per-head max and sum over the chunk
  for (int g = 0; g < G; ++g) {
    float m = ps[g][t];
    for (int o = 32; o > 0; o >>= 1) {
      const float v = __shfl_xor(m, o, 64);
      m = v > m ? v : m;
    }
    if ((t & 63) == 0) red[g][wave] = m;
  }
  __syncthreads();
  float mg[G];
  for (int g = 0; g < G; ++g) {
    float m = red[g][0];
    for (int w = 1; w < kAttnChunk / 64; ++w) m = red[g][w] > m ? red[g][w] : m;
    mg[g] = m;
  }
  __syncthreads();
  for (int g = 0; g < G; ++g) {
    const float pv = valid ? expf_(ps[g][t] - mg[g]) : 0.0f;
    ps[g][t] = pv;
    float l = pv;
    for (int o = 32; o > 0; o >>= 1) l = l + __shfl_xor(l, o, 64);
    if ((t & 63) == 0) red[g][wave] = l;
  }
  __syncthreads();
  const int heads = d.heads;
  if (t < G) {
    const int g = t;
    float l = red[g][0];
    for (int w = 1; w < kAttnChunk / 64; ++w) l = l + red[g][w];
    float* ml = ml_part + ((size_t(row) * heads + h0 + g) * max_chunks + chunk) * 2;
    ml[0] = mg[g];
    ml[1] = l;
  }
  {
    // values: per (head, dim) one fma chain over the wave's positions
    float o[G][DPL];
    for (int g = 0; g < G; ++g)
      for (int i = 0; i < DPL; ++i) o[g][i] = 0.0f;
#pragma unroll
    for (int b = 0; b < 64; ++b) {
      if (b >= nv) continue;  // uniform per wave
      float v[DPL];
      if constexpr (DPL == 4) {
        v[0] = u2f(vraw[b].x << 16), v[1] = u2f(vraw[b].x & 0xffff0000u);
        v[2] = u2f(vraw[b].y << 16), v[3] = u2f(vraw[b].y & 0xffff0000u);
      } else if constexpr (DPL == 2) {
        v[0] = u2f(vraw[b] << 16), v[1] = u2f(vraw[b] & 0xffff0000u);
      } else {
        v[0] = bf16_to_f32(vraw[b]);
      }
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int i = 0; i < DPL; ++i) o[g][i] = fmaf_(ps[g][ja + b], v[i], o[g][i]);
    }
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int i = 0; i < DPL; ++i) ow[wave][g][lane * DPL + i] = o[g][i];
  }
  __syncthreads();
  if (t < hd) {
    for (int g = 0; g < G; ++g)
      o_part[((size_t(row) * heads + h0 + g) * max_chunks + chunk) * hd + t] =
          ((ow[0][g][t] + ow[1][g][t]) + ow[2][g][t]) + ow[3][g][t];
  }
}

// ---------------------------------------------------------------------------
// Matrix-core decode (fast mode): a workgroup of four waves handles
// kAttnFastChunk = 64 positions of one (row, kv head), 16 per wave, for all G
// q heads of the kv head.
// Scores: one v_mfma_f32_16x16x32_bf16 per 32 dims with A = the q heads (row
// = head, rows >= G zero) and B = the wave's 16 K rows (column = position),
// both read straight from memory as 16-byte pieces: lane l = 16 qd + j loads
// dims 32 kk + 8 qd .. +7 of q head j and of position j, so one MFMA step
// covers 16 positions x 64 bytes of K.  Lane l then holds the scores of heads
// 4 qd .. +3 at position j.
// Softmax: max and sum per head over the 16 lanes of a quarter (xor
// butterfly), then over the four waves through LDS; p = e^(s - m) into LDS.
// Values: wave w owns dims [w HD/4, (w+1) HD/4) in 8-dim blocks; lane
// (position group pg, block db) accumulates o[g][8] over positions pg,
// pg + NPG, ... (one 16-byte V load each, all issued together), and the
// position groups are summed with xor shuffles.  Positions past the row's
// length load the last valid row (always in bounds) and weigh it 0.
template <int G, int HD>
__global__ __launch_bounds__(256) void decode_fast_kernel(
    const uint16_t* __restrict__ q, const int32_t* __restrict__ slots,
    const int32_t* __restrict__ pos, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, AttnDims d, int max_chunks, float scale,
    float* __restrict__ o_part, float* __restrict__ ml_part) {
  constexpr int C = kAttnFastChunk;
  constexpr int KS = HD / 32;  // MFMA steps over the head dim
  __shared__ float ps[16][C];
  __shared__ float red[2][4][16];
  const int chunk = blockIdx.x;
  const int kvh = blockIdx.y;
  const int row = blockIdx.z;
  const int t = threadIdx.x;
  const int wave = t >> 6, lane = t & 63;
  const int j = lane & 15, qd = lane >> 4;
  const int n_pos = pos[row] + 1;
  const int j0 = chunk * C;
  if (j0 >= n_pos) return;  // uniform per workgroup
  const size_t base = size_t(slots[row]) * d.slot_stride + size_t(kvh) * d.max_ctx * HD;

  const int p = j0 + 16 * wave + j;
  const bool valid = p < n_pos;
  const uint16_t* kr = k_cache + base + size_t(valid ? p : n_pos - 1) * HD + qd * 8;
  const uint16_t* qr = q + (size_t(row) * d.heads + kvh * G + (j < G ? j : 0)) * HD + qd * 8;
  uint4 kb[KS], qa[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) kb[kk] = *reinterpret_cast<const uint4*>(kr + kk * 32);
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    const uint4 v = *reinterpret_cast<const uint4*>(qr + kk * 32);
    qa[kk] = j < G ? v : make_uint4(0u, 0u, 0u, 0u);
  }
  // the value rows go out with the keys: their addresses do not depend on
  // the scores, so one memory round trip serves both
  constexpr int DB = HD / 32;   // 8-dim blocks per wave
  constexpr int NPG = 64 / DB;  // position groups per wave
  constexpr int PPL = C / NPG;  // positions per lane
  const int db = lane % DB, pg = lane / DB;
  const int dim0 = wave * (HD / 4) + db * 8;
  uint4 vv[PPL];
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const int pp = j0 + pg + NPG * i;
    vv[i] = *reinterpret_cast<const uint4*>(v_cache + base + size_t(pp < n_pos ? pp : n_pos - 1) * HD +
                                            dim0);
  }
  sk::floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) acc = sk::mfma(qa[kk], kb[kk], acc);

  float s[4], e[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = valid ? acc[i] * scale : u2f(0xff800000u);
    float m = s[i];
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
      const float v = __shfl_xor(m, o, 64);
      m = v > m ? v : m;
    }
    if (j == 0) red[0][wave][4 * qd + i] = m;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * qd + i;
    float m = red[0][0][h];
#pragma unroll
    for (int w = 1; w < 4; ++w) m = red[0][w][h] > m ? red[0][w][h] : m;
    e[i] = valid ? expf_(s[i] - m) : 0.0f;
    ps[h][16 * wave + j] = e[i];
    float l = e[i];
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) l = l + __shfl_xor(l, o, 64);
    if (j == 0) red[1][wave][h] = l;
  }
  __syncthreads();
  if (t < G) {
    float m = red[0][0][t], l = red[1][0][t];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      m = red[0][w][t] > m ? red[0][w][t] : m;
      l = l + red[1][w][t];
    }
    float* ml = ml_part + ((size_t(row) * d.heads + kvh * G + t) * max_chunks + chunk) * 2;
    ml[0] = m;
    ml[1] = l;
  }

  float o[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int c = 0; c < 8; ++c) o[g][c] = 0.0f;
#pragma unroll
  for (int i = 0; i < PPL; ++i) {
    const uint4 r = vv[i];
    const float v[8] = {u2f(r.x << 16), u2f(r.x & 0xffff0000u), u2f(r.y << 16),
                        u2f(r.y & 0xffff0000u), u2f(r.z << 16), u2f(r.z & 0xffff0000u),
                        u2f(r.w << 16), u2f(r.w & 0xffff0000u)};
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float pr = ps[g][pg + NPG * i];
#pragma unroll
      for (int c = 0; c < 8; ++c) o[g][c] = fmaf_(pr, v[c], o[g][c]);
    }
  }
#pragma unroll
  for (int off = DB; off < 64; off <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int c = 0; c < 8; ++c) o[g][c] = o[g][c] + __shfl_xor(o[g][c], off, 64);
  if (pg == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float4* dst = reinterpret_cast<float4*>(
          o_part + ((size_t(row) * d.heads + kvh * G + g) * max_chunks + chunk) * HD + dim0);
      dst[0] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
      dst[1] = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
    }
  }
}

// Combines the chunks of one (row, head) and applies the output gate:
//   M = max m_c; w_c = e^(m_c - M); L = sum l_c w_c; O = sum o_c w_c (fma, c
//   ascending); y = bf16(bf16(O / L) * sigmoid_bf16(gate)).
__global__ __launch_bounds__(kMaxHd) void combine_kernel(const float* __restrict__ o_part,
                                                         const float* __restrict__ ml_part,
                                                         const uint16_t* __restrict__ qkv,
                                                         int64_t qkv_stride,
                                                         const int32_t* __restrict__ pos,
                                                         AttnDims d, int max_chunks,
                                                         int chunk,
                                                         uint16_t* __restrict__ out,
                                                         char* __restrict__ plane) {
  __shared__ __align__(16) uint16_t ob[kMaxHd];  // the head's output row (plane only)
  const int h = blockIdx.x;
  const int row = blockIdx.y;
  const int t = threadIdx.x;
  const int hd = d.head_dim;
  if (t < hd) {
  const int chunks = (pos[row] + chunk) / chunk;
  const float* ml = ml_part + (size_t(row) * d.heads + h) * max_chunks * 2;
  const float* op = o_part + (size_t(row) * d.heads + h) * max_chunks * hd + t;
  float M = ml[0];
  for (int c = 1; c < chunks; ++c) M = ml[2 * c] > M ? ml[2 * c] : M;
  float L = 0.0f, O = 0.0f;
  for (int c = 0; c < chunks; ++c) {
    const float wc = expf_(ml[2 * c] - M);
    L = fmaf_(ml[2 * c + 1], wc, L);
    O = fmaf_(op[size_t(c) * hd], wc, O);
  }
  const float attn = round_bf16(O / L);
  const float gate = bf16_to_f32(qkv[size_t(row) * qkv_stride + size_t(h) * 2 * hd + hd + t]);
  const uint16_t o = f32_to_bf16(attn * sigmoid_bf16(gate));
  out[(size_t(row) * d.heads + h) * hd + t] = o;
  ob[t] = o;
  }
  if (!plane) return;
  // the head's hd / 64 groups of this row, digitised by wave 0 (lanes
  // 16 kb + gl, gl < hd / 64), for the output projection
  __syncthreads();
  if (t < 64) {
    const int kb = t >> 4, gl = t & 15, ng = hd / xq::kGroup;
    const bool unit = gl < ng;
    float f[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) f[q] = unit ? bf16_to_f32(ob[gl * xq::kGroup + 16 * kb + q]) : 0.0f;
    xq::digitize_unit(f, row, h * ng + (unit ? gl : 0), kb, unit, plane, d.heads * ng);
  }
}

// Fast-mode combine (matrix-core decode partials, 64-position chunks): the
// chunk weights w_c = e^(m_c - M) are formed once per chunk by threads c and
// shared through LDS (hardware exp2); L = sum_c l_c w_c as a block sum;
// O[d] = sum_c o_c[d] w_c (fma, c ascending); y = bf16(bf16(O / L) * sigmoid(gate)).
// chunks <= 256 (max_ctx <= 16384, checked on the host).
__global__ __launch_bounds__(256) void combine_fast_kernel(const float* __restrict__ o_part,
                                                           const float* __restrict__ ml_part,
                                                           const uint16_t* __restrict__ qkv,
                                                           int64_t qkv_stride,
                                                           const int32_t* __restrict__ pos,
                                                           AttnDims d, int max_chunks,
                                                           int chunk_len,
                                                           uint16_t* __restrict__ out) {
  __shared__ float wsh[256];
  __shared__ float red[2][4];
  const int h = blockIdx.x;
  const int row = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int hd = d.head_dim;
  const int chunks = (pos[row] + chunk_len) / chunk_len;
  const float* ml = ml_part + (size_t(row) * d.heads + h) * max_chunks * 2;
  const float* op = o_part + (size_t(row) * d.heads + h) * max_chunks * hd + min(t, hd - 1);
  const float gate =
      bf16_to_f32(qkv[size_t(row) * qkv_stride + size_t(h) * 2 * hd + hd + min(t, hd - 1)]);
  const float mc = t < chunks ? ml[2 * t] : u2f(0xff800000u);
  const float lc = t < chunks ? ml[2 * t + 1] : 0.0f;
  float m = mc;
  for (int o = 32; o > 0; o >>= 1) {
    const float v = __shfl_xor(m, o, 64);
    m = v > m ? v : m;
  }
  if (lane == 0) red[0][wave] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
  const float wc = t < chunks ? __builtin_amdgcn_exp2f((mc - M) * 1.4426950408889634f) : 0.0f;
  wsh[t] = wc;
  float l = lc * wc;
  for (int o = 32; o > 0; o >>= 1) l = l + __shfl_xor(l, o, 64);
  if (lane == 0) red[1][wave] = l;
  __syncthreads();
  if (t >= hd) return;
  const float L = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  float O = 0.0f;
  int c = 0;
  for (; c + 4 <= chunks; c += 4) {
    const float a0 = op[size_t(c) * hd], a1 = op[size_t(c + 1) * hd];
    const float a2 = op[size_t(c + 2) * hd], a3 = op[size_t(c + 3) * hd];
    O = fmaf_(a0, wsh[c], O);
    O = fmaf_(a1, wsh[c + 1], O);
    O = fmaf_(a2, wsh[c + 2], O);
    O = fmaf_(a3, wsh[c + 3], O);
  }
  for (; c < chunks; ++c) O = fmaf_(op[size_t(c) * hd], wsh[c], O);
  const float attn = round_bf16(O * __builtin_amdgcn_rcpf(L));
  const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gate * 1.4426950408889634f));
  out[(size_t(row) * d.heads + h) * hd + t] = f32_to_bf16(attn * sg);
}

// ---------------------------------------------------------------------------
// Prefill attention on the matrix cores (fast mode, a chunk of query rows of
// one slot): a workgroup of eight waves takes QB = 8 * 16 / G query rows, one
// kv head and one split of kPfSplit key positions, so the key and value rows
// of a tile are read once for all QB rows x G heads.  Wave w owns one M tile
// of 16 (row, head) pairs: pair i = row qb0 + w * 16 / G + i / G, head
// kvh * G + i % G.  Per tile of kPfKeys keys: K rows and V (transposed) are
// staged in LDS; S = Q K^T on the matrix cores (Q held as A operands for the
// whole launch); the online softmax per pair (max and sum over the 16 lanes
// of a quarter and the tile's four 16-key columns, hardware exp2); P goes
// through LDS into A-operand order as two bf16 parts (hi + lo), and O += P V
// on the matrix cores (fp32 accumulators, rescaled by e^(m_old - m_new)).
// The split's (m, l, O) per pair go to o_part / ml_part at chunk index =
// split, which combine_fast_kernel merges with chunk length kPfSplit.  Rows of
// one query block must share a slot (a prefill chunk's rows do).
constexpr int kPfKeys = 64;     // keys per tile
constexpr int kPfSplit = 256;   // keys per split (one partial per pair and split)
static_assert(attn_prefill_splits(kPfSplit + 1) == 2, "attn_prefill_splits counts kPfSplit keys");
constexpr int kPfKLd = kMaxHd + 8;      // padded K row in LDS (bf16)
constexpr int kPfVLd = kPfKeys + 8;     // padded transposed-V row (bf16)

template <int HD>
__host__ __device__ constexpr int prefill_attn_lds() {
  return (kPfKeys * kPfKLd + HD * kPfVLd + 8 * 2 * 16 * kPfVLd) * 2;
}

template <int G, int HD>
__global__ __launch_bounds__(512) void prefill_attn_kernel(
    const uint16_t* __restrict__ q, int rows, const int32_t* __restrict__ slots,
    const int32_t* __restrict__ pos, const uint16_t* __restrict__ k_cache,
    const uint16_t* __restrict__ v_cache, AttnDims d, int max_chunks, float scale,
    float* __restrict__ o_part, float* __restrict__ ml_part) {
  constexpr int RPW = 16 / G;       // query rows per wave
  constexpr int QB = 8 * RPW;       // query rows per workgroup
  constexpr int KS = HD / 32;       // MFMA steps over the head dim
  constexpr int NO = HD / 16;       // 16-dim output tiles
  extern __shared__ __align__(16) uint16_t pf_lds[];
  uint16_t* ks = pf_lds;                              // [kPfKeys][kPfKLd]
  uint16_t* vt = ks + kPfKeys * kPfKLd;               // [HD][kPfVLd]
  uint16_t* pw = vt + HD * kPfVLd;                    // [8 waves][hi, lo][16][kPfVLd]
  __shared__ int blk_max;
  const int split = blockIdx.x, kvh = blockIdx.y, qb0 = blockIdx.z * QB;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int j = lane & 15, kq = lane >> 4;
  if (t == 0) {
    int mx = -1;
    for (int r = qb0; r < min(qb0 + QB, rows); ++r) mx = max(mx, pos[r]);
    blk_max = mx;
  }
  __syncthreads();
  const int key0 = split * kPfSplit;
  const int kend = min(key0 + kPfSplit, blk_max + 1);  // keys [key0, kend)
  if (key0 >= kend) return;                             // uniform
  const size_t base = size_t(slots[qb0]) * d.slot_stride + size_t(kvh) * d.max_ctx * HD;
  // this lane's A-operand pair (j) and the D-layout pairs 4 kq + r
  const int arow = qb0 + wave * RPW + j / G;
  const bool alive = arow < rows;
  const uint16_t* qr =
      q + (size_t(alive ? arow : 0) * d.heads + kvh * G + j % G) * HD + 8 * kq;
  uint4 qa[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k)
    qa[k] = alive ? *reinterpret_cast<const uint4*>(qr + 32 * k) : make_uint4(0u, 0u, 0u, 0u);
  int lim[4];  // exclusive key limit of D-layout pair 4 kq + r
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = qb0 + wave * RPW + (4 * kq + r) / G;
    lim[r] = row < rows ? min(pos[row] + 1, kend) : key0;
  }
  const float sl2 = scale * 1.4426950408889634f;  // scores in log2 units
  float m_run[4], l_run[4];
  sk::floatx4_t o[NO];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m_run[r] = u2f(0xff800000u);
    l_run[r] = 0.0f;
  }
#pragma unroll
  for (int n = 0; n < NO; ++n) o[n] = sk::floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
  uint16_t* ph = pw + wave * 2 * 16 * kPfVLd;
  uint16_t* pl = ph + 16 * kPfVLd;
  // a tile's K pieces and V key pairs per thread, loaded one tile ahead
  constexpr int KPT = kPfKeys * HD / 8 / 512, VPT = (kPfKeys / 2) * (HD / 8) / 512;
  static_assert(KPT * 512 == kPfKeys * HD / 8 && VPT * 512 == (kPfKeys / 2) * (HD / 8),
                "tile pieces divide among 512 threads");
  uint4 kr[KPT], va[VPT], vb[VPT];
  // constant indices from the start, so the arrays stay in registers
  auto load_k = [&](int kt, int u) {
    const int i = t + 512 * u, key = i / (HD / 8), pc = i % (HD / 8);
    const int kk = min(kt + key, kend - 1);  // keys past kend: the last valid one
    return *reinterpret_cast<const uint4*>(k_cache + base + size_t(kk) * HD + 8 * pc);
  };
  auto load_v = [&](int kt, int u, int second) {
    const int i = t + 512 * u;
    const int kp = i % (kPfKeys / 2), dg = i / (kPfKeys / 2);  // neighbours: keys (banks)
    const int kk = min(kt + 2 * kp + second, kend - 1);
    return *reinterpret_cast<const uint4*>(v_cache + base + size_t(kk) * HD + 8 * dg);
  };
#define MX_PF_LOAD(KT)                                                                  \
  {                                                                                     \
    const int kt_ = (KT);                                                               \
    [&]<int... U>(std::integer_sequence<int, U...>) {                                   \
      ((kr[U] = load_k(kt_, U)), ...);                                                  \
    }(std::make_integer_sequence<int, KPT>{});                                          \
    [&]<int... U>(std::integer_sequence<int, U...>) {                                   \
      ((va[U] = load_v(kt_, U, 0), vb[U] = load_v(kt_, U, 1)), ...);                    \
    }(std::make_integer_sequence<int, VPT>{});                                          \
  }
  MX_PF_LOAD(key0)
  for (int kt = key0; kt < kend; kt += kPfKeys) {
    __syncthreads();  // the previous tile's K, V and P are consumed
    // K rows; V transposed, one 32-bit word (two keys) per dim
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int i = t + 512 * u, key = i / (HD / 8), pc = i % (HD / 8);
      *reinterpret_cast<uint4*>(ks + key * kPfKLd + 8 * pc) = kr[u];
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int i = t + 512 * u;
      const int kp = i % (kPfKeys / 2), dg = i / (kPfKeys / 2);
      const uint32_t av[4] = {va[u].x, va[u].y, va[u].z, va[u].w};
      const uint32_t bv[4] = {vb[u].x, vb[u].y, vb[u].z, vb[u].w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        *reinterpret_cast<uint32_t*>(vt + (8 * dg + 2 * w) * kPfVLd + 2 * kp) =
            (av[w] & 0xffffu) | (bv[w] << 16);
        *reinterpret_cast<uint32_t*>(vt + (8 * dg + 2 * w + 1) * kPfVLd + 2 * kp) =
            (av[w] >> 16) | (bv[w] & 0xffff0000u);
      }
    }
    __syncthreads();
    if (kt + kPfKeys < kend) MX_PF_LOAD(kt + kPfKeys)  // in flight during this tile's work
    // S = Q K^T: four 16-key columns; lane (j, kq) gets pairs 4 kq + r at key kt + 16 c + j
    sk::floatx4_t sc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      sc[c] = sk::floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k = 0; k < KS; ++k)
        sc[c] = sk::mfma(qa[k],
                         *reinterpret_cast<const uint4*>(ks + (16 * c + j) * kPfKLd + 32 * k + 8 * kq),
                         sc[c]);
    }
    // online softmax per pair
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float mt = u2f(0xff800000u);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bool v = kt + 16 * c + j < lim[r];
        sc[c][r] = v ? sc[c][r] * sl2 : u2f(0xff800000u);
        mt = fmaxf(mt, sc[c][r]);
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) mt = fmaxf(mt, __shfl_xor(mt, off, 64));
      const float mn = fmaxf(m_run[r], mt);
      const bool none = mn == u2f(0xff800000u);  // no valid key yet
      const float alpha = none || m_run[r] == u2f(0xff800000u)
                              ? 0.0f
                              : __builtin_amdgcn_exp2f(m_run[r] - mn);
      float ls = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float pv = none || sc[c][r] == u2f(0xff800000u)
                             ? 0.0f
                             : __builtin_amdgcn_exp2f(sc[c][r] - mn);
        sc[c][r] = pv;
        ls += pv;
      }
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) ls += __shfl_xor(ls, off, 64);
      l_run[r] = l_run[r] * alpha + ls;
      m_run[r] = mn;
#pragma unroll
      for (int n = 0; n < NO; ++n) o[n][r] *= alpha;
    }
    // P (pair 4 kq + r, key 16 c + j) into LDS as bf16 hi and lo
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = sc[c][r];
        const __bf16 h = __bf16(pv);
        const float hf = float(h);
        ph[(4 * kq + r) * kPfVLd + 16 * c + j] = __builtin_bit_cast(uint16_t, h);
        pl[(4 * kq + r) * kPfVLd + 16 * c + j] = __builtin_bit_cast(uint16_t, __bf16(pv - hf));
      }
    __syncthreads();
    // O += P V: A = P (pair j, keys 32 s + 8 kq ..), B = V^T rows (dim 16 n + j)
#pragma unroll
    for (int st = 0; st < kPfKeys / 32; ++st) {
      const uint4 ah = *reinterpret_cast<const uint4*>(ph + j * kPfVLd + 32 * st + 8 * kq);
      const uint4 al = *reinterpret_cast<const uint4*>(pl + j * kPfVLd + 32 * st + 8 * kq);
#pragma unroll
      for (int n = 0; n < NO; ++n) {
        const uint4 bv = *reinterpret_cast<const uint4*>(vt + (16 * n + j) * kPfVLd + 32 * st + 8 * kq);
        o[n] = sk::mfma(ah, bv, o[n]);
        o[n] = sk::mfma(al, bv, o[n]);
      }
    }
  }
#undef MX_PF_LOAD
  // partials of this split (chunk index = split)
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * kq + r;
    const int row = qb0 + wave * RPW + i / G;
    if (row >= rows) continue;
    const size_t ph_ = (size_t(row) * d.heads + kvh * G + i % G) * max_chunks + split;
#pragma unroll
    for (int n = 0; n < NO; ++n) o_part[ph_ * HD + 16 * n + j] = o[n][r];
    if (j == 0) {
      // m in natural-log units, as the decode kernels write it
      ml_part[ph_ * 2] = m_run[r] * 0.6931471805599453f;
      ml_part[ph_ * 2 + 1] = l_run[r];
    }
  }
}

}  // namespace

int attn_prep(const uint16_t* qkv, int64_t qkv_stride, int rows, const int32_t* slots,
              const int32_t* pos, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
              const float* rope_cos, const float* rope_sin, AttnDims d, uint16_t* q_out,
              uint16_t* k_cache, uint16_t* v_cache, hipStream_t s) {
  if (d.head_dim > kMaxHd || d.head_dim % 8 != 0) return MX_EUNSUPPORTED;
  hipLaunchKernelGGL(prep_kernel, dim3(d.heads + 2 * d.kv_heads, rows), dim3(64), 0, s, qkv,
                     qkv_stride, slots, pos, q_norm, k_norm, eps, rope_cos, rope_sin, d, q_out,
                     k_cache, v_cache);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

bool attn_fast_supported(AttnDims d) {
  if (d.kv_heads <= 0 || d.heads % d.kv_heads != 0) return false;
  const int g = d.heads / d.kv_heads;
  return (d.head_dim == 128 || d.head_dim == 256) && (g == 1 || g == 2 || g == 4 || g == 8) &&
         d.slot_stride % 8 == 0 && d.max_ctx <= 256 * kAttnFastChunk;
}

int attn_decode(const uint16_t* q, int rows, const int32_t* slots, const int32_t* pos,
                const uint16_t* k_cache, const uint16_t* v_cache, AttnDims d, int max_chunks,
                bool fast, float* o_part, float* ml_part, hipStream_t s) {
  if (d.head_dim > kMaxHd || d.heads % d.kv_heads != 0 || d.heads / d.kv_heads > kMaxGroup)
    return MX_EUNSUPPORTED;
  const float scale = 1.0f / __builtin_sqrtf(float(d.head_dim));
  if (fast) {
    if (!attn_fast_supported(d)) return MX_EUNSUPPORTED;
    const int chunks = (d.max_ctx + kAttnFastChunk - 1) / kAttnFastChunk;
    if (chunks > max_chunks) return MX_EINVAL;
    const dim3 grid(chunks, d.kv_heads, rows);
#define MX_FDEC(GG, HH)                                                                       \
  if (d.heads / d.kv_heads == GG && d.head_dim == HH) {                                       \
    hipLaunchKernelGGL((decode_fast_kernel<GG, HH>), grid, dim3(256), 0, s, q, slots, pos,    \
                       k_cache, v_cache, d, max_chunks, scale, o_part, ml_part);              \
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;                                 \
  }
    MX_FDEC(1, 128) MX_FDEC(2, 128) MX_FDEC(4, 128) MX_FDEC(8, 128)
    MX_FDEC(1, 256) MX_FDEC(2, 256) MX_FDEC(4, 256) MX_FDEC(8, 256)
#undef MX_FDEC
    return MX_EUNSUPPORTED;
  }
  const int chunks = (d.max_ctx + kAttnChunk - 1) / kAttnChunk;
  if (chunks > max_chunks) return MX_EINVAL;
  // two q heads per workgroup (one when the kv head has one)
  const int grp = d.heads / d.kv_heads;
  if (grp != 1 && grp != 2 && grp != 4 && grp != 8 && grp != 16) return MX_EUNSUPPORTED;
  const int splits = grp == 1 ? 1 : grp / 2;
  const int groups = chunks * d.kv_heads * rows;
  const dim3 grid((groups + 7) / 8 * 8 * splits);
#define MX_DEC(GG, DD)                                                                          \
  if ((grp == 1 ? 1 : 2) == GG && d.head_dim == 64 * DD) {                                      \
    hipLaunchKernelGGL((decode_kernel<GG, DD>), grid, dim3(kAttnChunk), 0, s, q, slots, pos,    \
                       k_cache, v_cache, d, max_chunks, scale, o_part, ml_part, chunks, rows);  \
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;                                   \
  }
  MX_DEC(1, 1) MX_DEC(1, 2) MX_DEC(1, 4) MX_DEC(2, 1) MX_DEC(2, 2) MX_DEC(2, 4)
#undef MX_DEC
  return MX_EUNSUPPORTED;  // head_dim other than 64, 128 or 256
}

int attn_combine(const float* o_part, const float* ml_part, const uint16_t* qkv,
                 int64_t qkv_stride, int rows, const int32_t* pos, AttnDims d, int max_chunks,
                 bool fast, uint16_t* out, hipStream_t s, char* plane) {
  if (fast) {
    if ((d.max_ctx + kAttnFastChunk - 1) / kAttnFastChunk > 256) return MX_EUNSUPPORTED;
    hipLaunchKernelGGL(combine_fast_kernel, dim3(d.heads, rows), dim3(256), 0, s, o_part,
                       ml_part, qkv, qkv_stride, pos, d, max_chunks, kAttnFastChunk, out);
  } else {
    const bool pl = plane && rows <= 8 && d.head_dim % xq::kGroup == 0;
    hipLaunchKernelGGL(combine_kernel, dim3(d.heads, rows), dim3(kMaxHd), 0, s, o_part, ml_part,
                       qkv, qkv_stride, pos, d, max_chunks, kAttnChunk, out,
                       pl ? plane : nullptr);
  }
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

bool attn_prefill_supported(AttnDims d) {
  if (!attn_fast_supported(d)) return false;
  const int g = d.heads / d.kv_heads;
  return (d.head_dim == 256 || d.head_dim == 128) && (g == 2 || g == 4 || g == 8) &&
         (d.max_ctx + kPfSplit - 1) / kPfSplit <= 256;
}

int attn_prefill(const uint16_t* q, int rows, const int32_t* slots, const int32_t* pos,
                 const uint16_t* k_cache, const uint16_t* v_cache, AttnDims d, int max_chunks,
                 float* o_part, float* ml_part, hipStream_t s) {
  if (!attn_prefill_supported(d)) return MX_EUNSUPPORTED;
  const int splits = (d.max_ctx + kPfSplit - 1) / kPfSplit;
  if (splits > max_chunks) return MX_EINVAL;
  const float scale = 1.0f / __builtin_sqrtf(float(d.head_dim));
  const int g = d.heads / d.kv_heads;
#define MX_PF(GG, HH)                                                                        \
  if (g == GG && d.head_dim == HH) {                                                         \
    const auto fn = prefill_attn_kernel<GG, HH>;                                             \
    constexpr int lb = prefill_attn_lds<HH>();                                               \
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(fn),                               \
                            hipFuncAttributeMaxDynamicSharedMemorySize, lb) != hipSuccess)   \
      return MX_EHIP;                                                                        \
    constexpr int qb = 8 * 16 / GG;                                                          \
    hipLaunchKernelGGL(fn, dim3(splits, d.kv_heads, (rows + qb - 1) / qb), dim3(512), lb, s, \
                       q, rows, slots, pos, k_cache, v_cache, d, max_chunks, scale, o_part,  \
                       ml_part);                                                             \
    return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;                                \
  }
  MX_PF(2, 128) MX_PF(4, 128) MX_PF(8, 128) MX_PF(2, 256) MX_PF(4, 256) MX_PF(8, 256)
#undef MX_PF
  return MX_EUNSUPPORTED;
}

int attn_combine_splits(const float* o_part, const float* ml_part, const uint16_t* qkv,
                        int64_t qkv_stride, int rows, const int32_t* pos, AttnDims d,
                        int max_chunks, uint16_t* out, hipStream_t s) {
  if ((d.max_ctx + kPfSplit - 1) / kPfSplit > 256) return MX_EUNSUPPORTED;
  hipLaunchKernelGGL(combine_fast_kernel, dim3(d.heads, rows), dim3(256), 0, s, o_part, ml_part,
                     qkv, qkv_stride, pos, d, max_chunks, kPfSplit, out);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
