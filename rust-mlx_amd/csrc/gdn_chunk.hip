// Chunked GatedDeltaNet prefill scan (gfx950 matrix cores).
//
// Reference: the delta-rule recurrence of gdn_kernel::recurrent
// (src/gdn_kernel.rs:7-71, kernels/gated_delta.metal), per value head:
//   S_t = g_t S_{t-1} + k_t d_t^T,  d_t = beta_t (v_t - g_t S_{t-1}^T k_t),
//   y_t = bf16(S_t^T q_t)
// with S fp32 [dk][dv] (dk-major, as the decode kernels keep it).
//
// Chunked form over chunks of C = 64 tokens (gamma_t = prod_{r<=t} g_r within
// the chunk, S_0 the state entering it):
//   S_t = gamma_t S_0 + sum_{s<=t} (gamma_t / gamma_s) k_s d_s^T
//   (I + A) D = beta V - (beta gamma K) S_0,  A[t][s] = beta_t (gamma_t/gamma_s) k_t.k_s (s < t)
//   so D = U - W S_0 with T = (I + A)^-1, U = T (beta V), W = T (beta gamma K);
//   O = (gamma Q) S_0 + P D,  P[t][s] = (gamma_t/gamma_s) q_t.k_s (s <= t);
//   S_C = gamma_C S_0 + K'^T D,  K'_s = (gamma_C/gamma_s) k_s.
// Every product that touches the fp32 state is an fp32 matrix-core product
// (v_mfma_f32_16x16x4_f32), so the state agrees with the sequential fp32
// recurrence to rounding; the Gram matrices K K^T and Q K^T of bf16 inputs
// are exact products with fp32 sums on the bf16 matrix cores.  Decay ratios
// come from an fp64 prefix sum of log2 g (no underflow of the ratios; g = 0
// is clamped to 2^-200, i.e. a full reset).
//
//  chunk_prep_kernel (chunks x heads x groups, parallel): the per-chunk
//    quantities above, written to a workspace in matrix-core operand order.
//  chunk_scan_kernel (16-column state slices x heads x groups): walks the
//    chunks in order, carrying its 128 x 16 slice of the state in LDS.
#include "common.hpp"
#include "kernels.hpp"
#include "skinny_core.hpp"

namespace mx {

namespace {

constexpr int kC = 64;   // tokens per chunk
constexpr int kD = 128;  // head dim (dk == dv)
constexpr int kSlice = 16;
constexpr int kLd = kC + 1;  // padded LDS row

// Workspace of one (group, head, chunk), in floats.
constexpr int kWOff = 0;                // W  A-operand order [4 tiles][64 lanes][32]
constexpr int kQOff = kWOff + kC * kD;  // gamma Q, same order
constexpr int kKOff = kQOff + kC * kD;  // K'^T A-operand order [8 tiles][64 lanes][16]
constexpr int kPOff = kKOff + kC * kD;  // P A-operand order [4 tiles][64 lanes][16]
constexpr int kUOff = kPOff + kC * kC;  // U [64][128]
constexpr int kGOff = kUOff + kC * kD;  // gamma_C
constexpr int kWsFloats = kGOff + 16;

typedef float floatx4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4_t mfma4(float a, float b, floatx4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// acc += X Y for 16 x 16 blocks in LDS (row-major, leading dims ldx / ldy):
// lane l supplies X[l%16][4kk + l/16] and Y[4kk + l/16][l%16].
__device__ __forceinline__ floatx4_t mm16(const float* X, int ldx, const float* Y, int ldy,
                                          floatx4_t acc) {
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) acc = mfma4(X[j * ldx + 4 * kk + q], Y[(4 * kk + q) * ldy + j], acc);
  return acc;
}

// Stores a 16 x 16 D block (lane: rows 4q + r, column j) scaled by `scale`.
__device__ __forceinline__ void store16(float* Z, int ldz, floatx4_t v, float scale) {
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) Z[(4 * q + r) * ldz + j] = v[r] * scale;
}

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void chunk_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ g,
    const uint16_t* __restrict__ beta, int hk, int hv, int t, int nchunks, int64_t v_stride,
    float* __restrict__ ws) {
  __shared__ double Ls[kC];            // inclusive prefix sum of log2 g
  __shared__ float bs[kC];             // beta
  __shared__ float Am[kC * kLd];       // K K^T, then A
  __shared__ float QKm[kC * kLd];      // Q K^T
  __shared__ float Tm[kC * kLd];       // T = (I + A)^-1
  __shared__ float tmp[3][16 * 17];    // level products of the blocked inverse
  __shared__ uint16_t Ks[kC * kD];     // K chunk (bf16)
  __shared__ uint16_t Vs[kC * kD];     // V chunk (bf16)
  const int c = blockIdx.x, h = blockIdx.y, grp = blockIdx.z;
  const int kh = h / (hv / hk);
  const int t0 = c * kC;
  const int len = min(kC, t - t0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 15, qd = lane >> 4;
  const size_t row0 = size_t(grp) * t + t0;
  float* out = ws + ((size_t(grp) * hv + h) * nchunks + c) * kWsFloats;

  // K, V chunk into LDS (rows past len are zero); 16-byte units
  for (int u = tid; u < kC * kD / 8; u += 256) {
    const int r = u / (kD / 8), cu = u - r * (kD / 8);
    const bool ok = r < len;
    const size_t rr = row0 + (ok ? r : 0);
    uint4 kv = *reinterpret_cast<const uint4*>(k + (rr * hk + kh) * kD + cu * 8);
    uint4 vv = *reinterpret_cast<const uint4*>(v + rr * v_stride + h * kD + cu * 8);
    if (!ok) kv = vv = make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(Ks + r * kD + cu * 8) = kv;
    *reinterpret_cast<uint4*>(Vs + r * kD + cu * 8) = vv;
  }
  // log2 g prefix (fp64, wave 0) and beta
  if (tid < kC) {
    const bool ok = tid < len;
    const float gv = ok ? g[(row0 + tid) * hv + h] : 1.0f;
    const float bv = ok ? bf16_to_f32(beta[(row0 + tid) * hv + h]) : 0.0f;
    double l = double(gv > 0x1p-126f ? __builtin_amdgcn_logf(gv) : -200.0f);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const double n = __shfl_up(l, o, 64);
      if (lane >= o) l += n;
    }
    Ls[tid] = l;
    bs[tid] = bv;
  }
  // Gram matrices on the bf16 matrix cores (exact products, fp32 sums):
  // wave w computes row tile w of K K^T and of Q K^T
  {
    const int rt = wave;
    const int ra = min(t0 + 16 * rt + j, t - 1) - t0;  // clamped token of this lane's A row
    const bool rok = 16 * rt + j < len;
    sk::floatx4_t gk[4], gq[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) gk[ct] = gq[ct] = sk::floatx4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < kD / 32; ++kk) {
      const int d0 = 32 * kk + 8 * qd;
      uint4 ak = *reinterpret_cast<const uint4*>(k + ((row0 + ra) * hk + kh) * kD + d0);
      uint4 aq = *reinterpret_cast<const uint4*>(q + ((row0 + ra) * hk + kh) * kD + d0);
      if (!rok) ak = aq = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int cb = min(t0 + 16 * ct + j, t - 1) - t0;
        uint4 bk = *reinterpret_cast<const uint4*>(k + ((row0 + cb) * hk + kh) * kD + d0);
        if (16 * ct + j >= len) bk = make_uint4(0u, 0u, 0u, 0u);
        gk[ct] = sk::mfma(ak, bk, gk[ct]);
        gq[ct] = sk::mfma(aq, bk, gq[ct]);
      }
    }
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        Am[(16 * rt + 4 * qd + r) * kLd + 16 * ct + j] = gk[ct][r];
        QKm[(16 * rt + 4 * qd + r) * kLd + 16 * ct + j] = gq[ct][r];
      }
  }
  __syncthreads();
  // A (strictly lower) and P (lower incl. diagonal) with the decay ratios
  for (int e = tid; e < kC * kC; e += 256) {
    const int tr = e >> 6, sc = e & 63;
    const float ratio = sc <= tr ? __builtin_amdgcn_exp2f(float(Ls[tr] - Ls[sc])) : 0.0f;
    Am[tr * kLd + sc] = sc < tr ? bs[tr] * ratio * Am[tr * kLd + sc] : 0.0f;
    QKm[tr * kLd + sc] = ratio * QKm[tr * kLd + sc];
  }
  __syncthreads();
  // T = (I + A)^-1, blocked 4 x 4 over 16 x 16 blocks.
  // Diagonal blocks: wave w, lane j < 16 owns column j of block w.
  if (j == lane) {  // lanes 0..15 of every wave
    const int b0 = 16 * wave;
    float col[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float acc = r == j ? 1.0f : 0.0f;
#pragma unroll
      for (int p = 0; p < r; ++p) acc = fmaf_(-Am[(b0 + r) * kLd + b0 + p], col[p], acc);
      col[r] = acc;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) Tm[(b0 + r) * kLd + b0 + j] = col[r];
  }
  // zero the strictly upper blocks
  for (int e = tid; e < kC * kC; e += 256) {
    const int tr = e >> 6, sc = e & 63;
    if ((sc >> 4) > (tr >> 4)) Tm[tr * kLd + sc] = 0.0f;
  }
  __syncthreads();
  // off-diagonal blocks by distance: T_ij = -T_ii sum_{m=j}^{i-1} A_im T_mj
  for (int dist = 1; dist < 4; ++dist) {
    const int bi = wave + dist, bj = wave;  // waves 0 .. 3 - dist
    const bool act = bi < 4;
    if (act) {
      floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int m = bj; m < bi; ++m)
        acc = mm16(Am + (16 * bi) * kLd + 16 * m, kLd, Tm + (16 * m) * kLd + 16 * bj, kLd, acc);
      store16(tmp[wave], 17, acc, 1.0f);
    }
    __syncthreads();
    if (act) {
      floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      acc = mm16(Tm + (16 * bi) * kLd + 16 * bi, kLd, tmp[wave], 17, acc);
      store16(Tm + (16 * bi) * kLd + 16 * bj, kLd, acc, -1.0f);
    }
    __syncthreads();
  }
  // W = T (beta gamma K), U = T (beta V): 4 row tiles x 8 column tiles each;
  // wave w takes row tile w.  B values formed on the fly from LDS.
  {
    const int rt = wave;
    float* wop = out + kWOff;
    float* uo = out + kUOff;
    for (int ct = 0; ct < kD / 16; ++ct) {
      floatx4_t aw = {0.0f, 0.0f, 0.0f, 0.0f}, au = aw;
#pragma unroll 4
      for (int kk = 0; kk < kC / 4; ++kk) {
        const int s = 4 * kk + qd;
        const float a = Tm[(16 * rt + j) * kLd + s];
        const float bsc = bs[s];
        const float gs = __builtin_amdgcn_exp2f(float(Ls[s]));
        aw = mfma4(a, bsc * gs * bf16_to_f32(Ks[s * kD + 16 * ct + j]), aw);
        au = mfma4(a, bsc * bf16_to_f32(Vs[s * kD + 16 * ct + j]), au);
      }
      // W in A-operand order: tile rt, lane (row j', k-slot q'), index kk'
      // element W[16 rt + rr][d] with d = 16 ct + j -> kk' = d / 4, q' = d % 4
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rr = 4 * qd + r, d = 16 * ct + j;
        const int l2 = (d & 3) * 16 + rr;
        wop[(rt * 64 + l2) * 32 + (d >> 2)] = aw[r];
        uo[(16 * rt + rr) * kD + d] = au[r];
      }
    }
  }
  // gamma Q (A-operand order like W), K'^T (A operand rows d, k = s), P
  {
    const double lc = Ls[kC - 1];
    float* qop = out + kQOff;
    float* kop = out + kKOff;
    float* pop = out + kPOff;
    for (int e = tid; e < kC * kD; e += 256) {
      const int tr = e >> 7, d = e & 127;
      const bool ok = tr < len;
      const size_t rr = row0 + (ok ? tr : 0);
      const float qv = ok ? bf16_to_f32(q[(rr * hk + kh) * kD + d]) : 0.0f;
      const float gt = __builtin_amdgcn_exp2f(float(Ls[tr]));
      // gamma Q: tile tr / 16, lane (d % 4) * 16 + tr % 16, index d / 4
      qop[((tr >> 4) * 64 + (d & 3) * 16 + (tr & 15)) * 32 + (d >> 2)] = gt * qv;
      // K'^T [d][s = tr]: tile d / 16, lane (s % 4) * 16 + d % 16, index s / 4
      const float kv = bf16_to_f32(Ks[tr * kD + d]) * __builtin_amdgcn_exp2f(float(lc - Ls[tr]));
      kop[((d >> 4) * 64 + (tr & 3) * 16 + (d & 15)) * 16 + (tr >> 2)] = kv;
    }
    for (int e = tid; e < kC * kC; e += 256) {
      const int tr = e >> 6, sc = e & 63;
      pop[((tr >> 4) * 64 + (sc & 3) * 16 + (tr & 15)) * 16 + (sc >> 2)] = QKm[tr * kLd + sc];
    }
    if (tid == 0) out[kGOff] = __builtin_amdgcn_exp2f(float(lc));
  }
}

// ---------------------------------------------------------------------------
// One 16-column slice of one head's state, chunk after chunk.  Wave w owns
// output row tile w (tokens 16 w ..) and state row tiles 2 w, 2 w + 1.
__global__ __launch_bounds__(256) void chunk_scan_kernel(const float* __restrict__ ws, int hv,
                                                         int t, int nchunks,
                                                         const int32_t* __restrict__ slots,
                                                         float* __restrict__ state,
                                                         uint16_t* __restrict__ y) {
  __shared__ float Sl[kD * 17];  // state slice [d][16]
  __shared__ float Dl[kC * 17];  // D of the chunk [s][16]
  const int slice = blockIdx.x, h = blockIdx.y, grp = blockIdx.z;
  const int i0 = slice * kSlice;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 15, qd = lane >> 4;
  float* sp = state + (size_t(slots[grp]) * hv + h) * kD * kD + i0;
  for (int e = tid; e < kD * kSlice; e += 256) {
    const int d = e >> 4, i = e & 15;
    Sl[d * 17 + i] = sp[size_t(d) * kD + i];
  }
  __syncthreads();
  // a chunk's workspace operands of this lane; the next chunk's are
  // requested before this chunk's work (they do not depend on the state)
  struct ChunkOps {
    float4 w[8], q[8], p[4], k[2][4];
    float u[4];
    float gc;
  };
  auto load_ops = [&](int c, ChunkOps& o) {
    const float* in = ws + ((size_t(grp) * hv + h) * nchunks + c) * kWsFloats;
    const float4* wrow = reinterpret_cast<const float4*>(in + kWOff + (wave * 64 + lane) * 32);
    const float4* qrow = reinterpret_cast<const float4*>(in + kQOff + (wave * 64 + lane) * 32);
#pragma unroll
    for (int k4 = 0; k4 < 8; ++k4) {
      o.w[k4] = wrow[k4];
      o.q[k4] = qrow[k4];
    }
    const float4* prow = reinterpret_cast<const float4*>(in + kPOff + (wave * 64 + lane) * 16);
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) o.p[k4] = k4 <= wave ? prow[k4] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float4* krow =
          reinterpret_cast<const float4*>(in + kKOff + ((2 * wave + u) * 64 + lane) * 16);
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) o.k[u][k4] = krow[k4];
    }
    const float* uo = in + kUOff;
#pragma unroll
    for (int r = 0; r < 4; ++r) o.u[r] = uo[(16 * wave + 4 * qd + r) * kD + i0 + j];
    o.gc = in[kGOff];
  };
  ChunkOps cur, nxt;
  load_ops(0, cur);
  for (int c = 0; c < nchunks; ++c) {
    if (c + 1 < nchunks) load_ops(c + 1, nxt);  // in flight during this chunk
    const int t0 = c * kC;
    const int len = min(kC, t - t0);
    // D = U - W S and the first part of O = (gamma Q) S, row tile `wave`
    floatx4_t dacc = {0.0f, 0.0f, 0.0f, 0.0f}, oacc = dacc;
#pragma unroll
    for (int k4 = 0; k4 < 8; ++k4) {
      const float4 wv = cur.w[k4], qv = cur.q[k4];
      const float wa[4] = {wv.x, wv.y, wv.z, wv.w}, qa[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int kk = 4 * k4 + e;
        const float sb = Sl[(4 * kk + qd) * 17 + j];
        dacc = mfma4(wa[e], sb, dacc);
        oacc = mfma4(qa[e], sb, oacc);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tr = 16 * wave + 4 * qd + r;
      Dl[tr * 17 + j] = cur.u[r] - dacc[r];
    }
    const float gc = cur.gc;
    __syncthreads();
    // O += P D (P lower triangular: k-steps up to the tile's diagonal)
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      if (k4 > wave) break;  // uniform per wave
      const float4 pv = cur.p[k4];
      const float pa[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int kk = 4 * k4 + e;
        oacc = mfma4(pa[e], Dl[(4 * kk + qd) * 17 + j], oacc);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tr = 16 * wave + 4 * qd + r;
      if (tr < len)
        y[((size_t(grp) * t + t0 + tr) * hv + h) * kD + i0 + j] = f32_to_bf16(oacc[r]);
    }
    // S_new = gamma_C S + K'^T D for state row tiles 2 wave, 2 wave + 1
    floatx4_t sacc[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int dt = 2 * wave + u;
      floatx4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) {
        const float4 kv = cur.k[u][k4];
        const float ka[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int kk = 4 * k4 + e;
          acc = mfma4(ka[e], Dl[(4 * kk + qd) * 17 + j], acc);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = fmaf_(gc, Sl[(16 * dt + 4 * qd + r) * 17 + j], acc[r]);
      sacc[u] = acc;
    }
    __syncthreads();  // every read of Sl and Dl for this chunk is done
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int dt = 2 * wave + u;
#pragma unroll
      for (int r = 0; r < 4; ++r) Sl[(16 * dt + 4 * qd + r) * 17 + j] = sacc[u][r];
    }
    __syncthreads();
    cur = nxt;
  }
  for (int e = tid; e < kD * kSlice; e += 256) {
    const int d = e >> 4, i = e & 15;
    sp[size_t(d) * kD + i] = Sl[d * 17 + i];
  }
}

}  // namespace

size_t gdn_chunk_workspace_bytes(int groups, int hv, int t) {
  const size_t nchunks = (size_t(t) + kC - 1) / kC;
  return size_t(groups) * hv * nchunks * kWsFloats * sizeof(float);
}

int gdn_prefill_chunked(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                        const uint16_t* beta, GdnDims d, int groups, int t, const int32_t* slots,
                        float* state, uint16_t* y, float* workspace, hipStream_t s,
                        int64_t v_stride) {
  if (d.dk != kD || d.dv != kD || d.hk <= 0 || d.hv % d.hk != 0) return MX_EUNSUPPORTED;
  if (groups <= 0 || t <= 0) return MX_OK;
  const int nchunks = (t + kC - 1) / kC;
  if (v_stride <= 0) v_stride = int64_t(d.hv) * kD;
  hipLaunchKernelGGL(chunk_prep_kernel, dim3(nchunks, d.hv, groups), dim3(256), 0, s, q, k, v, g,
                     beta, d.hk, d.hv, t, nchunks, v_stride, workspace);
  hipLaunchKernelGGL(chunk_scan_kernel, dim3(kD / kSlice, d.hv, groups), dim3(256), 0, s,
                     workspace, d.hv, t, nchunks, slots, state, y);
  return hipGetLastError() == hipSuccess ? MX_OK : MX_EHIP;
}

}  // namespace mx
