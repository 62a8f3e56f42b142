// Routing tail of one activation row in one wave (gfx950): softmax (fp32, MLX
// precise exp) -> bf16 gates -> top-k under the (bf16 gate, expert index) key
// -> bf16 renormalisation.  Lane l owns experts PER*l .. PER*l + PER - 1.
//
// Reference: moe_route::tail (src/moe_route.rs:25-70,
// kernels/moe_route_tail.{h,metal}).  Used by the standalone routing kernel
// and by the persistent expert gate/up kernel, which routes its rows itself.
#pragma once

#include "common.hpp"

namespace mx {
namespace rt {

template <int CTRL>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xF, 0xF, false));
}

// DPP with a row mask: rows outside ROWS keep v.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_rows(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(int(v), int(v), CTRL, ROWS, 0xF, false));
}

// Wave-wide maxima in VALU (no LDS round trip): within rows by quad and
// mirror permutes, across rows by row_bcast:15 and row_bcast:31, then one read
// of lane 63; a maximum is the same in any order.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp<0xB1>(v));             // quad_perm [1,0,3,2]
  v = max(v, dpp<0x4E>(v));             // quad_perm [2,3,0,1]
  v = max(v, dpp<0x141>(v));            // row_half_mirror
  v = max(v, dpp<0x140>(v));            // row_mirror: every lane of a row holds its max
  v = max(v, dpp_rows<0x142, 0xA>(v));  // row_bcast:15 into rows 1, 3
  v = max(v, dpp_rows<0x143, 0xC>(v));  // row_bcast:31 into rows 2, 3
  return uint32_t(__builtin_amdgcn_readlane(int(v), 63));
}

// Largest of the lanes' values under `b > a ? b : a` (any order gives the
// same value when none is NaN).
__device__ __forceinline__ float wave_max_f32(float x) {
  auto mx2 = [](float a, float b) { return b > a ? b : a; };
  x = mx2(x, __uint_as_float(dpp<0xB1>(__float_as_uint(x))));
  x = mx2(x, __uint_as_float(dpp<0x4E>(__float_as_uint(x))));
  x = mx2(x, __uint_as_float(dpp<0x141>(__float_as_uint(x))));
  x = mx2(x, __uint_as_float(dpp<0x140>(__float_as_uint(x))));
  x = mx2(x, __uint_as_float(dpp_rows<0x142, 0xA>(__float_as_uint(x))));
  x = mx2(x, __uint_as_float(dpp_rows<0x143, 0xC>(__float_as_uint(x))));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

// The xor-butterfly wave sum (levels 32, 16, 8, 4, 2, 1; each lane adds its
// partner's value) with the butterfly's own tree, in VALU: levels 32 and 16
// by lane swaps, 8 by row_ror:8 (= xor 8 within a row), 4 by row_ror:4 (after
// level 8, lanes l and l ^ 8 hold equal values, so lane (l + 4) mod 16 holds
// what lane l ^ 4 holds), 2 and 1 by quad permutes.  Addition is commutative,
// so every lane gets the bits of the shuffle form.
__device__ __forceinline__ float wave_sum_xor(float s) {
  {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false,
                                                    false);
    s = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(s), __float_as_uint(s), false,
                                                    false);
    s = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  s = s + __uint_as_float(dpp<0x128>(__float_as_uint(s)));  // row_ror:8
  s = s + __uint_as_float(dpp<0x124>(__float_as_uint(s)));  // row_ror:4
  s = s + __uint_as_float(dpp<0x4E>(__float_as_uint(s)));   // quad_perm [2,3,0,1]
  s = s + __uint_as_float(dpp<0xB1>(__float_as_uint(s)));   // quad_perm [1,0,3,2]
  return s;
}

struct RouteLane {
  uint32_t id;     // lanes < top_k: the expert of slot `lane`
  uint16_t score;  // lanes < top_k: its renormalised bf16 score
};

// logits: the row's PER * 64 expert logits (bf16).  Slots are ascending: slot
// top_k - 1 holds the largest gate.
template <int PER>
__device__ __forceinline__ RouteLane route_row(const uint16_t* __restrict__ logits, int top_k) {
  const int lane = threadIdx.x & 63;
  const uint16_t* in = logits + lane * PER;
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) v[i] = bf16_to_f32(in[i]);
  float mx_ = v[0];
#pragma unroll
  for (int i = 1; i < PER; ++i) mx_ = v[i] > mx_ ? v[i] : mx_;
  mx_ = wave_max_f32(mx_);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    v[i] = expf_(v[i] - mx_);
    sum = sum + v[i];
  }
  // the softmax total: xor butterfly (its order fixes the bits)
  sum = wave_sum_xor(sum);
  const float inv = 1.0f / sum;
  uint32_t key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint32_t g = f32_to_bf16(v[i] * inv);
    // order-preserving map of the bf16 pattern (moe_route_tail.h:13-16)
    const uint32_t k16 = (g & 0x8000u) ? (~g & 0xffffu) : (g | 0x8000u);
    key[i] = (k16 << 16) | uint32_t(lane * PER + i);
  }
  // round s picks the s-th largest key; slot top_k - 1 - s is kept by the
  // lane of that number
  uint32_t mine_key = 0;
  for (int s = 0; s < top_k; ++s) {
    uint32_t best = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) best = key[i] > best ? key[i] : best;
    best = wave_max_u32(best);
    if (lane == top_k - 1 - s) mine_key = best;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (key[i] == best) key[i] = 0u;  // keys are unique; real keys are never 0
  }
  const uint32_t k16 = mine_key >> 16;
  const uint32_t g = (k16 & 0x8000u) ? (k16 & 0x7fffu) : (~k16 & 0xffffu);
  const float mine = bf16_to_f32(uint16_t(g));
  // the renormalising total: one bf16 add per slot, ascending, read lane by
  // lane (the same value in every lane)
  float total = 0.0f;
  for (int j = 0; j < top_k; ++j)
    total = round_bf16(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), j)) + total);
  return RouteLane{mine_key & 0xffffu, f32_to_bf16(mine / total)};
}

}  // namespace rt
}  // namespace mx
