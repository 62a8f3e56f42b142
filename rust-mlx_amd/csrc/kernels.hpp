// Internal launcher declarations shared by the C ABI and the engine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mx355.h"

namespace mx {

struct QWeight {
  const uint32_t* codes;
  const uint16_t* scales;
  const uint16_t* biases;
  int n, k, bits, group_size;
};

inline QWeight to_qweight(const mx_qweight& w) {
  return QWeight{w.codes, w.scales, w.biases, w.n, w.k, w.bits, w.group_size};
}

// Shape rules shared by every quantised projection; returns an error message
// or nullptr.
const char* check_qweight(const QWeight& w);

int qmv(const QWeight& w, const uint16_t* x, int m, uint16_t* y, hipStream_t s);
int dequant_rows(const QWeight& w, const uint32_t* ids, int count, uint16_t* out, hipStream_t s);

int fill_bf16(uint16_t* dst, size_t count, uint64_t seed, int dist, float a, float b,
              hipStream_t s);
int fill_codes(uint32_t* dst, int64_t rows, int k, int bits, uint64_t seed, hipStream_t s);
int eval_math(int op, const float* in, float* out, int64_t n, hipStream_t s);

}  // namespace mx
