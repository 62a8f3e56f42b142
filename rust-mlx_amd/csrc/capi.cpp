// C ABI: argument validation, error reporting and dispatch to the launchers.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "kernels.hpp"

namespace mx {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_error(hipError_t e, const char* what) {
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return e == hipErrorOutOfMemory ? MX_ENOMEM : MX_EHIP;
}

const char* last_error() { return g_last_error.c_str(); }

const char* check_qweight(const QWeight& w) {
  if (!w.codes || !w.scales || !w.biases) return "null weight pointer";
  if (w.bits != 4 && w.bits != 5 && w.bits != 6 && w.bits != 8) return "bits must be 4, 5, 6 or 8";
  if (w.group_size != 32 && w.group_size != 64 && w.group_size != 128)
    return "group_size must be 32, 64 or 128";
  if (w.n <= 0 || w.k <= 0) return "n and k must be positive";
  if (w.k % 32 != 0 || w.k % w.group_size != 0) return "k must be a multiple of 32 and group_size";
  if (int64_t(w.n) * w.k * w.bits / 8 > (int64_t(1) << 40)) return "weight too large";
  return nullptr;
}

// Converts a launcher's return code into the ABI status, filling in the
// message for HIP launch failures.
mx_status finish(int rc, const char* what) {
  if (rc == MX_EHIP) {
    const hipError_t e = hipGetLastError();
    return mx_status(hip_error(e, what));
  }
  if (rc != MX_OK)
    set_error(rc, std::string(what) + (rc == MX_EUNSUPPORTED ? ": unsupported geometry" : ": failed"));
  return mx_status(rc);
}

}  // namespace mx

using namespace mx;

#define MX_ABI extern "C" __attribute__((visibility("default")))

MX_ABI const char* mx_last_error(void) { return last_error(); }
MX_ABI int32_t mx_abi_version(void) { return 1; }

MX_ABI mx_status mx_malloc(void** ptr, size_t bytes) {
  MX_CHECK(ptr != nullptr, MX_EINVAL, "mx_malloc: null out pointer");
  *ptr = nullptr;
  if (bytes == 0) return MX_OK;
  MX_HIP(hipMalloc(ptr, bytes));
  return MX_OK;
}
MX_ABI mx_status mx_free(void* ptr) {
  if (ptr) MX_HIP(hipFree(ptr));
  return MX_OK;
}
MX_ABI mx_status mx_memcpy_htod(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return MX_OK;
  MX_CHECK(dst && src, MX_EINVAL, "mx_memcpy_htod: null pointer");
  MX_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return MX_OK;
}
MX_ABI mx_status mx_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return MX_OK;
  MX_CHECK(dst && src, MX_EINVAL, "mx_memcpy_dtoh: null pointer");
  MX_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return MX_OK;
}
MX_ABI mx_status mx_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return MX_OK;
  MX_CHECK(dst && src, MX_EINVAL, "mx_memcpy_dtod: null pointer");
  MX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, hipStream_t(stream)));
  return MX_OK;
}
MX_ABI mx_status mx_memset(void* dst, int value, size_t bytes, void* stream) {
  if (bytes == 0) return MX_OK;
  MX_CHECK(dst != nullptr, MX_EINVAL, "mx_memset: null pointer");
  MX_HIP(hipMemsetAsync(dst, value, bytes, hipStream_t(stream)));
  return MX_OK;
}
MX_ABI mx_status mx_stream_create(void** stream) {
  MX_CHECK(stream != nullptr, MX_EINVAL, "mx_stream_create: null out pointer");
  hipStream_t s = nullptr;
  MX_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return MX_OK;
}
MX_ABI mx_status mx_stream_destroy(void* stream) {
  if (stream) MX_HIP(hipStreamDestroy(hipStream_t(stream)));
  return MX_OK;
}
MX_ABI mx_status mx_stream_sync(void* stream) {
  MX_HIP(hipStreamSynchronize(hipStream_t(stream)));
  return MX_OK;
}
MX_ABI mx_status mx_device_sync(void) {
  MX_HIP(hipDeviceSynchronize());
  return MX_OK;
}
MX_ABI mx_status mx_event_create(void** event) {
  MX_CHECK(event != nullptr, MX_EINVAL, "mx_event_create: null out pointer");
  hipEvent_t e = nullptr;
  MX_HIP(hipEventCreate(&e));
  *event = e;
  return MX_OK;
}
MX_ABI mx_status mx_event_destroy(void* event) {
  if (event) MX_HIP(hipEventDestroy(hipEvent_t(event)));
  return MX_OK;
}
MX_ABI mx_status mx_event_record(void* event, void* stream) {
  MX_CHECK(event != nullptr, MX_EINVAL, "mx_event_record: null event");
  MX_HIP(hipEventRecord(hipEvent_t(event), hipStream_t(stream)));
  return MX_OK;
}
MX_ABI mx_status mx_event_elapsed_ms(void* start, void* stop, float* ms) {
  MX_CHECK(start && stop && ms, MX_EINVAL, "mx_event_elapsed_ms: null argument");
  MX_HIP(hipEventSynchronize(hipEvent_t(stop)));
  MX_HIP(hipEventElapsedTime(ms, hipEvent_t(start), hipEvent_t(stop)));
  return MX_OK;
}

MX_ABI mx_status mx_fill_bf16(uint16_t* dst, size_t count, uint64_t seed, int32_t dist, float a,
                              float b, void* stream) {
  MX_CHECK(dst != nullptr || count == 0, MX_EINVAL, "mx_fill_bf16: null pointer");
  MX_CHECK(dist == 0 || dist == 1, MX_EINVAL, "mx_fill_bf16: dist must be 0 or 1");
  return finish(fill_bf16(dst, count, seed, dist, a, b, hipStream_t(stream)), "mx_fill_bf16");
}

MX_ABI mx_status mx_fill_codes(uint32_t* dst, int64_t rows, int32_t k, int32_t bits, uint64_t seed,
                               void* stream) {
  MX_CHECK(dst != nullptr, MX_EINVAL, "mx_fill_codes: null pointer");
  MX_CHECK(bits == 4 || bits == 5 || bits == 6 || bits == 8, MX_EINVAL,
           "mx_fill_codes: bits must be 4, 5, 6 or 8");
  MX_CHECK(rows >= 0 && k > 0 && k % 32 == 0, MX_EINVAL,
           "mx_fill_codes: k must be a positive multiple of 32");
  return finish(fill_codes(dst, rows, k, bits, seed, hipStream_t(stream)), "mx_fill_codes");
}

MX_ABI mx_status mx_eval_math(int32_t op, const float* in, float* out, int64_t n, void* stream) {
  MX_CHECK(op >= 0 && op <= 4, MX_EINVAL, "mx_eval_math: op must be 0..4");
  MX_CHECK((in && out) || n == 0, MX_EINVAL, "mx_eval_math: null pointer");
  return finish(eval_math(op, in, out, n, hipStream_t(stream)), "mx_eval_math");
}

MX_ABI mx_status mx_qmv(const mx_qweight* w, const uint16_t* x, int32_t m, uint16_t* y,
                        void* stream) {
  MX_CHECK(w != nullptr && x != nullptr && y != nullptr, MX_EINVAL, "mx_qmv: null pointer");
  const QWeight q = to_qweight(*w);
  if (const char* err = check_qweight(q)) return mx_status(set_error(MX_EINVAL, std::string("mx_qmv: ") + err));
  MX_CHECK(m >= 1 && m <= 8, MX_EUNSUPPORTED, "mx_qmv: m must be in 1..8");
  return finish(qmv(q, x, m, y, hipStream_t(stream)), "mx_qmv");
}

MX_ABI mx_status mx_dequant_rows(const mx_qweight* w, const uint32_t* ids, int32_t count,
                                 uint16_t* out, void* stream) {
  MX_CHECK(w != nullptr, MX_EINVAL, "mx_dequant_rows: null weight");
  MX_CHECK(count >= 0, MX_EINVAL, "mx_dequant_rows: negative count");
  if (count == 0) return MX_OK;
  MX_CHECK(ids && out, MX_EINVAL, "mx_dequant_rows: null pointer");
  const QWeight q = to_qweight(*w);
  if (const char* err = check_qweight(q))
    return mx_status(set_error(MX_EINVAL, std::string("mx_dequant_rows: ") + err));
  MX_CHECK(count <= 65535, MX_EUNSUPPORTED, "mx_dequant_rows: count must be <= 65535");
  return finish(dequant_rows(q, ids, count, out, hipStream_t(stream)), "mx_dequant_rows");
}
