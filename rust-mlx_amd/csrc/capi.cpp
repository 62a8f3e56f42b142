// C ABI: argument validation, error reporting and dispatch to the launchers.
#include <hip/hip_runtime.h>

#include <cstring>
#include <new>
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
MX_ABI int32_t mx_prefill_chunk_tokens(void) { return kPrefillChunk; }

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

// ---- MoE ------------------------------------------------------------------
namespace {
const char* check_bank(const QBank& b) {
  if (b.experts <= 0) return "bank needs at least one expert";
  const QWeight w{b.codes, b.scales, b.biases, b.n, b.k, b.bits, b.group_size};
  return check_qweight(w);
}
}  // namespace

MX_ABI mx_status mx_moe_route(const uint16_t* logits, int64_t logit_stride,
                              const uint16_t* shared_logit, int64_t shared_stride, int32_t rows,
                              int32_t experts, int32_t top_k, uint32_t* ids, uint16_t* scores,
                              uint16_t* factor, void* stream) {
  MX_CHECK(rows >= 0, MX_EINVAL, "mx_moe_route: negative rows");
  if (rows == 0) return MX_OK;
  MX_CHECK(logits && shared_logit && ids && scores && factor, MX_EINVAL,
           "mx_moe_route: null pointer");
  MX_CHECK(experts % 64 == 0 && (experts / 64 == 1 || experts / 64 == 2 || experts / 64 == 4 ||
                                 experts / 64 == 8 || experts / 64 == 16),
           MX_EUNSUPPORTED, "mx_moe_route: experts must be 64, 128, 256, 512 or 1024");
  MX_CHECK(top_k >= 1 && top_k <= 16, MX_EUNSUPPORTED, "mx_moe_route: top_k must be in 1..16");
  MX_CHECK(logit_stride >= experts && shared_stride >= 1, MX_EINVAL,
           "mx_moe_route: row strides too small");
  return finish(moe_route(logits, logit_stride, shared_logit, shared_stride, rows, experts, top_k,
                          ids, scores, factor, hipStream_t(stream)),
                "mx_moe_route");
}

MX_ABI size_t mx_moe_workspace_bytes(int32_t rows, int32_t top_k, int32_t inter) {
  if (rows <= 0 || top_k <= 0 || inter <= 0) return 0;
  return moe_workspace_bytes(rows, top_k, inter);
}

MX_ABI mx_status mx_moe_experts(const uint16_t* x, const uint32_t* ids, const uint16_t* scores,
                                int32_t rows, int32_t top_k, const mx_qbank* gate,
                                const mx_qbank* up, const mx_qbank* down,
                                const mx_qweight* shared_gate, const mx_qweight* shared_up,
                                const mx_qweight* shared_down, void* workspace, uint16_t* partial,
                                void* stream) {
  MX_CHECK(x && ids && scores && gate && up && down && shared_gate && shared_up && shared_down &&
               workspace && partial,
           MX_EINVAL, "mx_moe_experts: null pointer");
  MX_CHECK(rows >= 1 && rows <= 8, MX_EUNSUPPORTED, "mx_moe_experts: rows must be in 1..8");
  MX_CHECK(top_k >= 1 && top_k <= 16, MX_EUNSUPPORTED, "mx_moe_experts: top_k must be in 1..16");
  const QBank g = to_qbank(*gate), u = to_qbank(*up), d = to_qbank(*down);
  const QWeight sg = to_qweight(*shared_gate), su = to_qweight(*shared_up),
                sd = to_qweight(*shared_down);
  for (const QBank* b : {&g, &u, &d})
    if (const char* err = check_bank(*b))
      return mx_status(set_error(MX_EINVAL, std::string("mx_moe_experts: ") + err));
  for (const QWeight* w : {&sg, &su, &sd})
    if (const char* err = check_qweight(*w))
      return mx_status(set_error(MX_EINVAL, std::string("mx_moe_experts: shared ") + err));
  MX_CHECK(g.n == u.n && g.k == u.k && d.k == g.n && d.n == g.k && g.experts == u.experts &&
               g.experts == d.experts && g.bits == u.bits && g.group_size == u.group_size,
           MX_EINVAL, "mx_moe_experts: gate/up/down banks disagree in shape");
  MX_CHECK(sg.n == su.n && sg.k == g.k && su.k == g.k && sd.k == sg.n && sd.n == g.k &&
               sg.bits == su.bits && sg.group_size == su.group_size && sd.bits == d.bits &&
               sd.group_size == d.group_size && sg.bits == g.bits &&
               sg.group_size == g.group_size,
           MX_EINVAL, "mx_moe_experts: shared expert disagrees with the banks");
  return finish(moe_experts(x, ids, scores, rows, top_k, g, u, d, sg, su, sd, workspace, partial,
                            hipStream_t(stream)),
                "mx_moe_experts");
}

MX_ABI mx_status mx_moe_reduce(const uint16_t* partial, int32_t rows, int32_t top_k,
                               int32_t hidden, uint16_t* routed, void* stream) {
  MX_CHECK(rows >= 0 && hidden > 0 && top_k >= 1, MX_EINVAL, "mx_moe_reduce: bad shape");
  if (rows == 0) return MX_OK;
  MX_CHECK(partial && routed, MX_EINVAL, "mx_moe_reduce: null pointer");
  return finish(moe_reduce(partial, rows, top_k, hidden, routed, hipStream_t(stream)),
                "mx_moe_reduce");
}

MX_ABI mx_status mx_moe_hc_epilogue(const uint16_t* routed, const uint16_t* shared,
                                    const uint16_t* factor, const uint16_t* residual,
                                    const uint16_t* gate, int32_t rows, int32_t hc,
                                    int32_t hidden, uint16_t* out, void* stream) {
  MX_CHECK(rows >= 0 && hc >= 1 && hidden > 0, MX_EINVAL, "mx_moe_hc_epilogue: bad shape");
  if (rows == 0) return MX_OK;
  MX_CHECK(routed && shared && factor && residual && gate && out, MX_EINVAL,
           "mx_moe_hc_epilogue: null pointer");
  return finish(moe_hc_epilogue(routed, shared, factor, residual, gate, rows, hc, hidden, out,
                                hipStream_t(stream)),
                "mx_moe_hc_epilogue");
}

MX_ABI mx_status mx_moe_reduce_hc_epilogue(const uint16_t* partial, const uint16_t* factor,
                                           const uint16_t* residual, const uint16_t* gate,
                                           int32_t rows, int32_t top_k, int32_t hc,
                                           int32_t hidden, uint16_t* out, void* stream) {
  MX_CHECK(rows >= 0 && hc >= 1 && hidden > 0 && top_k >= 1, MX_EINVAL,
           "mx_moe_reduce_hc_epilogue: bad shape");
  if (rows == 0) return MX_OK;
  MX_CHECK(partial && factor && residual && gate && out, MX_EINVAL,
           "mx_moe_reduce_hc_epilogue: null pointer");
  return finish(moe_reduce_hc_epilogue(partial, factor, residual, gate, rows, top_k, hc, hidden,
                                       out, hipStream_t(stream)),
                "mx_moe_reduce_hc_epilogue");
}

// ---- greedy head ----------------------------------------------------------
MX_ABI size_t mx_head_workspace_bytes(int32_t n, int32_t k, int32_t m) {
  if (n <= 0 || k <= 0 || m <= 0) return 0;
  return size_t(head_parts(n, k)) * m * (sizeof(float) + sizeof(uint32_t));
}

MX_ABI mx_status mx_head_argmax(const mx_qweight* w, const uint16_t* x, int32_t m,
                                uint32_t* tokens, void* workspace, void* stream) {
  MX_CHECK(w && x && tokens && workspace, MX_EINVAL, "mx_head_argmax: null pointer");
  const QWeight q = to_qweight(*w);
  if (const char* err = check_qweight(q))
    return mx_status(set_error(MX_EINVAL, std::string("mx_head_argmax: ") + err));
  MX_CHECK(m >= 1 && m <= 8, MX_EUNSUPPORTED, "mx_head_argmax: m must be in 1..8");
  const int parts = head_parts(q.n, q.k);
  float* maxima = static_cast<float*>(workspace);
  uint32_t* indices = reinterpret_cast<uint32_t*>(maxima + size_t(parts) * m);
  int got = 0;
  int rc = head_partials(q, x, m, maxima, indices, &got, hipStream_t(stream));
  if (rc != MX_OK) return finish(rc, "mx_head_argmax");
  return finish(argmax_reduce(maxima, indices, m, parts, tokens, hipStream_t(stream)),
                "mx_head_argmax");
}

MX_ABI size_t mx_head_noalloc_max_bytes(void) { return kHeadNoAllocScratchBytes; }

MX_ABI mx_status mx_head_argmax_noalloc(const mx_qweight* w, const uint16_t* x, int32_t m,
                                        uint32_t* tokens, void* stream) {
  MX_CHECK(w && x && tokens, MX_EINVAL, "mx_head_argmax_noalloc: null pointer");
  const QWeight q = to_qweight(*w);
  if (const char* err = check_qweight(q))
    return mx_status(set_error(MX_EINVAL, std::string("mx_head_argmax_noalloc: ") + err));
  MX_CHECK(m >= 1 && m <= 8, MX_EUNSUPPORTED, "mx_head_argmax_noalloc: m must be in 1..8");
  MX_CHECK(head_noalloc_bytes(q.n, q.k, m) <= kHeadNoAllocScratchBytes, MX_EUNSUPPORTED,
           "mx_head_argmax_noalloc: the partials of this head (mx_head_workspace_bytes) exceed "
           "the static scratch (mx_head_noalloc_max_bytes)");
  return finish(head_argmax_noalloc(q, x, m, tokens, hipStream_t(stream)),
                "mx_head_argmax_noalloc");
}

MX_ABI mx_status mx_head_argmax_mfma(const mx_qweight* w, const uint16_t* x, int32_t m,
                                     uint32_t* tokens, void* workspace, void* stream) {
  MX_CHECK(w && x && tokens && workspace, MX_EINVAL, "mx_head_argmax_mfma: null pointer");
  const QWeight q = to_qweight(*w);
  if (const char* err = check_qweight(q))
    return mx_status(set_error(MX_EINVAL, std::string("mx_head_argmax_mfma: ") + err));
  MX_CHECK(m >= 1 && m <= 8, MX_EUNSUPPORTED, "mx_head_argmax_mfma: m must be in 1..8");
  MX_CHECK(skinny_supported(q) && q.k % 512 == 0 && q.k <= 2048, MX_EUNSUPPORTED,
           "mx_head_argmax_mfma: needs group_size 64, k % 512 == 0 and k <= 2048");
  const int parts = skinny_head_parts(q.n);
  float* maxima = static_cast<float*>(workspace);
  uint32_t* indices = reinterpret_cast<uint32_t*>(maxima + size_t(parts) * m);
  int got = 0;
  int rc = skinny_head(q, x, m, maxima, indices, &got, hipStream_t(stream));
  if (rc != MX_OK) return finish(rc, "mx_head_argmax_mfma");
  return finish(argmax_reduce(maxima, indices, m, parts, tokens, hipStream_t(stream)),
                "mx_head_argmax_mfma");
}

MX_ABI mx_status mx_argmax_bf16(const uint16_t* logits, int32_t rows, int32_t n, uint32_t* tokens,
                                void* stream) {
  MX_CHECK(rows >= 0 && n > 0, MX_EINVAL, "mx_argmax_bf16: bad shape");
  if (rows == 0) return MX_OK;
  MX_CHECK(logits && tokens, MX_EINVAL, "mx_argmax_bf16: null pointer");
  return finish(argmax_bf16(logits, rows, n, tokens, hipStream_t(stream)), "mx_argmax_bf16");
}

// ---- GatedDeltaNet --------------------------------------------------------
MX_ABI mx_status mx_gdn_conv(const uint16_t* qkv, int64_t row_stride, int32_t groups, int32_t t,
                             const int32_t* slots, uint16_t* conv_state, const float* conv_w,
                             int32_t channels, int32_t conv_k, uint16_t* out, int64_t out_stride,
                             uint16_t* window_history, void* stream) {
  MX_CHECK(groups >= 0 && t >= 1 && channels > 0, MX_EINVAL, "mx_gdn_conv: bad shape");
  if (groups == 0) return MX_OK;
  MX_CHECK(qkv && slots && conv_state && conv_w && out, MX_EINVAL, "mx_gdn_conv: null pointer");
  MX_CHECK(conv_k >= 2 && conv_k <= 8, MX_EUNSUPPORTED, "mx_gdn_conv: conv_k must be in 2..8");
  MX_CHECK(row_stride >= channels && out_stride >= channels, MX_EINVAL,
           "mx_gdn_conv: row strides too small");
  return finish(gdn_conv(qkv, row_stride, groups, t, slots, conv_state, conv_w, channels, conv_k,
                         out, out_stride, window_history, hipStream_t(stream)),
                "mx_gdn_conv");
}

MX_ABI mx_status mx_gdn_recurrence(const uint16_t* conv_out, int64_t conv_stride,
                                   const uint16_t* z, const uint16_t* a, const uint16_t* b,
                                   int64_t zab_stride, const float* a_log,
                                   const uint16_t* dt_bias, const uint16_t* norm_w, float eps,
                                   const mx_gdn_dims* dims, int32_t groups, int32_t t,
                                   const int32_t* slots, float* state, float* history,
                                   uint16_t* y, void* stream) {
  MX_CHECK(dims != nullptr, MX_EINVAL, "mx_gdn_recurrence: null dims");
  MX_CHECK(groups >= 0 && t >= 1, MX_EINVAL, "mx_gdn_recurrence: bad shape");
  if (groups == 0) return MX_OK;
  MX_CHECK(conv_out && z && a && b && a_log && dt_bias && norm_w && slots && state && y,
           MX_EINVAL, "mx_gdn_recurrence: null pointer");
  const GdnDims d{dims->hk, dims->hv, dims->dk, dims->dv, dims->conv_k};
  MX_CHECK(d.hk > 0 && d.hv > 0 && d.hv % d.hk == 0, MX_EINVAL,
           "mx_gdn_recurrence: value heads must be a multiple of key heads");
  MX_CHECK(d.dk == 128 && d.dv == 128, MX_EUNSUPPORTED,
           "mx_gdn_recurrence: head dims must be 128");
  MX_CHECK(conv_stride >= int64_t(2) * d.hk * d.dk + int64_t(d.hv) * d.dv, MX_EINVAL,
           "mx_gdn_recurrence: conv row stride too small");
  return finish(gdn_recurrence(conv_out, conv_stride, z, a, b, zab_stride, a_log, dt_bias, norm_w,
                               eps, d, groups, t, slots, state, history, y, hipStream_t(stream)),
                "mx_gdn_recurrence");
}

MX_ABI mx_status mx_gdn_recurrence_fast(const uint16_t* conv_out, int64_t conv_stride,
                                        const uint16_t* z, const uint16_t* a, const uint16_t* b,
                                        int64_t zab_stride, const float* a_log,
                                        const uint16_t* dt_bias, const uint16_t* norm_w,
                                        float eps, const mx_gdn_dims* dims, int32_t groups,
                                        int32_t t, const int32_t* slots, float* state,
                                        float* history, uint16_t* y, void* stream) {
  MX_CHECK(dims != nullptr, MX_EINVAL, "mx_gdn_recurrence_fast: null dims");
  MX_CHECK(groups >= 0 && t >= 1, MX_EINVAL, "mx_gdn_recurrence_fast: bad shape");
  if (groups == 0) return MX_OK;
  MX_CHECK(conv_out && z && a && b && a_log && dt_bias && norm_w && slots && state && y,
           MX_EINVAL, "mx_gdn_recurrence_fast: null pointer");
  const GdnDims d{dims->hk, dims->hv, dims->dk, dims->dv, dims->conv_k};
  MX_CHECK(d.hk > 0 && d.hv > 0 && d.hv % d.hk == 0, MX_EINVAL,
           "mx_gdn_recurrence_fast: value heads must be a multiple of key heads");
  MX_CHECK(d.dk == 128 && d.dv == 128, MX_EUNSUPPORTED,
           "mx_gdn_recurrence_fast: head dims must be 128");
  MX_CHECK(conv_stride >= int64_t(2) * d.hk * d.dk + int64_t(d.hv) * d.dv, MX_EINVAL,
           "mx_gdn_recurrence_fast: conv row stride too small");
  return finish(gdn_recurrence_fast(conv_out, conv_stride, z, a, b, zab_stride, a_log, dt_bias,
                                    norm_w, eps, d, groups, t, slots, state, history, y,
                                    hipStream_t(stream)),
                "mx_gdn_recurrence_fast");
}

MX_ABI mx_status mx_gdn_scan(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             const float* g, const uint16_t* beta, const mx_gdn_dims* dims,
                             int32_t groups, int32_t t, const int32_t* slots, float* state,
                             float* history, uint16_t* y, void* stream) {
  MX_CHECK(dims != nullptr, MX_EINVAL, "mx_gdn_scan: null dims");
  MX_CHECK(groups >= 0 && t >= 1, MX_EINVAL, "mx_gdn_scan: bad shape");
  if (groups == 0) return MX_OK;
  MX_CHECK(q && k && v && g && beta && slots && state && y, MX_EINVAL,
           "mx_gdn_scan: null pointer");
  const GdnDims d{dims->hk, dims->hv, dims->dk, dims->dv, dims->conv_k};
  MX_CHECK(d.hk > 0 && d.hv > 0 && d.hv % d.hk == 0, MX_EINVAL,
           "mx_gdn_scan: value heads must be a multiple of key heads");
  MX_CHECK(d.dk == 128 && d.dv == 128, MX_EUNSUPPORTED, "mx_gdn_scan: head dims must be 128");
  return finish(gdn_scan(q, k, v, g, beta, d, groups, t, slots, state, history, y,
                         hipStream_t(stream)),
                "mx_gdn_scan");
}

MX_ABI size_t mx_gdn_prefill_workspace_bytes(int32_t groups, int32_t hv, int32_t t) {
  if (groups <= 0 || hv <= 0 || t <= 0) return 0;
  return gdn_chunk_workspace_bytes(groups, hv, t);
}

MX_ABI mx_status mx_gdn_prefill_chunked(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                        const float* g, const uint16_t* beta,
                                        const mx_gdn_dims* dims, int32_t groups, int32_t t,
                                        const int32_t* slots, float* state, uint16_t* y,
                                        void* workspace, void* stream) {
  MX_CHECK(dims != nullptr, MX_EINVAL, "mx_gdn_prefill_chunked: null dims");
  MX_CHECK(groups >= 0 && t >= 1, MX_EINVAL, "mx_gdn_prefill_chunked: bad shape");
  if (groups == 0) return MX_OK;
  MX_CHECK(q && k && v && g && beta && slots && state && y && workspace, MX_EINVAL,
           "mx_gdn_prefill_chunked: null pointer");
  const GdnDims d{dims->hk, dims->hv, dims->dk, dims->dv, dims->conv_k};
  MX_CHECK(d.hk > 0 && d.hv > 0 && d.hv % d.hk == 0, MX_EINVAL,
           "mx_gdn_prefill_chunked: value heads must be a multiple of key heads");
  MX_CHECK(d.dk == 128 && d.dv == 128, MX_EUNSUPPORTED,
           "mx_gdn_prefill_chunked: head dims must be 128");
  return finish(gdn_prefill_chunked(q, k, v, g, beta, d, groups, t, slots, state, y,
                                    static_cast<float*>(workspace), hipStream_t(stream)),
                "mx_gdn_prefill_chunked");
}

MX_ABI mx_status mx_gemv_bf16(const uint16_t* w, int32_t n, int32_t k, const uint16_t* x,
                              int32_t rows, uint16_t* y, void* stream) {
  MX_CHECK(rows >= 0 && n >= 0 && k >= 0, MX_EINVAL, "mx_gemv_bf16: negative size");
  if (rows == 0 || n == 0) return MX_OK;
  MX_CHECK(w && x && y, MX_EINVAL, "mx_gemv_bf16: null pointer");
  MX_CHECK(rows <= 8 && k >= 128 && k % 128 == 0, MX_EUNSUPPORTED,
           "mx_gemv_bf16: needs 1..8 rows and k a positive multiple of 128");
  return finish(gemv_bf16(w, n, k, x, rows, y, hipStream_t(stream)), "mx_gemv_bf16");
}

// ---- attention --------------------------------------------------------------
MX_ABI size_t mx_attn_workspace_bytes(int32_t rows, int32_t heads, int32_t head_dim,
                                      int32_t max_ctx) {
  if (rows <= 0 || heads <= 0 || head_dim <= 0 || max_ctx <= 0) return 0;
  const size_t chunks = (size_t(max_ctx) + kAttnFastChunk - 1) / kAttnFastChunk;
  const size_t o = size_t(rows) * heads * chunks * head_dim * 4;
  return o + size_t(rows) * heads * chunks * 2 * 4;
}

MX_ABI mx_status mx_attn_decode(const uint16_t* q, const uint16_t* qkv, int64_t qkv_stride,
                                int32_t rows, const int32_t* slots, const int32_t* pos,
                                const uint16_t* k_cache, const uint16_t* v_cache,
                                const mx_attn_dims* dims, int32_t flags, void* workspace,
                                uint16_t* out, void* stream) {
  MX_CHECK(dims != nullptr, MX_EINVAL, "mx_attn_decode: null dims");
  MX_CHECK(rows >= 0, MX_EINVAL, "mx_attn_decode: negative rows");
  if (rows == 0) return MX_OK;
  MX_CHECK(q && qkv && slots && pos && k_cache && v_cache && workspace && out, MX_EINVAL,
           "mx_attn_decode: null pointer");
  const AttnDims d{dims->heads, dims->kv_heads, dims->head_dim, 0, dims->max_ctx,
                   dims->slot_stride};
  MX_CHECK(d.heads > 0 && d.kv_heads > 0 && d.heads % d.kv_heads == 0, MX_EINVAL,
           "mx_attn_decode: heads must be a positive multiple of kv_heads");
  MX_CHECK(d.head_dim > 0 && d.head_dim <= 256 && d.head_dim % 8 == 0 && d.max_ctx > 0,
           MX_EUNSUPPORTED, "mx_attn_decode: head_dim must be a multiple of 8 up to 256");
  MX_CHECK(d.slot_stride >= int64_t(d.kv_heads) * d.max_ctx * d.head_dim &&
               d.slot_stride % 8 == 0 && qkv_stride >= int64_t(2) * d.heads * d.head_dim,
           MX_EINVAL, "mx_attn_decode: bad strides");
  const bool fast = (flags & 1) != 0;
  MX_CHECK(!fast || attn_fast_supported(d), MX_EUNSUPPORTED,
           "mx_attn_decode: matrix-core kernel needs head_dim 128/256 and 1..8 q heads per kv head");
  const int chunks = (d.max_ctx + kAttnFastChunk - 1) / kAttnFastChunk;
  float* o_part = static_cast<float*>(workspace);
  float* ml_part = o_part + size_t(rows) * d.heads * chunks * d.head_dim;
  const hipStream_t s = hipStream_t(stream);
  if (flags & 2) {  // the prefill form: rows of one slot, query blocks sharing key tiles
    MX_CHECK(attn_prefill_supported(d), MX_EUNSUPPORTED,
             "mx_attn_decode: prefill form needs head_dim 128/256 and 2, 4 or 8 q heads per kv head");
    int rc = attn_prefill(q, rows, slots, pos, k_cache, v_cache, d, chunks, o_part, ml_part, s);
    if (rc == MX_OK)
      rc = attn_combine_splits(o_part, ml_part, qkv, qkv_stride, rows, pos, d, chunks, out, s);
    return finish(rc, "mx_attn_decode");
  }
  int rc = attn_decode(q, rows, slots, pos, k_cache, v_cache, d, chunks, fast, o_part, ml_part, s);
  if (rc == MX_OK)
    rc = attn_combine(o_part, ml_part, qkv, qkv_stride, rows, pos, d, chunks, fast, out, s);
  return finish(rc, "mx_attn_decode");
}

// ---- engine ---------------------------------------------------------------
struct mx_engine {
  mx::Engine* impl;
};

namespace {
const char* check_config(const mx_model_config& c) {
  if (c.hidden <= 0 || c.hidden % 64 != 0) return "hidden must be a positive multiple of 64";
  if (c.layers <= 0 || c.attn_every <= 0) return "layers and attn_every must be positive";
  if (c.vocab <= 0) return "vocab must be positive";
  if (c.hc != 4) return "hc must be 4";
  if (c.hc_rank <= 0 || c.hc_rank % 64 != 0) return "hc_rank must be a positive multiple of 64";
  if (c.gdn_dk != 128 || c.gdn_dv != 128) return "GDN head dims must be 128";
  if (c.gdn_hk <= 0 || c.gdn_hv % c.gdn_hk != 0) return "GDN value heads must be a multiple of key heads";
  if (c.conv_k < 2 || c.conv_k > 8) return "conv_k must be in 2..8";
  if (c.kv_heads <= 0 || c.heads % c.kv_heads != 0) return "heads must be a multiple of kv_heads";
  const int g = c.heads / (c.kv_heads > 0 ? c.kv_heads : 1);
  if (g != 1 && g != 2 && g != 4 && g != 8 && g != 16) return "heads / kv_heads must be 1, 2, 4, 8 or 16";
  if (c.head_dim <= 0 || c.head_dim > 256 || c.head_dim % 64 != 0) return "head_dim must be 64, 128, 192 or 256";
  if (c.rotary_dim <= 0 || c.rotary_dim % 2 != 0 || c.rotary_dim > c.head_dim) return "bad rotary_dim";
  if (c.experts % 64 != 0 || c.experts / 64 > 16 || (c.experts / 64) & (c.experts / 64 - 1))
    return "experts must be 64, 128, 256, 512 or 1024";
  if (c.top_k < 1 || c.top_k > 16) return "top_k must be in 1..16";
  if (c.moe_inter <= 0 || c.shared_inter <= 0 || c.moe_inter % 64 || c.shared_inter % 64)
    return "expert intermediate sizes must be positive multiples of 64";
  if (c.group_size != 64)
    return "group_size must be 64 (the engine's exact-integer kernels combine 64-value groups)";
  if (c.layers > MX_MAX_LAYERS) return "layers must be at most MX_MAX_LAYERS";
  for (int b : {c.bits, c.down_bits, c.embed_bits, c.head_bits})
    if (b != 4 && b != 5 && b != 6 && b != 8) return "bits must be 4, 5, 6 or 8";
  for (int b : c.layer_widths)
    if (b != 0 && b != 4 && b != 5 && b != 6 && b != 8) return "layer_widths entries must be 0, 4, 5, 6 or 8";
  if (c.max_slots < 1 || c.max_slots > 4096) return "max_slots must be in 1..4096";
  if (c.max_context < 1) return "max_context must be positive";
  if (c.max_verify < 1 || c.max_verify > 8) return "max_verify must be in 1..8";
  return nullptr;
}

mx_status engine_status(int rc, const std::string& err, const char* what) {
  if (rc == MX_OK) return MX_OK;
  if (!err.empty()) {
    set_error(rc, std::string(what) + ": " + err);
    return mx_status(rc);
  }
  return finish(rc, what);
}

bool tokens_ok(const mx::Engine& e, const uint32_t* t, int n) {
  for (int i = 0; i < n; ++i)
    if (t[i] >= uint32_t(engine_config(e).vocab)) return false;
  return true;
}
bool slot_ok(const mx::Engine& e, int s) { return s >= 0 && s < engine_config(e).max_slots; }
}  // namespace

MX_ABI mx_status mx_engine_create(const mx_model_config* cfg, mx_engine** out) {
  MX_CHECK(cfg && out, MX_EINVAL, "mx_engine_create: null pointer");
  if (const char* err = check_config(*cfg))
    return mx_status(set_error(MX_EINVAL, std::string("mx_engine_create: ") + err));
  mx::Engine* e = nullptr;
  const int rc = engine_create(*cfg, &e);
  if (rc != MX_OK) return finish(rc, "mx_engine_create");
  *out = new mx_engine{e};
  return MX_OK;
}

MX_ABI mx_status mx_engine_destroy(mx_engine* e) {
  if (e) {
    engine_destroy(e->impl);
    delete e;
  }
  return MX_OK;
}

MX_ABI mx_status mx_engine_reset_slot(mx_engine* e, int32_t slot) {
  MX_CHECK(e && slot_ok(*e->impl, slot), MX_EINVAL, "mx_engine_reset_slot: bad engine or slot");
  return finish(engine_reset_slot(*e->impl, slot), "mx_engine_reset_slot");
}

MX_ABI mx_status mx_engine_clone_slot(mx_engine* e, int32_t src, int32_t dst) {
  MX_CHECK(e && slot_ok(*e->impl, src) && slot_ok(*e->impl, dst) && src != dst, MX_EINVAL,
           "mx_engine_clone_slot: bad engine or slots");
  MX_CHECK(!engine_slot_failed(*e->impl, src), MX_ESTATE,
           "mx_engine_clone_slot: the source slot was left partly updated by a failed step");
  return finish(engine_clone_slot(*e->impl, src, dst), "mx_engine_clone_slot");
}

MX_ABI int32_t mx_engine_offset(mx_engine* e, int32_t slot) {
  if (!e || !slot_ok(*e->impl, slot)) return -1;
  return engine_offset(*e->impl, slot);
}

MX_ABI int32_t mx_engine_slot_failed(mx_engine* e, int32_t slot) {
  if (!e || !slot_ok(*e->impl, slot)) return -1;
  return engine_slot_failed(*e->impl, slot);
}

MX_ABI mx_status mx_engine_inject_failure(mx_engine* e, int32_t after_layers) {
  MX_CHECK(e && after_layers >= 0, MX_EINVAL, "mx_engine_inject_failure: bad arguments");
  engine_inject_failure(*e->impl, after_layers);
  return MX_OK;
}

static mx_status decode_common(mx_engine* e, const int32_t* slots, const uint32_t* tokens,
                               int32_t rows, uint32_t* next, bool equal, const char* what,
                               uint16_t* logits = nullptr, uint16_t* hidden = nullptr) {
  MX_CHECK(e && slots && tokens && next, MX_EINVAL, std::string(what) + ": null pointer");
  MX_CHECK(rows >= 1 && rows <= 8, MX_EUNSUPPORTED, std::string(what) + ": rows must be in 1..8");
  for (int r = 0; r < rows; ++r)
    MX_CHECK(slot_ok(*e->impl, slots[r]), MX_EINVAL, std::string(what) + ": slot out of range");
  MX_CHECK(tokens_ok(*e->impl, tokens, rows), MX_EINVAL,
           std::string(what) + ": token outside vocabulary");
  if (equal)
    for (int r = 1; r < rows; ++r)
      MX_CHECK(engine_offset(*e->impl, slots[r]) == engine_offset(*e->impl, slots[0]), MX_ESTATE,
               std::string(what) + ": rows must share one cache offset");
  std::string err;
  const int rc = (logits || hidden)
                     ? engine_decode_outputs(*e->impl, slots, tokens, rows, next, logits, hidden, &err)
                     : engine_decode_rows(*e->impl, slots, tokens, rows, next, &err);
  return engine_status(rc, err, what);
}

MX_ABI mx_status mx_engine_decode_batch_outputs(mx_engine* e, const int32_t* slots,
                                                const uint32_t* tokens, int32_t rows,
                                                uint32_t* next, uint16_t* logits,
                                                uint16_t* hidden) {
  return decode_common(e, slots, tokens, rows, next, true, "mx_engine_decode_batch_outputs",
                       logits, hidden);
}

MX_ABI mx_status mx_engine_decode_forced(mx_engine* e, const int32_t* slots,
                                         const uint32_t* tokens, int32_t rows,
                                         const uint16_t* h_in, uint16_t* h_out,
                                         uint32_t* ids_out, uint32_t* next) {
  MX_CHECK(e && slots && tokens && h_in && h_out && ids_out && next, MX_EINVAL,
           "mx_engine_decode_forced: null pointer");
  MX_CHECK(rows >= 1 && rows <= 8, MX_EUNSUPPORTED, "mx_engine_decode_forced: rows must be in 1..8");
  for (int r = 0; r < rows; ++r)
    MX_CHECK(slot_ok(*e->impl, slots[r]), MX_EINVAL, "mx_engine_decode_forced: slot out of range");
  MX_CHECK(tokens_ok(*e->impl, tokens, rows), MX_EINVAL,
           "mx_engine_decode_forced: token outside vocabulary");
  std::string err;
  const int rc = engine_decode_forced(*e->impl, slots, tokens, rows, h_in, h_out, ids_out, next, &err);
  return engine_status(rc, err, "mx_engine_decode_forced");
}

MX_ABI mx_status mx_engine_decode_batch(mx_engine* e, const int32_t* slots, const uint32_t* tokens,
                                        int32_t rows, uint32_t* next) {
  return decode_common(e, slots, tokens, rows, next, true, "mx_engine_decode_batch");
}

MX_ABI mx_status mx_engine_decode_rows(mx_engine* e, const int32_t* slots, const uint32_t* tokens,
                                       int32_t rows, uint32_t* next) {
  return decode_common(e, slots, tokens, rows, next, false, "mx_engine_decode_rows");
}

MX_ABI mx_status mx_engine_prefill(mx_engine* e, int32_t slot, const uint32_t* tokens,
                                   int32_t count, uint32_t* next) {
  MX_CHECK(e && tokens && next, MX_EINVAL, "mx_engine_prefill: null pointer");
  MX_CHECK(slot_ok(*e->impl, slot), MX_EINVAL, "mx_engine_prefill: slot out of range");
  MX_CHECK(count >= 1, MX_EINVAL, "mx_engine_prefill: empty input");
  MX_CHECK(tokens_ok(*e->impl, tokens, count), MX_EINVAL,
           "mx_engine_prefill: token outside vocabulary");
  uint32_t out[8];
  for (int i = 0; i < count; i += 8) {
    const int n = count - i < 8 ? count - i : 8;
    std::string err;
    const int rc = engine_block(*e->impl, slot, tokens + i, n, false, out, &err);
    if (rc != MX_OK) return engine_status(rc, err, "mx_engine_prefill");
    *next = out[n - 1];
  }
  return MX_OK;
}

MX_ABI mx_status mx_engine_prefill_chunked(mx_engine* e, int32_t slot, const uint32_t* tokens,
                                           int32_t count, uint32_t* next) {
  MX_CHECK(e && tokens && next, MX_EINVAL, "mx_engine_prefill_chunked: null pointer");
  MX_CHECK(slot_ok(*e->impl, slot), MX_EINVAL, "mx_engine_prefill_chunked: slot out of range");
  MX_CHECK(count >= 1, MX_EINVAL, "mx_engine_prefill_chunked: empty input");
  MX_CHECK(tokens_ok(*e->impl, tokens, count), MX_EINVAL,
           "mx_engine_prefill_chunked: token outside vocabulary");
  std::string err;
  return engine_status(engine_prefill_chunked(*e->impl, slot, tokens, count, next, &err), err,
                       "mx_engine_prefill_chunked");
}

MX_ABI mx_status mx_engine_verify(mx_engine* e, int32_t slot, const uint32_t* tokens,
                                  int32_t count, uint32_t* argmax) {
  MX_CHECK(e && tokens && argmax, MX_EINVAL, "mx_engine_verify: null pointer");
  MX_CHECK(slot_ok(*e->impl, slot), MX_EINVAL, "mx_engine_verify: slot out of range");
  MX_CHECK(count >= 1 && count <= engine_config(*e->impl).max_verify, MX_EUNSUPPORTED,
           "mx_engine_verify: count must be in 1..max_verify");
  MX_CHECK(tokens_ok(*e->impl, tokens, count), MX_EINVAL,
           "mx_engine_verify: token outside vocabulary");
  std::string err;
  return engine_status(engine_verify(*e->impl, slot, tokens, count, argmax, &err), err,
                       "mx_engine_verify");
}

MX_ABI mx_status mx_engine_generate(mx_engine* e, int32_t slot, const uint32_t* prompt,
                                    int32_t n_prompt, int32_t max_tokens, int32_t depth,
                                    uint32_t* tokens, int32_t* n_tokens,
                                    mx_generate_stats* stats, uint32_t* drafts) {
  MX_CHECK(e && prompt && tokens && n_tokens, MX_EINVAL, "mx_engine_generate: null pointer");
  MX_CHECK(slot_ok(*e->impl, slot), MX_EINVAL, "mx_engine_generate: slot out of range");
  for (int32_t i = 0; i < n_prompt; ++i)
    MX_CHECK(prompt[i] < uint32_t(engine_config(*e->impl).vocab), MX_EINVAL,
             "mx_engine_generate: token outside vocabulary");
  std::string err;
  int n = 0;
  const int rc = engine_generate(*e->impl, slot, prompt, n_prompt, max_tokens, depth, tokens, &n,
                                 stats, drafts, &err);
  *n_tokens = n;
  return engine_status(rc, err, "mx_engine_generate");
}

MX_ABI mx_status mx_engine_commit(mx_engine* e, int32_t slot, int32_t keep) {
  MX_CHECK(e && slot_ok(*e->impl, slot), MX_EINVAL, "mx_engine_commit: bad engine or slot");
  std::string err;
  return engine_status(engine_commit(*e->impl, slot, keep, &err), err, "mx_engine_commit");
}

MX_ABI mx_status mx_engine_set_flags(mx_engine* e, int32_t flags) {
  MX_CHECK(e != nullptr, MX_EINVAL, "mx_engine_set_flags: null engine");
  engine_set_flags(*e->impl, flags & 1, (flags & 2) ? 0 : 1, (flags & 4) ? 1 : 0,
                   (flags >> 3) & 127, (flags >> 10) & 1);
  return MX_OK;
}

MX_ABI mx_status mx_engine_read(mx_engine* e, const char* what, void* host, size_t bytes) {
  MX_CHECK(e && what && host, MX_EINVAL, "mx_engine_read: null pointer");
  std::string err;
  return engine_status(engine_read(*e->impl, what, host, bytes, &err), err, "mx_engine_read");
}

MX_ABI mx_status mx_engine_tensor(mx_engine* e, const char* name, void** device_ptr,
                                  size_t* bytes) {
  MX_CHECK(e && name && device_ptr && bytes, MX_EINVAL, "mx_engine_tensor: null pointer");
  MX_CHECK(engine_tensor(*e->impl, name, device_ptr, bytes) == MX_OK, MX_EINVAL,
           std::string("mx_engine_tensor: unknown tensor ") + name);
  return MX_OK;
}

MX_ABI mx_status mx_engine_load_tensor(mx_engine* e, const char* name, int32_t dtype,
                                       const int64_t* shape, int32_t ndim, const void* data,
                                       size_t bytes) {
  MX_CHECK(e && name && shape && data, MX_EINVAL, "mx_engine_load_tensor: null pointer");
  MX_CHECK(dtype >= MX_DT_U32 && dtype <= MX_DT_F32, MX_EINVAL, "mx_engine_load_tensor: bad dtype");
  std::string err;
  try {
    return engine_status(engine_load_tensor(*e->impl, name, dtype, shape, ndim, data, bytes, &err),
                         err, "mx_engine_load_tensor");
  } catch (const std::bad_alloc&) {
    return mx_status(set_error(MX_ENOMEM, "mx_engine_load_tensor: out of host memory"));
  } catch (...) {
    return mx_status(set_error(MX_EINVAL, "mx_engine_load_tensor: failed"));
  }
}

MX_ABI mx_status mx_checkpoint_target(const mx_model_config* cfg, const char* name, char* tensor,
                                      size_t cap, int32_t* info) {
  MX_CHECK(cfg && name && tensor && info && cap > 0, MX_EINVAL,
           "mx_checkpoint_target: null pointer");
  CheckpointTarget t;
  const int rc = checkpoint_target(*cfg, name, &t);
  if (rc == MX_EUNSUPPORTED)
    return mx_status(set_error(MX_EUNSUPPORTED, std::string("mx_checkpoint_target: the engine has "
                                                            "no module for tensor ") + name));
  MX_CHECK(rc == MX_OK, MX_EINVAL, std::string("mx_checkpoint_target: unknown tensor name ") + name);
  MX_CHECK(t.tensor.size() < cap, MX_EINVAL, "mx_checkpoint_target: name buffer too small");
  std::memcpy(tensor, t.tensor.c_str(), t.tensor.size() + 1);
  const int32_t v[8] = {int32_t(t.kind), t.part, t.row0, t.rows, t.n, t.k, t.bits,
                        int32_t(t.count)};
  std::memcpy(info, v, sizeof(v));
  return MX_OK;
}

MX_ABI mx_status mx_engine_load_safetensors(mx_engine* e, const char* path, int32_t* loaded) {
  MX_CHECK(e && path && loaded, MX_EINVAL, "mx_engine_load_safetensors: null pointer");
  std::string err;
  int n = 0;
  int rc;
  try {
    rc = engine_load_safetensors(*e->impl, path, &n, &err);
  } catch (const std::bad_alloc&) {
    rc = MX_ENOMEM;
    err = "out of host memory";
  } catch (...) {
    rc = MX_EINVAL;
    err = "failed";
  }
  *loaded = n;
  return engine_status(rc, err, "mx_engine_load_safetensors");
}

MX_ABI mx_status mx_checkpoint_check(const mx_model_config* cfg, const char* path,
                                     int32_t* checked) {
  MX_CHECK(cfg && path && checked, MX_EINVAL, "mx_checkpoint_check: null pointer");
  if (const char* err = check_config(*cfg))
    return mx_status(set_error(MX_EINVAL, std::string("mx_checkpoint_check: ") + err));
  std::string err;
  int n = 0;
  int rc;
  try {
    rc = checkpoint_check(*cfg, path, &n, &err);
  } catch (const std::bad_alloc&) {
    rc = MX_ENOMEM;
    err = "out of host memory";
  } catch (...) {
    rc = MX_EINVAL;
    err = "failed";
  }
  *checked = n;
  return engine_status(rc, err, "mx_checkpoint_check");
}

MX_ABI mx_status mx_engine_time_experts(mx_engine* e, int32_t rows, mx_expert_timing* out) {
  MX_CHECK(e && out, MX_EINVAL, "mx_engine_time_experts: null pointer");
  std::string err;
  return engine_status(engine_time_experts(*e->impl, rows, out, &err), err,
                       "mx_engine_time_experts");
}

MX_ABI mx_status mx_engine_profile_step(mx_engine* e, const int32_t* slots, const uint32_t* tokens,
                                        int32_t rows, uint32_t* next, mx_step_profile* out) {
  MX_CHECK(e && slots && tokens && next && out, MX_EINVAL, "mx_engine_profile_step: null pointer");
  MX_CHECK(rows >= 1 && rows <= 8, MX_EUNSUPPORTED, "mx_engine_profile_step: rows must be in 1..8");
  for (int r = 0; r < rows; ++r)
    MX_CHECK(slot_ok(*e->impl, slots[r]), MX_EINVAL, "mx_engine_profile_step: slot out of range");
  MX_CHECK(tokens_ok(*e->impl, tokens, rows), MX_EINVAL,
           "mx_engine_profile_step: token outside vocabulary");
  std::string err;
  return engine_status(engine_profile_step(*e->impl, slots, tokens, rows, next, out, &err), err,
                       "mx_engine_profile_step");
}

MX_ABI mx_status mx_engine_profile_verify(mx_engine* e, int32_t slot, const uint32_t* tokens,
                                          int32_t count, uint32_t* argmax, mx_step_profile* out) {
  MX_CHECK(e && tokens && argmax && out, MX_EINVAL, "mx_engine_profile_verify: null pointer");
  MX_CHECK(slot_ok(*e->impl, slot), MX_EINVAL, "mx_engine_profile_verify: slot out of range");
  MX_CHECK(count >= 1 && count <= engine_config(*e->impl).max_verify, MX_EUNSUPPORTED,
           "mx_engine_profile_verify: count must be in 1..max_verify");
  MX_CHECK(tokens_ok(*e->impl, tokens, count), MX_EINVAL,
           "mx_engine_profile_verify: token outside vocabulary");
  std::string err;
  return engine_status(engine_profile_verify(*e->impl, slot, tokens, count, argmax, out, &err),
                       err, "mx_engine_profile_verify");
}

MX_ABI mx_status mx_engine_draft_bytes(mx_engine* e, int32_t pos, double* bytes) {
  MX_CHECK(e && bytes, MX_EINVAL, "mx_engine_draft_bytes: null pointer");
  MX_CHECK(pos >= 0, MX_EINVAL, "mx_engine_draft_bytes: negative position");
  std::string err;
  return engine_status(engine_draft_bytes(*e->impl, pos, bytes, &err), err,
                       "mx_engine_draft_bytes");
}

MX_ABI mx_status mx_qmm(const mx_qweight* w, const uint16_t* x, int32_t m, uint16_t* y,
                        void* stream) {
  MX_CHECK(w != nullptr && x != nullptr && y != nullptr, MX_EINVAL, "mx_qmm: null pointer");
  const QWeight q = to_qweight(*w);
  if (const char* err = check_qweight(q)) return mx_status(set_error(MX_EINVAL, std::string("mx_qmm: ") + err));
  MX_CHECK(qmm_supported(q), MX_EUNSUPPORTED, "mx_qmm: needs group_size 64 and k <= 8192");
  MX_CHECK(m >= 1 && m <= kQmmMaxRows, MX_EUNSUPPORTED, "mx_qmm: m must be in 1..512");
  ProjEpilogue e{};
  e.mode = kPlain;
  e.y = y;
  e.y_stride = q.n;
  if (m <= 8 && skinny_supported(q))
    return finish(skinny_dense(q, x, q.k, m, e, hipStream_t(stream)), "mx_qmm");
  return finish(qmm(q, x, q.k, m, e, hipStream_t(stream)), "mx_qmm");
}

MX_ABI mx_status mx_xq(const mx_qweight* w, const uint16_t* x, int32_t m, uint16_t* y,
                       void* stream) {
  MX_CHECK(w != nullptr && x != nullptr && y != nullptr, MX_EINVAL, "mx_xq: null pointer");
  const QWeight q = to_qweight(*w);
  if (const char* err = check_qweight(q)) return mx_status(set_error(MX_EINVAL, std::string("mx_xq: ") + err));
  MX_CHECK(xq_supported(q), MX_EUNSUPPORTED,
           "mx_xq: needs group_size 64 and k a multiple of 64 up to 512 or of 512 up to 8192");
  MX_CHECK(m >= 1 && m <= 8, MX_EUNSUPPORTED, "mx_xq: m must be in 1..8");
  ProjEpilogue e{};
  e.mode = kPlain;
  e.y = y;
  e.y_stride = q.n;
  return finish(xq_dense(q, x, q.k, m, e, hipStream_t(stream)), "mx_xq");
}

MX_ABI mx_status mx_qmm_conv(const mx_qweight* w, const uint16_t* x, int32_t m,
                             int32_t conv_channels, int32_t conv_k, const int32_t* slots,
                             uint16_t* conv_state, const float* conv_w, uint16_t* conv_out,
                             int64_t conv_stride, uint16_t* y, int64_t y_stride, void* stream) {
  MX_CHECK(w && x && slots && conv_state && conv_w && conv_out && y, MX_EINVAL,
           "mx_qmm_conv: null pointer");
  const QWeight q = to_qweight(*w);
  if (const char* err = check_qweight(q))
    return mx_status(set_error(MX_EINVAL, std::string("mx_qmm_conv: ") + err));
  MX_CHECK(m >= 1 && m <= 8, MX_EUNSUPPORTED, "mx_qmm_conv: m must be in 1..8");
  MX_CHECK(q.bits == 4 && skinny_supported(q), MX_EUNSUPPORTED,
           "mx_qmm_conv: needs 4-bit codes, group_size 64 and k a multiple of 512");
  MX_CHECK(conv_k >= 2 && conv_k <= kConvMaxTaps, MX_EUNSUPPORTED,
           "mx_qmm_conv: conv_k must be in 2..4");
  MX_CHECK(conv_channels >= 1 && conv_channels <= q.n && conv_stride >= conv_channels &&
               y_stride >= q.n,
           MX_EINVAL, "mx_qmm_conv: bad channel count or strides");
  ProjEpilogue e{};
  e.mode = kConv;
  e.y = y;
  e.y_stride = y_stride;
  e.conv_state = conv_state;
  e.conv_w = conv_w;
  e.slots = slots;
  e.conv_out = conv_out;
  e.conv_stride = conv_stride;
  e.conv_ch = conv_channels;
  e.taps = conv_k;
  return finish(skinny_dense(q, x, q.k, m, e, hipStream_t(stream)), "mx_qmm_conv");
}

MX_ABI size_t mx_hc_workspace_bytes(int32_t n_down) {
  return n_down > 0 ? hc_fused_part_bytes(n_down) : 0;
}

MX_ABI mx_status mx_hc_forward_mfma(const mx_qweight* down, const mx_qweight* up,
                                    const uint16_t* h, const uint16_t* scale, int32_t rows,
                                    int32_t hc, int32_t hidden, int32_t rank, float eps,
                                    void* workspace, uint16_t* mixed, uint16_t* inj,
                                    void* stream) {
  MX_CHECK(down && up && h && scale && workspace && mixed, MX_EINVAL,
           "mx_hc_forward_mfma: null pointer");
  MX_CHECK(rows >= 1 && rows <= 8, MX_EUNSUPPORTED, "mx_hc_forward_mfma: rows must be in 1..8");
  const QWeight d = to_qweight(*down), u = to_qweight(*up);
  for (const QWeight* q : {&d, &u})
    if (const char* err = check_qweight(*q))
      return mx_status(set_error(MX_EINVAL, std::string("mx_hc_forward_mfma: ") + err));
  MX_CHECK(hc_fused_supported(d, u, hc, hidden, rank), MX_EUNSUPPORTED,
           "mx_hc_forward_mfma: needs hc 4, hidden <= 2048, rank 256 or 512, down rows rank "
           "(+ hc inject rows), group_size 64");
  MX_CHECK(d.n == rank || inj != nullptr, MX_EINVAL, "mx_hc_forward_mfma: inject rows need inj");
  return finish(hc_fused(d, u, h, scale, rows, hc, hidden, rank, eps,
                         static_cast<float*>(workspace), mixed, inj, hipStream_t(stream)),
                "mx_hc_forward_mfma");
}

MX_ABI mx_status mx_moe_experts_mfma(const uint16_t* x, const uint32_t* ids, const uint16_t* scores,
                                     int32_t rows, int32_t top_k, const mx_qbank* gate,
                                     const mx_qbank* up, const mx_qbank* down,
                                     const mx_qweight* shared_gate, const mx_qweight* shared_up,
                                     const mx_qweight* shared_down, void* workspace,
                                     uint16_t* partial, void* stream) {
  MX_CHECK(x && ids && scores && gate && up && down && shared_gate && shared_up && shared_down &&
               workspace && partial,
           MX_EINVAL, "mx_moe_experts_mfma: null pointer");
  MX_CHECK(rows >= 1 && rows <= kPrefillChunk, MX_EUNSUPPORTED,
           "mx_moe_experts_mfma: rows must be in 1..512");
  MX_CHECK(top_k >= 1 && top_k <= 16, MX_EUNSUPPORTED, "mx_moe_experts_mfma: top_k must be in 1..16");
  const QBank g = to_qbank(*gate), u = to_qbank(*up), d = to_qbank(*down);
  const QWeight sg = to_qweight(*shared_gate), su = to_qweight(*shared_up), sd = to_qweight(*shared_down);
  for (const QBank* b : {&g, &u, &d}) {
    if (const char* err = check_bank(*b))
      return mx_status(set_error(MX_EINVAL, std::string("mx_moe_experts_mfma: ") + err));
    MX_CHECK(qmm_supported(QWeight{b->codes, b->scales, b->biases, b->n, b->k, b->bits, b->group_size}),
             MX_EUNSUPPORTED, "mx_moe_experts_mfma: banks need group_size 64");
  }
  MX_CHECK(g.n == u.n && g.k == u.k && d.k == g.n && d.n == g.k && g.experts == u.experts &&
               g.experts == d.experts && g.bits == u.bits && sg.n == su.n && sg.k == g.k &&
               su.k == g.k && sd.k == sg.n && sd.n == g.k && sg.bits == g.bits &&
               sd.bits == d.bits && qmm_supported(sg) && qmm_supported(sd),
           MX_EINVAL, "mx_moe_experts_mfma: banks and shared expert disagree in shape");
  const int inter = g.n > sg.n ? g.n : sg.n;
  uint16_t* h = static_cast<uint16_t*>(workspace);
  const size_t hb = size_t(rows) * (top_k + 1) * inter * sizeof(uint16_t);
  char* list = static_cast<char*>(workspace) + ((hb + 255) / 256) * 256;
  hipStream_t s = hipStream_t(stream);
  if (rows > 8) {  // a prefill chunk's rows: routes grouped by expert, 16-row tiles
    MX_CHECK(g.experts <= kChunkMaxExperts, MX_EUNSUPPORTED,
             "mx_moe_experts_mfma: more than 1023 experts beyond eight rows");
    ChunkPlan* cp = reinterpret_cast<ChunkPlan*>(list);
    int rc = chunk_plan(ids, rows, g.experts, top_k, cp, s);
    if (rc == MX_OK) rc = qmm_chunk_gate_up(x, cp, rows, g.experts, top_k, g, u, sg, su, h, s);
    if (rc == MX_OK)
      rc = qmm_chunk_down(h, cp, scores, rows, g.experts, top_k, g.n, sg.n, d, sd, partial, s);
    return finish(rc, "mx_moe_experts_mfma");
  }
  MoePlan* plan = reinterpret_cast<MoePlan*>(list);
  int rc = skinny_gate_up(x, ids, rows, top_k, g, u, sg, su, h, s);
  if (rc == MX_OK) rc = skinny_down(h, ids, scores, rows, top_k, g.n, sg.n, d, sd, partial, s);
  if (rc != MX_EUNSUPPORTED) return finish(rc, "mx_moe_experts_mfma");
  // depths the skinny kernels do not cover: the 16-row-tile kernels with a plan
  rc = moe_plan(ids, rows, top_k, plan, s);
  if (rc == MX_OK) rc = qmm_gate_up(x, plan, rows, top_k, g, u, sg, su, h, s);
  if (rc == MX_OK) rc = qmm_down(h, plan, scores, rows, top_k, g.n, sg.n, d, sd, partial, s);
  return finish(rc, "mx_moe_experts_mfma");
}

MX_ABI mx_status mx_moe_routed_experts_mfma(
    const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
    int64_t shared_stride, int32_t experts, const uint16_t* x, int32_t rows, int32_t top_k,
    const mx_qbank* gate, const mx_qbank* up, const mx_qbank* down, const mx_qweight* shared_gate,
    const mx_qweight* shared_up, const mx_qweight* shared_down, void* workspace, uint32_t* ids,
    uint16_t* scores, uint16_t* factor, uint16_t* partial, void* stream) {
  MX_CHECK(logits && shared_logit && x && gate && up && down && shared_gate && shared_up &&
               shared_down && workspace && ids && scores && factor && partial,
           MX_EINVAL, "mx_moe_routed_experts_mfma: null pointer");
  MX_CHECK(rows >= 1 && rows <= 8, MX_EUNSUPPORTED,
           "mx_moe_routed_experts_mfma: rows must be in 1..8");
  MX_CHECK(top_k >= 1 && top_k <= 16, MX_EUNSUPPORTED,
           "mx_moe_routed_experts_mfma: top_k must be in 1..16");
  MX_CHECK(experts % 64 == 0 && (experts / 64 == 1 || experts / 64 == 2 || experts / 64 == 4 ||
                                 experts / 64 == 8 || experts / 64 == 16),
           MX_EUNSUPPORTED, "mx_moe_routed_experts_mfma: experts must be 64, 128, 256, 512 or 1024");
  MX_CHECK(logit_stride >= experts && shared_stride >= 1, MX_EINVAL,
           "mx_moe_routed_experts_mfma: row strides too small");
  const QBank g = to_qbank(*gate), u = to_qbank(*up), d = to_qbank(*down);
  const QWeight sg = to_qweight(*shared_gate), su = to_qweight(*shared_up), sd = to_qweight(*shared_down);
  for (const QBank* b : {&g, &u, &d}) {
    if (const char* err = check_bank(*b))
      return mx_status(set_error(MX_EINVAL, std::string("mx_moe_routed_experts_mfma: ") + err));
  }
  MX_CHECK(experts <= g.experts, MX_EINVAL, "mx_moe_routed_experts_mfma: more logits than experts");
  MX_CHECK(g.n == u.n && g.k == u.k && d.k == g.n && d.n == g.k && g.experts == u.experts &&
               g.experts == d.experts && g.bits == u.bits && sg.n == su.n && sg.k == g.k &&
               su.k == g.k && sd.k == sg.n && sd.n == g.k && sg.bits == g.bits && sd.bits == d.bits,
           MX_EINVAL, "mx_moe_routed_experts_mfma: banks and shared expert disagree in shape");
  uint16_t* h = static_cast<uint16_t*>(workspace);
  hipStream_t s = hipStream_t(stream);
  const RouteIO ro{logits, logit_stride, shared_logit, shared_stride, ids, scores, factor};
  int rc = skinny_route_gate_up(ro, experts, x, rows, top_k, g, u, sg, su, h, s);
  if (rc == MX_OK) rc = skinny_down(h, ids, scores, rows, top_k, g.n, sg.n, d, sd, partial, s);
  return finish(rc, "mx_moe_routed_experts_mfma");
}

MX_ABI mx_status mx_moe_routed_experts_hc_mfma(
    const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
    int64_t shared_stride, int32_t experts, const uint16_t* x, int32_t rows, int32_t top_k,
    int32_t hc, const mx_qbank* gate, const mx_qbank* up, const mx_qbank* down,
    const mx_qweight* shared_gate, const mx_qweight* shared_up, const mx_qweight* shared_down,
    void* workspace, uint32_t* ids, uint16_t* scores, uint16_t* factor, const uint16_t* hc_gate,
    uint16_t* hcs, void* stream) {
  MX_CHECK(logits && shared_logit && x && gate && up && down && shared_gate && shared_up &&
               shared_down && workspace && ids && scores && factor && hc_gate && hcs,
           MX_EINVAL, "mx_moe_routed_experts_hc_mfma: null pointer");
  MX_CHECK(rows >= 1 && rows <= 8, MX_EUNSUPPORTED,
           "mx_moe_routed_experts_hc_mfma: rows must be in 1..8");
  MX_CHECK(top_k >= 1 && top_k <= 15, MX_EUNSUPPORTED,
           "mx_moe_routed_experts_hc_mfma: top_k must be in 1..15");
  MX_CHECK(hc == 4, MX_EUNSUPPORTED, "mx_moe_routed_experts_hc_mfma: hc must be 4");
  MX_CHECK(experts % 64 == 0 && (experts / 64 == 1 || experts / 64 == 2 || experts / 64 == 4 ||
                                 experts / 64 == 8 || experts / 64 == 16),
           MX_EUNSUPPORTED,
           "mx_moe_routed_experts_hc_mfma: experts must be 64, 128, 256, 512 or 1024");
  MX_CHECK(logit_stride >= experts && shared_stride >= 1, MX_EINVAL,
           "mx_moe_routed_experts_hc_mfma: row strides too small");
  const QBank g = to_qbank(*gate), u = to_qbank(*up), d = to_qbank(*down);
  const QWeight sg = to_qweight(*shared_gate), su = to_qweight(*shared_up), sd = to_qweight(*shared_down);
  for (const QBank* b : {&g, &u, &d}) {
    if (const char* err = check_bank(*b))
      return mx_status(set_error(MX_EINVAL, std::string("mx_moe_routed_experts_hc_mfma: ") + err));
  }
  MX_CHECK(experts <= g.experts, MX_EINVAL,
           "mx_moe_routed_experts_hc_mfma: more logits than experts");
  MX_CHECK(g.n == u.n && g.k == u.k && d.k == g.n && d.n == g.k && g.experts == u.experts &&
               g.experts == d.experts && g.bits == u.bits && sg.n == su.n && sg.k == g.k &&
               su.k == g.k && sd.k == sg.n && sd.n == g.k && sg.bits == g.bits && sd.bits == d.bits,
           MX_EINVAL, "mx_moe_routed_experts_hc_mfma: banks and shared expert disagree in shape");
  MX_CHECK(skinny_down_hc_supported(rows, top_k, hc, d, sd), MX_EUNSUPPORTED,
           "mx_moe_routed_experts_hc_mfma: experts must be 512 deep (routed and shared), "
           "group_size 64, 4/5/6/8 bits, hidden a multiple of 16");
  uint16_t* h = static_cast<uint16_t*>(workspace);
  hipStream_t s = hipStream_t(stream);
  const RouteIO ro{logits, logit_stride, shared_logit, shared_stride, ids, scores, factor};
  int rc = skinny_route_gate_up(ro, experts, x, rows, top_k, g, u, sg, su, h, s);
  if (rc == MX_OK)
    rc = skinny_down_hc(h, ids, scores, factor, hc_gate, rows, top_k, hc, g.n, sg.n, d, sd, hcs,
                        s);
  return finish(rc, "mx_moe_routed_experts_hc_mfma");
}

MX_ABI mx_status mx_engine_fill_slot(mx_engine* e, int32_t slot, int32_t length, uint64_t seed) {
  MX_CHECK(e && slot_ok(*e->impl, slot), MX_EINVAL, "mx_engine_fill_slot: bad engine or slot");
  std::string err;
  return engine_status(engine_fill_slot(*e->impl, slot, length, seed, &err), err,
                       "mx_engine_fill_slot");
}
