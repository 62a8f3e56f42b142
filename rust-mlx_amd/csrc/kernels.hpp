// Internal launcher declarations shared by the C ABI and the engine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

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

// A bank of `experts` equally shaped quantised matrices stored back to back
// (MLX SwitchLinear layout: codes [E, n, k*bits/32], scales/biases [E, n, k/gs]).
struct QBank {
  const uint32_t* codes;
  const uint16_t* scales;
  const uint16_t* biases;
  int experts, n, k, bits, group_size;
};

inline QBank to_qbank(const mx_qbank& b) {
  return QBank{b.codes, b.scales, b.biases, b.experts, b.n, b.k, b.bits, b.group_size};
}

// Shape rules shared by every quantised projection; returns an error message
// or nullptr.
const char* check_qweight(const QWeight& w);

int qmv(const QWeight& w, const uint16_t* x, int m, uint16_t* y, hipStream_t s);
int dequant_rows(const QWeight& w, const uint32_t* ids, int count, uint16_t* out, hipStream_t s);

// ---- projections with fused epilogues (proj.hip) ----
enum ProjMode { kPlain = 0, kHcDown = 1, kHcUpMix = 2, kHcWrite = 3, kConv = 4 };
struct ProjEpilogue {
  int mode;
  uint16_t* y;        // output (kPlain/kHcDown/kHcUpMix) or the residual [M, hc*n] (kHcWrite)
  int64_t y_stride;   // elements between activation rows of y
  uint16_t* aux;      // injection gates [M, hc]: written by kHcDown, read by kHcWrite
  int64_t aux_stride;
  const uint16_t* xn; // normed streams [M, hc*hidden] (kHcUpMix)
  int64_t xn_stride;
  int rank;           // kHcDown: rows below rank are the low-rank branch
  int hc;             // hyper-connection streams
  int hidden;         // kHcUpMix: stream width H (w.n == 4 * H)
  // kConv (matrix-core 4-bit projections, one token per row, rows' slots
  // distinct): columns below conv_ch are causal-conv channels; their
  // bf16(silu(bf16(conv))) goes to conv_out and the window [slots, taps-1,
  // conv_ch] shifts in place (gdn_conv's arithmetic), columns from conv_ch on
  // go to y as in kPlain.  taps in 2..kConvMaxTaps.
  uint16_t* conv_state;
  const float* conv_w;       // [taps, conv_ch]
  const int32_t* slots;      // [M]
  uint16_t* conv_out;
  int64_t conv_stride;
  int conv_ch;
  int taps;
  // set by the launcher: a one-dimensional grid placed by XCD (block-plane
  // projections over both four-row blocks) with xcd_groups tiles
  int xcd_blocks = 0;
  int xcd_groups = 0;
  // prefill GEMM (more than 16 rows): fp32 workspace for partial sums when k
  // is split across workgroups (null: no split)
  float* part = nullptr;
  size_t part_floats = 0;
};
constexpr int kConvMaxTaps = 4;
int proj(const QWeight& w, const uint16_t* x, int64_t x_stride, int m, const ProjEpilogue& e,
         hipStream_t s);
// rows of one prefill chunk (speculative::prepare's chunks,
// src/speculative.rs:38-68; the reference passes 128: a 512-token chunk routes
// 5120 tokens, so each expert's weights stream once per 512 prompt tokens)
constexpr int kPrefillChunk = 512;
// matrix-core (MFMA) projections, 1..kQmmMaxRows rows, group size 64 (qmm.hip)
constexpr int kQmmMaxRows = kPrefillChunk;
bool qmm_supported(const QWeight& w);
int qmm(const QWeight& w, const uint16_t* x, int64_t x_stride, int m, const ProjEpilogue& e,
        hipStream_t s);
// exact-integer projections for 1..8 rows (xq.hip): the CPU oracle's
// mxo_xq arithmetic bit for bit, on the int8 matrix cores
// plane (nullable): the activation operands of x, written by its producer in
// the layout of xq_plane_bytes(K) (xq_core.hpp), in place of a staging
bool xq_supported(const QWeight& w);
size_t xq_plane_bytes(int k);
int xq_dense(const QWeight& w, const uint16_t* x, int64_t x_stride, int m, const ProjEpilogue& e,
             hipStream_t s, const char* plane = nullptr);
// exact hyper-connection up-projection + stream mix (kHcUpMix arithmetic)
// that also writes the operand plane of its output `mixed`
int xq_upmix(const QWeight& up, const uint16_t* lo, int m, const uint16_t* xn, int hidden,
             uint16_t* mixed, char* mixed_plane, hipStream_t s);
struct MoePlan;
// exact-integer expert MLPs over a MoePlan (same contracts as moe_gate_up /
// moe_down) and greedy-head partials (same layout as head_partials, parts =
// xq_head_parts(n); logits, when non-null, receives the bf16 logits)
int xq_gate_up(const uint16_t* x, const char* plane, const MoePlan* plan, int rows, int top_k,
               const QBank& gate, const QBank& up, const QWeight& sgate, const QWeight& sup,
               uint16_t* h, hipStream_t s);
int xq_down(const uint16_t* h, const MoePlan* plan, const uint16_t* scores, int rows, int top_k,
            int inter, int shared_inter, const QBank& down, const QWeight& sdown, uint16_t* p,
            hipStream_t s);
int xq_head_parts(int n);
int xq_head(const QWeight& w, const uint16_t* x, const char* plane, int m, float* maxima,
            uint32_t* indices, uint16_t* logits, int* parts_out, hipStream_t s);
// matrix-core skinny projections for 1..8 rows (skinny.hip)
bool skinny_supported(const QWeight& w);
int skinny_dense(const QWeight& w, const uint16_t* x, int64_t x_stride, int m,
                 const ProjEpilogue& e, hipStream_t s);
int skinny_gate_up(const uint16_t* x, const uint32_t* ids, int rows, int top_k,
                   const QBank& gate, const QBank& up, const QWeight& sgate, const QWeight& sup,
                   uint16_t* h, hipStream_t s);

// Router outputs and where the routes go (skinny_route_gate_up).
struct RouteIO {
  const uint16_t* logits;        // [rows, logit_stride]: experts' logits first
  int64_t logit_stride;
  const uint16_t* shared_logit;  // [rows, shared_stride]: the shared-expert gate logit
  int64_t shared_stride;
  uint32_t* ids;                 // [rows, top_k] out
  uint16_t* scores;              // [rows, top_k] out
  uint16_t* factor;              // [rows] out
};
// Routing tail + expert gate/up (+SwiGLU) in one: for 512 routed experts the
// persistent kernel routes its rows itself (bit-identical to moe_route) and
// writes ids / scores / factor; otherwise moe_route then skinny_gate_up.
int skinny_route_gate_up(const RouteIO& ro, int experts, const uint16_t* x, int rows, int top_k,
                         const QBank& gate, const QBank& up, const QWeight& sgate,
                         const QWeight& sup, uint16_t* h, hipStream_t s);
int skinny_down(const uint16_t* h, const uint32_t* ids, const uint16_t* scores, int rows,
                int top_k, int inter, int shared_inter, const QBank& down, const QWeight& sdown,
                uint16_t* p, hipStream_t s);
// Expert down + score + slot sum + hyper-connection write (hc == 4, 512-deep
// experts); bit-identical to skinny_down then moe_reduce_hc_epilogue with out
// = hcs.  MX_EUNSUPPORTED outside those shapes.
bool skinny_down_hc_supported(int rows, int top_k, int hc, const QBank& down,
                              const QWeight& sdown);
int skinny_down_hc(const uint16_t* h, const uint32_t* ids, const uint16_t* scores,
                   const uint16_t* factor, const uint16_t* hc_gate, int rows, int top_k, int hc,
                   int inter, int shared_inter, const QBank& down, const QWeight& sdown,
                   uint16_t* hcs, hipStream_t s);
int skinny_head_parts(int n);
// logits (nullable): also writes the bf16 logits [m, n] that the argmax ranks
int skinny_head(const QWeight& w, const uint16_t* x, int m, float* maxima, uint32_t* indices,
                int* parts_out, hipStream_t s, uint16_t* logits = nullptr);
// hyper-connection input projection on the matrix cores, two launches (hc.hip)
bool hc_fused_supported(const QWeight& down, const QWeight& up, int hc, int hidden, int rank);
size_t hc_fused_part_bytes(int n_down);
int hc_fused(const QWeight& down, const QWeight& up, const uint16_t* h, const uint16_t* scale,
             int M, int hc, int hidden, int rank, float eps, float* part, uint16_t* mixed,
             uint16_t* inj, hipStream_t s);
// plane (nullable, rows <= 8): also the exact-integer operand plane of y
int hc_norm(const uint16_t* x, const uint16_t* scale, int rows, int hc, int hidden, float eps,
            uint16_t* y, hipStream_t s, char* plane = nullptr);
int embed(const QWeight& w, const uint32_t* ids, int count, int hc, uint16_t* out, hipStream_t s);
// y[r][s][c] = bf16(e[r][c] + f[r hc + s][c]) (the MTP input, src/mtp.rs:103-106).
int mtp_combine(const uint16_t* e, const uint16_t* f, int rows, int hc, int hidden, uint16_t* y,
                hipStream_t s);

// ---- attention (attn.hip) ----
struct AttnDims {
  int heads, kv_heads, head_dim, rotary_dim;
  int max_ctx;           // positions per (slot, layer, kv head) in the cache
  int64_t slot_stride;   // elements between slots in the K (and V) cache
};
int attn_prep(const uint16_t* qkv, int64_t qkv_stride, int rows, const int32_t* slots,
              const int32_t* pos, const uint16_t* q_norm, const uint16_t* k_norm, float eps,
              const float* rope_cos, const float* rope_sin, AttnDims d, uint16_t* q_out,
              uint16_t* k_cache, uint16_t* v_cache, hipStream_t s);
// fast: the matrix-core kernel (64-position chunks, within tolerance) instead
// of the fixed-order one (256-position chunks).  o_part / ml_part hold
// max_chunks chunks per (row, head); max_chunks must cover max_ctx in chunks
// of the chosen kernel.
bool attn_fast_supported(AttnDims d);
int attn_decode(const uint16_t* q, int rows, const int32_t* slots, const int32_t* pos,
                const uint16_t* k_cache, const uint16_t* v_cache, AttnDims d, int max_chunks,
                bool fast, float* o_part, float* ml_part, hipStream_t s);
// plane (exact form only, rows <= 8): also writes the exact-integer operand
// plane of `out` (xq_plane_bytes(heads * head_dim) layout)
int attn_combine(const float* o_part, const float* ml_part, const uint16_t* qkv,
                 int64_t qkv_stride, int rows, const int32_t* pos, AttnDims d, int max_chunks,
                 bool fast, uint16_t* out, hipStream_t s, char* plane = nullptr);
constexpr int kAttnChunk = 256;
constexpr int kAttnFastChunk = 64;
// Prefill (fast mode): query rows of one slot in blocks that share each key
// tile, one partial per (row, head) and split of 256 keys at chunk index =
// split; attn_combine_splits merges them (and applies the output gate).
bool attn_prefill_supported(AttnDims d);
constexpr int attn_prefill_splits(int max_ctx) { return (max_ctx + 255) / 256; }
int attn_prefill(const uint16_t* q, int rows, const int32_t* slots, const int32_t* pos,
                 const uint16_t* k_cache, const uint16_t* v_cache, AttnDims d, int max_chunks,
                 float* o_part, float* ml_part, hipStream_t s);
int attn_combine_splits(const float* o_part, const float* ml_part, const uint16_t* qkv,
                        int64_t qkv_stride, int rows, const int32_t* pos, AttnDims d,
                        int max_chunks, uint16_t* out, hipStream_t s);
constexpr int kAttnRows = 128;  // query rows per attention launch of a prefill chunk

// ---- MoE ----
constexpr int kMaxRoutes = 8 * 16 + 1;
// Work list of one MoE step: distinct routed experts (first appearance order)
// and the shared expert (-1), each with the (row, slot) routes it serves.
// item[]: the (entry, four-row block of rows) pairs that have a member, as
// 2 entry + block, entries in order (the exact gate/up kernel's work list).
struct MoePlan {
  int32_t count;
  int32_t expert[kMaxRoutes];
  int32_t m[kMaxRoutes];
  uint8_t row[kMaxRoutes][8];
  uint8_t slot[kMaxRoutes][8];
  int32_t nitems;
  uint16_t item[2 * kMaxRoutes];
};
int moe_plan(const uint32_t* ids, int rows, int top_k, MoePlan* plan, hipStream_t s);
// moe_route then moe_plan of its ids, in one launch (rows <= 8)
int moe_route_plan(const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
                   int64_t shared_stride, int rows, int experts, int top_k, uint32_t* ids,
                   uint16_t* scores, uint16_t* factor, MoePlan* plan, hipStream_t s);
size_t moe_workspace_bytes(int rows, int top_k, int inter);
int moe_route(const uint16_t* logits, int64_t logit_stride, const uint16_t* shared_logit,
              int64_t shared_stride, int rows, int experts, int top_k, uint32_t* ids,
              uint16_t* scores, uint16_t* factor, hipStream_t s);
int moe_experts(const uint16_t* x, const uint32_t* ids, const uint16_t* scores, int rows,
                int top_k, const QBank& gate, const QBank& up, const QBank& down,
                const QWeight& sgate, const QWeight& sup, const QWeight& sdown, void* workspace,
                uint16_t* p, hipStream_t s);
int moe_gate_up(const uint16_t* x, const MoePlan* plan, int rows, int top_k, const QBank& gate,
                const QBank& up, const QWeight& sgate, const QWeight& sup, uint16_t* h,
                hipStream_t s);
int moe_down(const uint16_t* h, const MoePlan* plan, const uint16_t* scores, int rows, int top_k,
             int inter, int shared_inter, const QBank& down, const QWeight& sdown, uint16_t* p,
             hipStream_t s);
int qmm_gate_up(const uint16_t* x, const MoePlan* plan, int rows, int top_k, const QBank& gate,
                const QBank& up, const QWeight& sgate, const QWeight& sup, uint16_t* h,
                hipStream_t s);
int qmm_down(const uint16_t* h, const MoePlan* plan, const uint16_t* scores, int rows, int top_k,
             int inter, int shared_inter, const QBank& down, const QWeight& sdown, uint16_t* p,
             hipStream_t s);
// Work list of a prefill chunk's experts (more than eight rows): the routes
// grouped by expert (experts in index order, then the shared expert -1), each
// expert's routes in row order, cut into items of at most 16 routes (one
// 16-row matrix-core tile).  member row / slot: the slot is top_k for the
// shared expert.
constexpr int kChunkRoutes = kPrefillChunk * 17;  // top_k <= 16, plus the shared slot
constexpr int kChunkMaxExperts = 1023;
struct ChunkPlan {
  int32_t nitems;
  int32_t expert[kChunkRoutes];
  int32_t start[kChunkRoutes];
  int32_t m[kChunkRoutes];
  uint16_t row[kChunkRoutes];
  uint8_t slot[kChunkRoutes];
};
// items a chunk of `rows` rows can produce (a bound: the grids' y extent)
int chunk_max_items(int rows, int experts, int top_k);
int chunk_plan(const uint32_t* ids, int rows, int experts, int top_k, ChunkPlan* plan,
               hipStream_t s);
// matrix-core expert MLPs over a ChunkPlan (qmm.hip): h [rows][top_k + 1][hs]
// and p [rows][top_k + 1][hidden], the contracts of moe_gate_up / moe_down
int qmm_chunk_gate_up(const uint16_t* x, const ChunkPlan* plan, int rows, int experts, int top_k,
                      const QBank& gate, const QBank& up, const QWeight& sgate,
                      const QWeight& sup, uint16_t* h, hipStream_t s);
int qmm_chunk_down(const uint16_t* h, const ChunkPlan* plan, const uint16_t* scores, int rows,
                   int experts, int top_k, int inter, int shared_inter, const QBank& down,
                   const QWeight& sdown, uint16_t* p, hipStream_t s);
int moe_reduce(const uint16_t* p, int rows, int top_k, int hidden, uint16_t* routed,
               hipStream_t s);
int moe_hc_epilogue(const uint16_t* routed, const uint16_t* shared, const uint16_t* factor,
                    const uint16_t* residual, const uint16_t* gate, int rows, int hc, int hidden,
                    uint16_t* out, hipStream_t s);
int moe_reduce_hc_epilogue(const uint16_t* p, const uint16_t* factor, const uint16_t* residual,
                           const uint16_t* gate, int rows, int top_k, int hc, int hidden,
                           uint16_t* out, hipStream_t s);
// moe_reduce_hc_epilogue in place on h, then hc_norm of the result with
// `scale` into xn and its operand plane, in one launch (same bits)
bool moe_reduce_norm_supported(int rows, int top_k, int hc, int hidden);
int moe_reduce_norm(const uint16_t* p, const uint16_t* factor, uint16_t* h, const uint16_t* gate,
                    int rows, int top_k, int hc, int hidden, const uint16_t* scale, float eps,
                    uint16_t* xn, char* plane, hipStream_t s);

// ---- greedy head ----
int head_parts(int n, int k);
int head_partials(const QWeight& w, const uint16_t* x, int m, float* maxima, uint32_t* indices,
                  int* parts, hipStream_t s);
// Greedy head without a workspace: the partials live in a static device
// array of kHeadNoAllocScratchBytes per GPU (head.hip); MX_EUNSUPPORTED when
// head_noalloc_bytes(n, k, m) exceeds it.
constexpr size_t kHeadNoAllocScratchBytes = size_t(1) << 20;
size_t head_noalloc_bytes(int n, int k, int m);
int head_argmax_noalloc(const QWeight& w, const uint16_t* x, int m, uint32_t* tokens,
                        hipStream_t s);
int argmax_reduce(const float* maxima, const uint32_t* indices, int rows, int parts,
                  uint32_t* tokens, hipStream_t s);
int argmax_bf16(const uint16_t* logits, int rows, int n, uint32_t* tokens, hipStream_t s);

// ---- GatedDeltaNet ----
struct GdnDims {
  int hk, hv, dk, dv, conv_k;  // key heads, value heads, head dims, conv taps
};
int gdn_conv(const uint16_t* qkv, int64_t row_stride, int groups, int t, const int32_t* slots,
             uint16_t* conv_state, const float* conv_w, int channels, int conv_k,
             uint16_t* out, int64_t out_stride, uint16_t* window_history, hipStream_t s);
// fast-mode step (t tokens per group, optional history; every token gives the
// bits of a one-token call), gdn.hip
int gdn_recurrence_fast(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                        const uint16_t* a, const uint16_t* b, int64_t zab_stride,
                        const float* a_log, const uint16_t* dt_bias, const uint16_t* norm_w,
                        float eps, GdnDims d, int groups, int t, const int32_t* slots,
                        float* state, float* history, uint16_t* y, hipStream_t s);
// plane (rows <= 8): also writes the exact-integer operand plane of y
// (xq_plane_bytes(hv * 128) layout)
int gdn_recurrence(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                   const uint16_t* a, const uint16_t* b, int64_t zab_stride, const float* a_log,
                   const uint16_t* dt_bias, const uint16_t* norm_w, float eps, GdnDims d,
                   int groups, int t, const int32_t* slots, float* state, float* history,
                   uint16_t* y, hipStream_t s, char* plane = nullptr);
int gdn_scan(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
             const uint16_t* beta, GdnDims d, int groups, int t, const int32_t* slots,
             float* state, float* history, uint16_t* y, hipStream_t s);
// unquantised bf16 GEMV, 1..8 rows, k % 128 == 0 (gemv.hip)
int gemv_bf16(const uint16_t* w, int n, int k, const uint16_t* x, int rows, uint16_t* y,
              hipStream_t s);
// chunked prefill form of gdn_scan (gdn_chunk.hip): same inputs and outputs,
// fp32 matrix-core products over 64-token chunks; workspace from
// gdn_chunk_workspace_bytes.  v_stride: elements between token rows of v
// (0: hv * dv, dense).
size_t gdn_chunk_workspace_bytes(int groups, int hv, int t);
int gdn_prefill_chunked(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                        const uint16_t* beta, GdnDims d, int groups, int t, const int32_t* slots,
                        float* state, uint16_t* y, float* workspace, hipStream_t s,
                        int64_t v_stride = 0);
// The fast GDN step of a prefill chunk (t tokens of each group) through the
// chunked scan: normalised q / k, decay and beta per token (the fast step's
// arithmetic) into `io`, gdn_prefill_chunked, then the gated RMS norm into y.
// io: gdn_chunk_io_bytes(rows, d) bytes; workspace as gdn_prefill_chunked.
size_t gdn_chunk_io_bytes(int rows, GdnDims d);
int gdn_chunk_fast(const uint16_t* conv_out, int64_t conv_stride, const uint16_t* z,
                   const uint16_t* a, const uint16_t* b, int64_t zab_stride, const float* a_log,
                   const uint16_t* dt_bias, const uint16_t* norm_w, float eps, GdnDims d,
                   int groups, int t, const int32_t* slots, float* state, uint16_t* y, void* io,
                   float* workspace, hipStream_t s);

// ---- engine (engine.cpp) ----
struct Engine;
int engine_create(const mx_model_config& cfg, Engine** out);
void engine_destroy(Engine* e);
int engine_reset_slot(Engine& e, int slot);
int engine_clone_slot(Engine& e, int src, int dst);
int engine_offset(const Engine& e, int slot);
int engine_slot_failed(const Engine& e, int slot);
void engine_inject_failure(Engine& e, int after_layers);
int engine_decode_rows(Engine& e, const int32_t* slots, const uint32_t* tokens, int rows,
                       uint32_t* next, std::string* err);
int engine_decode_outputs(Engine& e, const int32_t* slots, const uint32_t* tokens, int rows,
                          uint32_t* next, uint16_t* logits, uint16_t* hidden, std::string* err);
int engine_decode_forced(Engine& e, const int32_t* slots, const uint32_t* tokens, int rows,
                         const uint16_t* h_in, uint16_t* h_out, uint32_t* ids_out,
                         uint32_t* next, std::string* err);
int engine_block(Engine& e, int slot, const uint32_t* tokens, int count, bool history,
                 uint32_t* next, std::string* err);
int engine_prefill_chunked(Engine& e, int slot, const uint32_t* tokens, int count,
                           uint32_t* next, std::string* err);
int engine_verify(Engine& e, int slot, const uint32_t* tokens, int count, uint32_t* next,
                  std::string* err);
int engine_commit(Engine& e, int slot, int keep, std::string* err);
int engine_generate(Engine& e, int slot, const uint32_t* prompt, int n_prompt, int max_tokens,
                    int depth, uint32_t* out, int* n_out, mx_generate_stats* stats,
                    uint32_t* drafts, std::string* err);
int engine_read(Engine& e, const char* what, void* host, size_t bytes, std::string* err);
int engine_tensor(Engine& e, const char* name, void** ptr, size_t* bytes);
// Where an MLX-named checkpoint tensor goes (engine.cpp): rows [row0, row0 +
// rows) of the engine matrix `tensor` (n x k at `bits`; part 0 codes, 1
// scales, 2 biases), or `count` values of a bf16 / fp32 vector, or the GDN
// conv weight.  MX_EUNSUPPORTED for modules the engine does not build.
struct CheckpointTarget {
  enum Kind { kQuant = 0, kBf16 = 1, kF32 = 2, kConvW = 3 } kind = kQuant;
  std::string tensor;
  int n = 0, k = 0, bits = 0, row0 = 0, rows = 0, part = 0;
  size_t count = 0;
  int conv_ch = 0, taps = 0;
};
int checkpoint_target(const mx_model_config& c, std::string name, CheckpointTarget* t);
int engine_load_tensor(Engine& e, const char* name, int dtype, const int64_t* shape, int ndim,
                       const void* data, size_t bytes, std::string* err);
int engine_load_safetensors(Engine& e, const char* path, int* loaded, std::string* err);
int checkpoint_check(const mx_model_config& c, const char* path, int* checked, std::string* err);
int engine_fill_slot(Engine& e, int slot, int length, uint64_t seed, std::string* err);
int engine_time_experts(Engine& e, int rows, mx_expert_timing* out, std::string* err);
int engine_profile_step(Engine& e, const int32_t* slots, const uint32_t* tokens, int rows,
                        uint32_t* next, mx_step_profile* out, std::string* err);
int engine_profile_verify(Engine& e, int slot, const uint32_t* tokens, int count, uint32_t* next,
                          mx_step_profile* out, std::string* err);
int engine_draft_bytes(const Engine& e, int pos, double* bytes, std::string* err);
void engine_set_flags(Engine& e, int want_logits, int use_graphs, int exact, int exact_parts,
                      int chunked_generate);
const mx_model_config& engine_config(const Engine& e);
int engine_gdn_layers(const Engine& e);
int engine_attn_layers(const Engine& e);
hipStream_t engine_stream(const Engine& e);

int fill_bf16(uint16_t* dst, size_t count, uint64_t seed, int dist, float a, float b,
              hipStream_t s);
int fill_codes(uint32_t* dst, int64_t rows, int k, int bits, uint64_t seed, hipStream_t s);
int fill_bias_centered(uint16_t* b, const uint16_t* scales, size_t count, int bits, uint64_t seed,
                       float noise, hipStream_t s);
int fill_f32(float* dst, size_t count, uint64_t seed, float a, float b, hipStream_t s);
int eval_math(int op, const float* in, float* out, int64_t n, hipStream_t s);

}  // namespace mx
