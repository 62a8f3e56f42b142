// The decode engine: a synthetic hybrid GatedDeltaNet / gated-attention MoE
// model resident in HBM, per-slot recurrent and KV caches, and the batched
// step that runs every layer's kernels on one HIP stream.
//
// Reference: HybridModel / HybridLayer / HybridCache (src/hybrid.rs:500-759),
// HybridModel::decode_batch (src/batching.rs:34-170) and the generation entry
// points of src/speculative.rs (prepare 38-68, generate_prepared 225-483).
//
// MI355X-first differences from the reference's design:
//  * caches live in a slot arena (state/conv/KV indexed by slot id) instead of
//    being concatenated and split around every batched step
//    (batching.rs:54-90, 138-169): a step names its rows' slots;
//  * every row carries its own position, so rows at different offsets can
//    share one step (the reference's equal-offset rule is kept as the
//    decode_batch contract and checked on the host);
//  * the whole step is captured once per row shape into a HIP graph and
//    replayed; only the small per-step row table is copied in before launch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "kernels.hpp"

namespace mx {

namespace {

struct Buf {
  void* p = nullptr;
  size_t bytes = 0;
};

struct QW {
  QWeight w{};
};

struct HcW {
  uint16_t* scale = nullptr;  // [hc * H]
  QWeight down{};             // [rank (+ hc inject rows), hc * H]
  QWeight up{};               // [hc * H, rank]
  bool inject = false;
};

struct LayerW {
  bool attn = false;
  int cache_index = 0;  // index among GDN layers or among attention layers
  HcW attn_hc, mlp_hc;
  // GatedDeltaNet
  QWeight gdn_in{};  // [cd + vd + 2 hv, H]: qkv | z | a | b
  float* conv_w = nullptr;
  float* a_log = nullptr;
  uint16_t* dt_bias = nullptr;
  uint16_t* gdn_norm = nullptr;
  QWeight gdn_out{};
  // attention
  QWeight attn_in{};  // [heads*2*hd + 2*kvh*hd, H]: (q, gate) per head | k | v
  uint16_t* q_norm = nullptr;
  uint16_t* k_norm = nullptr;
  QWeight attn_out{};
  // MoE
  QWeight router{};  // [E + 1, H]: router rows then the shared-expert gate
  QBank gate{}, up{}, down{};
  QWeight sgate{}, sup{}, sdown{};
};

}  // namespace

struct Engine {
  mx_model_config cfg{};
  hipStream_t stream = nullptr;
  std::vector<Buf> allocs;
  std::map<std::string, Buf> tensors;
  std::vector<LayerW> layers;
  QWeight embed{}, head{};
  HcW mixer;
  int n_gdn = 0, n_attn = 0;
  int n_kv = 0;  // attention cache planes per slot: n_attn (+ 1 for the MTP layer)
  // MTP draft layer (src/mtp.rs:10-127): norms, the two input projections,
  // one attention + MoE layer with hyper-connections, and its mixer
  struct Mtp {
    uint16_t* norm_emb = nullptr;  // [H]
    uint16_t* norm_hid = nullptr;  // [hc * H]
    QWeight fc_emb{}, fc_hid{};    // [H, H]
    LayerW layer;
    HcW mixer;
  } mtp;
  bool has_mtp = false;
  uint16_t *mtp_emb = nullptr, *mtp_a = nullptr, *mtp_e = nullptr;   // [rows][H]
  uint16_t *mtp_prev = nullptr, *mtp_hn = nullptr, *mtp_f = nullptr;  // [rows][hc H]
  uint16_t* mtp_dh = nullptr;                                          // [hc H]
  // dims
  int H = 0, cd = 0, vd = 0, P = 0, Q = 0, max_chunks = 0;
  GdnDims gd{};
  AttnDims ad{};
  // caches
  float* gdn_state = nullptr;     // [slots][n_gdn][hv][dk][dv]
  uint16_t* conv_state = nullptr; // [slots][n_gdn][K-1][cd]
  uint16_t* k_cache = nullptr;    // [slots][n_attn][kvh][max_ctx][hd]
  uint16_t* v_cache = nullptr;
  float* rope_cos = nullptr;      // [max_ctx][rot/2]
  float* rope_sin = nullptr;
  // verify history and snapshot of one slot
  float* hist_state = nullptr;    // [n_gdn][max_verify][hv][dk][dv]
  uint16_t* hist_conv = nullptr;  // [n_gdn][K-1+max_verify][cd]
  float* snap_state = nullptr;    // [n_gdn][hv][dk][dv]
  uint16_t* snap_conv = nullptr;  // [n_gdn][K-1][cd]
  int verify_slot = -1, verify_count = 0, verify_base = 0;
  // activations (rows <= kPrefillChunk: a decode step or verify block uses
  // at most 8, a prefill chunk up to kPrefillChunk)
  uint16_t *h = nullptr, *xn = nullptr, *lo = nullptr, *inj = nullptr, *mixed = nullptr;
  uint16_t *pbuf = nullptr, *conv_out = nullptr, *y = nullptr, *qrot = nullptr, *attn_y = nullptr;
  uint16_t *logits_r = nullptr, *scores = nullptr, *factor = nullptr, *moe_p = nullptr;
  uint16_t *moe_h = nullptr, *logits = nullptr;
  void* moe_ws = nullptr;
  MoePlan* moe_plan_buf = nullptr;
  ChunkPlan* chunk_plan = nullptr;  // expert work list of a prefill chunk
  float* gemm_part = nullptr;       // a prefill chunk's k-split GEMM partials
  size_t gemm_part_floats = 0;
  void* gdn_io = nullptr;           // a prefill chunk's GDN scan inputs
  float* gdn_ws = nullptr;          // and the chunked scan's workspace
  uint32_t* ids = nullptr;
  float *o_part = nullptr, *ml_part = nullptr;
  void* head_ws = nullptr;
  float* hc_part = nullptr;  // partial sums of the fused HC projection
  // exact-integer operand planes of the normed streams xn and of `mixed`,
  // written by their producers (exact mode) and read by every projection of
  // those activations
  char* xn_plane = nullptr;
  char* mixed_plane = nullptr;
  char* y_plane = nullptr;  // operand plane of the GDN / attention output (exact mode)
  // per-step row table (device) and its pinned host mirror
  struct RowTable {
    uint32_t tokens[kPrefillChunk];
    int32_t slots[kPrefillChunk];
    int32_t pos[kPrefillChunk];
    int32_t gdn_slots[kPrefillChunk];
    uint32_t next[kPrefillChunk];
  };
  RowTable* dev_rows = nullptr;
  RowTable* host_rows = nullptr;
  std::vector<int32_t> offsets;
  bool want_logits = false;
  int last_rows = 0;
  // slots whose caches a failed step left partly advanced (refused until a
  // reset or a clone replaces them); a test hook makes the next step fail
  // after `fail_after` layers have been launched
  std::vector<uint8_t> failed;
  int fail_after = 0;
  // captured graphs keyed by (rows, groups, t, history, logits)
  std::map<int, hipGraphExec_t> graphs;
  bool use_graphs = true;
  // exact: every projection on the fixed-order VALU kernels (bit-identical to
  // the CPU oracle); otherwise dense and expert projections run on the matrix
  // cores (router and vocabulary head stay exact in both modes)
  bool exact = false;
  // finer diagnostic switch: components (kEx* bits) that run on the exact
  // kernels while the rest stays on the matrix cores
  int exact_parts = 0;
  // set while a prefill chunk is recorded: every component on the matrix-core
  // kernels, whatever `exact` says
  bool chunk = false;
  // engine_generate prefills its prompt in chunks (and runs the draft layer's
  // prompt pass chunk by chunk)
  bool chunked_generate = false;
  // set while recording: the last MoE slot sum also normed the streams for
  // the next hyper-connection (xn and its plane are written), whose own norm
  // launch is then skipped
  bool xn_ready = false;
  // profiling (eager steps only): events around each layer's expert kernels
  mx_step_profile* prof = nullptr;
  double prof_routed = 0.0;  // profiled steps: routed expert bytes, summed over layers
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};

  ~Engine();
};

Engine::~Engine() {
  for (auto& g : graphs) hipGraphExecDestroy(g.second);
  for (auto& v : ev)
    if (v) hipEventDestroy(v);
  for (auto& a : allocs) hipFree(a.p);
  if (host_rows) hipHostFree(host_rows);
  if (stream) hipStreamDestroy(stream);
}

namespace {

// Components of a layer that the diagnostic mask can move to the exact kernels.
enum : int {
  kExHc = 1,        // hyper-connection projections (and their norm / mix)
  kExGdnProj = 2,   // GDN input and output projections
  kExGdn = 4,       // GDN recurrence
  kExAttnProj = 8,  // attention input and output projections
  kExAttn = 16,     // attention core
  kExMoe = 32,      // router projection, routing and experts
  kExHead = 64,     // vocabulary head
};

bool ex(const Engine& e, int part) {
  return !e.chunk && (e.exact || (e.exact_parts & part) != 0);
}

// The operand plane of e.mixed when its producer wrote one (the exact
// hyper-connection path), else null (the consumer stages its operands).
const char* mixed_plane(const Engine& e, int rows) {
  return ex(e, kExHc) && rows <= 8 ? e.mixed_plane : nullptr;
}


uint64_t tensor_seed(uint64_t base, int layer, int id) {
  // distinct streams per (layer, tensor); QWeight-style tensors use seed, +1, +2
  return base + uint64_t(layer + 1) * 1000ull + uint64_t(id) * 10ull;
}

int alloc(Engine& e, const std::string& name, size_t bytes, void** out) {
  void* p = nullptr;
  const hipError_t err = hipMalloc(&p, bytes ? bytes : 1);
  if (err != hipSuccess) return hip_error(err, ("hipMalloc " + name).c_str());
  e.allocs.push_back({p, bytes});
  if (!name.empty()) e.tensors[name] = {p, bytes};
  *out = p;
  return MX_OK;
}

#define MX_TRY(x)                \
  do {                           \
    const int rc_ = (x);         \
    if (rc_ != MX_OK) return rc_; \
  } while (0)

int make_qw(Engine& e, const std::string& name, int n, int k, int bits, int layer, int id,
            QWeight* out, float s_lo = 0.005f, float s_hi = 0.03f) {
  const int gs = e.cfg.group_size;
  void *c, *s, *b;
  MX_TRY(alloc(e, name + ".codes", size_t(n) * k * bits / 8, &c));
  MX_TRY(alloc(e, name + ".scales", size_t(n) * (k / gs) * 2, &s));
  MX_TRY(alloc(e, name + ".biases", size_t(n) * (k / gs) * 2, &b));
  const uint64_t seed = tensor_seed(e.cfg.seed, layer, id);
  MX_TRY(fill_codes(static_cast<uint32_t*>(c), n, k, bits, seed, e.stream));
  MX_TRY(fill_bf16(static_cast<uint16_t*>(s), size_t(n) * (k / gs), seed + 1, 0, s_lo, s_hi, e.stream));
  // zero-mean weights (b ~ -s * mid): a random model whose rows stay distinct
  // through the stack, so routing spreads over the experts as in a trained model
  MX_TRY(fill_bias_centered(static_cast<uint16_t*>(b), static_cast<uint16_t*>(s), size_t(n) * (k / gs),
                            bits, seed + 2, 0.01f, e.stream));
  *out = QWeight{static_cast<uint32_t*>(c), static_cast<uint16_t*>(s), static_cast<uint16_t*>(b),
                 n, k, bits, gs};
  return MX_OK;
}

int make_bank(Engine& e, const std::string& name, int experts, int n, int k, int bits, int layer,
              int id, QBank* out) {
  QWeight w;
  MX_TRY(make_qw(e, name, experts * n, k, bits, layer, id, &w));
  *out = QBank{w.codes, w.scales, w.biases, experts, n, k, bits, w.group_size};
  return MX_OK;
}

int make_bf16(Engine& e, const std::string& name, size_t count, int layer, int id, int dist,
              float a, float b, uint16_t** out) {
  void* p;
  MX_TRY(alloc(e, name, count * 2, &p));
  MX_TRY(fill_bf16(static_cast<uint16_t*>(p), count, tensor_seed(e.cfg.seed, layer, id), dist, a, b,
                   e.stream));
  *out = static_cast<uint16_t*>(p);
  return MX_OK;
}

// fp32 tensor from a bf16 draw (exact widening), on the host then uploaded.
int make_f32_from_draw(Engine& e, const std::string& name, size_t count, int layer, int id,
                       int dist, float a, float b, bool log_of, float** out) {
  std::vector<uint16_t> tmp(count);
  // draw on the device, read back, widen (and optionally take log) on the host
  uint16_t* d16;
  MX_TRY(make_bf16(e, "", count, layer, id, dist, a, b, &d16));
  if (hipMemcpyAsync(tmp.data(), d16, count * 2, hipMemcpyDeviceToHost, e.stream) != hipSuccess ||
      hipStreamSynchronize(e.stream) != hipSuccess)
    return MX_EHIP;
  std::vector<float> f(count);
  for (size_t i = 0; i < count; ++i) {
    const float v = bf16_to_f32(tmp[i]);
    f[i] = log_of ? std::log(v) : v;
  }
  void* p;
  MX_TRY(alloc(e, name, count * 4, &p));
  if (hipMemcpy(p, f.data(), count * 4, hipMemcpyHostToDevice) != hipSuccess) return MX_EHIP;
  *out = static_cast<float*>(p);
  return MX_OK;
}

int layer_bits(const mx_model_config& c, int layer, int which) {
  // which: 0 = main projections, 1 = expert down; tensors outside the layer
  // stack (layer < 0) always use the base widths; a checkpoint's width table
  // overrides the base widths and the mixed_bits draw
  if (layer >= 0 && layer <= MX_MAX_LAYERS && c.layer_widths[2 * layer + which] != 0)
    return c.layer_widths[2 * layer + which];
  if (!c.mixed_bits || layer < 0) return which == 0 ? c.bits : c.down_bits;
  static const int choices[4] = {4, 5, 6, 8};
  const uint64_t r = rng_u64(c.seed ^ 0x5bd1e995ull, uint64_t(layer) * 2 + which);
  return choices[r & 3];
}

int make_hc(Engine& e, const std::string& p, int layer, int id0, bool inject, HcW* out) {
  const auto& c = e.cfg;
  const int bits = layer_bits(c, layer, 0);
  out->inject = inject;
  MX_TRY(make_bf16(e, p + ".scale", size_t(c.hc) * c.hidden, layer, id0, 1, 0.1f, 0.0f, &out->scale));
  MX_TRY(make_qw(e, p + ".down", c.hc_rank + (inject ? c.hc : 0), c.hc * c.hidden, bits, layer,
                 id0 + 1, &out->down));
  MX_TRY(make_qw(e, p + ".up", c.hc * c.hidden, c.hc_rank, bits, layer, id0 + 2, &out->up));
  return MX_OK;
}

// One layer's tensors (p: name prefix, i: layer index of the draws).
int make_layer(Engine& e, const std::string& p, int i, LayerW* out) {
  const auto& c = e.cfg;
  LayerW& L = *out;
  {
    const int bits = layer_bits(c, i, 0);
    const int dbits = layer_bits(c, i, 1);
    MX_TRY(make_hc(e, p + ".attn_hc", i, 1, true, &L.attn_hc));
    MX_TRY(make_hc(e, p + ".mlp_hc", i, 4, true, &L.mlp_hc));
    if (!L.attn) {
      MX_TRY(make_qw(e, p + ".gdn.in", e.P, c.hidden, bits, i, 7, &L.gdn_in));
      // conv weight ~ N(0, 0.5), A = exp(A_log) ~ U(0, 16), dt ~ U(-1, 1), norm ~ 1 + N(0, .1)
      MX_TRY(make_f32_from_draw(e, p + ".gdn.conv_w", size_t(c.conv_k) * e.cd, i, 8, 1, 0.5f, 0.0f,
                                false, &L.conv_w));
      MX_TRY(make_f32_from_draw(e, p + ".gdn.a_log", c.gdn_hv, i, 9, 0, 0.01f, 16.0f, true, &L.a_log));
      MX_TRY(make_bf16(e, p + ".gdn.dt_bias", c.gdn_hv, i, 10, 0, -1.0f, 1.0f, &L.dt_bias));
      MX_TRY(make_bf16(e, p + ".gdn.norm", c.gdn_dv, i, 11, 1, 0.1f, 1.0f, &L.gdn_norm));
      MX_TRY(make_qw(e, p + ".gdn.out", c.hidden, e.vd, bits, i, 12, &L.gdn_out));
    } else {
      MX_TRY(make_qw(e, p + ".attn.in", e.Q, c.hidden, bits, i, 7, &L.attn_in));
      MX_TRY(make_bf16(e, p + ".attn.q_norm", c.head_dim, i, 8, 1, 0.1f, 0.0f, &L.q_norm));
      MX_TRY(make_bf16(e, p + ".attn.k_norm", c.head_dim, i, 9, 1, 0.1f, 0.0f, &L.k_norm));
      MX_TRY(make_qw(e, p + ".attn.out", c.hidden, c.heads * c.head_dim, bits, i, 12, &L.attn_out));
    }
    MX_TRY(make_qw(e, p + ".moe.router", c.experts + 1, c.hidden, bits, i, 13, &L.router));
    MX_TRY(make_bank(e, p + ".moe.gate", c.experts, c.moe_inter, c.hidden, bits, i, 14, &L.gate));
    MX_TRY(make_bank(e, p + ".moe.up", c.experts, c.moe_inter, c.hidden, bits, i, 15, &L.up));
    MX_TRY(make_bank(e, p + ".moe.down", c.experts, c.hidden, c.moe_inter, dbits, i, 16, &L.down));
    MX_TRY(make_qw(e, p + ".moe.shared_gate", c.shared_inter, c.hidden, bits, i, 17, &L.sgate));
    MX_TRY(make_qw(e, p + ".moe.shared_up", c.shared_inter, c.hidden, bits, i, 18, &L.sup));
    MX_TRY(make_qw(e, p + ".moe.shared_down", c.hidden, c.shared_inter, dbits, i, 19, &L.sdown));
  }
  return MX_OK;
}

int build(Engine& e) {
  const auto& c = e.cfg;
  e.H = c.hidden;
  e.gd = GdnDims{c.gdn_hk, c.gdn_hv, c.gdn_dk, c.gdn_dv, c.conv_k};
  e.cd = 2 * c.gdn_hk * c.gdn_dk + c.gdn_hv * c.gdn_dv;
  e.vd = c.gdn_hv * c.gdn_dv;
  e.P = e.cd + e.vd + 2 * c.gdn_hv;
  e.Q = c.heads * 2 * c.head_dim + 2 * c.kv_heads * c.head_dim;
  e.max_chunks = (c.max_context + kAttnFastChunk - 1) / kAttnFastChunk;
  for (int i = 0; i < c.layers; ++i) {
    LayerW L;
    L.attn = (i % c.attn_every) == c.attn_every - 1;
    L.cache_index = L.attn ? e.n_attn++ : e.n_gdn++;
    e.layers.push_back(L);
  }
  e.n_kv = e.n_attn + (c.mtp ? 1 : 0);
  const int64_t attn_slot_stride = int64_t(e.n_kv) * c.kv_heads * c.max_context * c.head_dim;
  e.ad = AttnDims{c.heads, c.kv_heads, c.head_dim, c.rotary_dim, c.max_context, attn_slot_stride};

  // ---- weights ----
  MX_TRY(make_qw(e, "embed", c.vocab, c.hidden, c.embed_bits, -1, 1, &e.embed));
  MX_TRY(make_qw(e, "head", c.vocab, c.hidden, c.head_bits, -1, 2, &e.head));
  MX_TRY(make_hc(e, "mixer", -1, 3, false, &e.mixer));
  for (int i = 0; i < c.layers; ++i)
    MX_TRY(make_layer(e, "layers." + std::to_string(i), i, &e.layers[i]));
  if (c.mtp) {
    // the MTP layer draws its tensors as layer index `layers`
    // (mtp.rs:39-70: pre_fc_norm_embedding / _hidden, fc_embedding / _hidden,
    // one attention layer with its two hyper-connections, the mixer)
    const int m = c.layers;
    const int bits = layer_bits(c, m, 0);
    e.has_mtp = true;
    e.mtp.layer.attn = true;
    e.mtp.layer.cache_index = e.n_attn;  // the plane after the model's attention layers
    MX_TRY(make_layer(e, "mtp.layer", m, &e.mtp.layer));
    MX_TRY(make_bf16(e, "mtp.norm_emb", c.hidden, m, 20, 1, 0.1f, 0.0f, &e.mtp.norm_emb));
    MX_TRY(make_bf16(e, "mtp.norm_hidden", size_t(c.hc) * c.hidden, m, 21, 1, 0.1f, 0.0f,
                     &e.mtp.norm_hid));
    MX_TRY(make_qw(e, "mtp.fc_emb", c.hidden, c.hidden, bits, m, 22, &e.mtp.fc_emb));
    MX_TRY(make_qw(e, "mtp.fc_hidden", c.hidden, c.hidden, bits, m, 23, &e.mtp.fc_hid));
    MX_TRY(make_hc(e, "mtp.mixer", m, 24, false, &e.mtp.mixer));
  }

  // ---- caches ----
  void* v;
  const size_t S = size_t(c.max_slots);
  const size_t state_per = size_t(c.gdn_hv) * c.gdn_dk * c.gdn_dv;
  MX_TRY(alloc(e, "cache.gdn_state", S * e.n_gdn * state_per * 4, &v));
  e.gdn_state = static_cast<float*>(v);
  MX_TRY(alloc(e, "cache.conv_state", S * e.n_gdn * (c.conv_k - 1) * e.cd * 2, &v));
  e.conv_state = static_cast<uint16_t*>(v);
  MX_TRY(alloc(e, "cache.k", S * attn_slot_stride * 2, &v));
  e.k_cache = static_cast<uint16_t*>(v);
  MX_TRY(alloc(e, "cache.v", S * attn_slot_stride * 2, &v));
  e.v_cache = static_cast<uint16_t*>(v);
  MX_TRY(alloc(e, "verify.state", size_t(e.n_gdn) * c.max_verify * state_per * 4, &v));
  e.hist_state = static_cast<float*>(v);
  MX_TRY(alloc(e, "verify.conv", size_t(e.n_gdn) * (c.conv_k - 1 + c.max_verify) * e.cd * 2, &v));
  e.hist_conv = static_cast<uint16_t*>(v);
  MX_TRY(alloc(e, "verify.snap_state", size_t(e.n_gdn) * state_per * 4, &v));
  e.snap_state = static_cast<float*>(v);
  MX_TRY(alloc(e, "verify.snap_conv", size_t(e.n_gdn) * (c.conv_k - 1) * e.cd * 2, &v));
  e.snap_conv = static_cast<uint16_t*>(v);

  // RoPE table: inv_freq[i] = 1 / theta^(2i/rot) in fp32 (src/rope.rs:20-24);
  // the angle is the fp32 product pos * inv_freq (kernels/text_rope.metal),
  // cos/sin of that fp32 angle rounded to fp32.
  {
    const int half = c.rotary_dim / 2;
    std::vector<float> cs(size_t(c.max_context) * half), sn(cs.size());
    for (int i = 0; i < half; ++i) {
      const float power = float(2 * i) / float(c.rotary_dim);
      const float inv = 1.0f / ::powf(c.rope_theta, power);  // fp32 pow, as MLX's f32 power
      for (int p = 0; p < c.max_context; ++p) {
        const float a = float(p) * inv;
        cs[size_t(p) * half + i] = float(std::cos(double(a)));
        sn[size_t(p) * half + i] = float(std::sin(double(a)));
      }
    }
    MX_TRY(alloc(e, "rope.cos", cs.size() * 4, &v));
    e.rope_cos = static_cast<float*>(v);
    MX_TRY(alloc(e, "rope.sin", sn.size() * 4, &v));
    e.rope_sin = static_cast<float*>(v);
    if (hipMemcpy(e.rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(e.rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
      return MX_EHIP;
  }

  // ---- activations for up to kPrefillChunk rows ----
  const size_t R = kPrefillChunk;
  auto a16 = [&](const char* n, size_t count, uint16_t** out) -> int {
    void* q;
    MX_TRY(alloc(e, n, count * 2, &q));
    *out = static_cast<uint16_t*>(q);
    return MX_OK;
  };
  const int inter_max = c.moe_inter > c.shared_inter ? c.moe_inter : c.shared_inter;
  MX_TRY(a16("act.h", R * c.hc * c.hidden, &e.h));
  MX_TRY(a16("act.xn", R * c.hc * c.hidden, &e.xn));
  MX_TRY(a16("act.lo", R * c.hc_rank, &e.lo));
  MX_TRY(a16("act.inj", R * c.hc, &e.inj));
  MX_TRY(a16("act.mixed", R * c.hidden, &e.mixed));
  MX_TRY(a16("act.proj", R * (e.P > e.Q ? e.P : e.Q), &e.pbuf));
  MX_TRY(a16("act.conv_out", R * e.cd, &e.conv_out));
  MX_TRY(a16("act.y", R * (e.vd > c.heads * c.head_dim ? e.vd : c.heads * c.head_dim), &e.y));
  MX_TRY(a16("act.qrot", R * c.heads * c.head_dim, &e.qrot));
  MX_TRY(a16("act.router", R * (c.experts + 1), &e.logits_r));
  MX_TRY(a16("act.scores", R * c.top_k, &e.scores));
  MX_TRY(a16("act.factor", R, &e.factor));
  MX_TRY(a16("act.moe_p", R * (c.top_k + 1) * c.hidden, &e.moe_p));
  {
    const size_t ws = moe_workspace_bytes(int(R), c.top_k, inter_max);
    MX_TRY(alloc(e, "act.moe_ws", ws, &e.moe_ws));
    e.moe_h = static_cast<uint16_t*>(e.moe_ws);
    e.moe_plan_buf = reinterpret_cast<MoePlan*>(static_cast<char*>(e.moe_ws) + ws - sizeof(MoePlan));
  }
  MX_TRY(alloc(e, "act.chunk_plan", sizeof(ChunkPlan), &v));
  e.chunk_plan = static_cast<ChunkPlan*>(v);
  e.gemm_part_floats = size_t(4) << 20;  // 16 MB: the projections' k-split partials
  MX_TRY(alloc(e, "act.gemm_part", e.gemm_part_floats * 4, &v));
  e.gemm_part = static_cast<float*>(v);
  if (e.n_gdn > 0) {
    MX_TRY(alloc(e, "act.gdn_chunk_io", gdn_chunk_io_bytes(int(R), e.gd), &e.gdn_io));
    MX_TRY(alloc(e, "act.gdn_chunk_ws", gdn_chunk_workspace_bytes(1, c.gdn_hv, int(R)), &v));
    e.gdn_ws = static_cast<float*>(v);
  }
  // bf16 logits of a decode step or verify block (at most 8 rows)
  MX_TRY(a16("act.logits", size_t(8) * c.vocab, &e.logits));
  if (c.mtp) {
    MX_TRY(a16("mtp.act.emb", R * c.hidden, &e.mtp_emb));
    MX_TRY(a16("mtp.act.a", R * c.hidden, &e.mtp_a));
    MX_TRY(a16("mtp.act.e", R * c.hidden, &e.mtp_e));
    MX_TRY(a16("mtp.act.prev", R * c.hc * c.hidden, &e.mtp_prev));
    MX_TRY(a16("mtp.act.hn", R * c.hc * c.hidden, &e.mtp_hn));
    MX_TRY(a16("mtp.act.f", R * c.hc * c.hidden, &e.mtp_f));
    MX_TRY(a16("mtp.act.dh", size_t(c.hc) * c.hidden, &e.mtp_dh));
  }
  MX_TRY(alloc(e, "act.ids", R * c.top_k * 4, &v));
  e.ids = static_cast<uint32_t*>(v);
  const size_t AR = R < size_t(kAttnRows) ? R : size_t(kAttnRows);  // attention rows per launch
  // partials per (row, head): decode chunks for AR rows, or the prefill
  // form's splits for all R rows of a chunk in one launch
  const size_t parts = std::max(AR * e.max_chunks, R * size_t(attn_prefill_splits(c.max_context)));
  MX_TRY(alloc(e, "act.o_part", parts * c.heads * c.head_dim * 4, &v));
  e.o_part = static_cast<float*>(v);
  MX_TRY(alloc(e, "act.ml_part", parts * c.heads * 2 * 4, &v));
  e.ml_part = static_cast<float*>(v);
  size_t hws = size_t(head_parts(c.vocab, c.hidden)) * 8 * 8;
  MX_TRY(alloc(e, "act.head_ws", hws, &e.head_ws));
  MX_TRY(alloc(e, "act.hc_part", hc_fused_part_bytes(c.hc_rank + c.hc), &v));
  e.hc_part = static_cast<float*>(v);
  MX_TRY(alloc(e, "act.xn_plane", xq_plane_bytes(c.hc * c.hidden), &v));
  e.xn_plane = static_cast<char*>(v);
  MX_TRY(alloc(e, "act.mixed_plane", xq_plane_bytes(c.hidden), &v));
  e.mixed_plane = static_cast<char*>(v);
  MX_TRY(alloc(e, "act.y_plane",
               xq_plane_bytes(std::max(c.gdn_hv * c.gdn_dv, c.heads * c.head_dim)), &v));
  e.y_plane = static_cast<char*>(v);
  MX_TRY(alloc(e, "rows", sizeof(Engine::RowTable), &v));
  e.dev_rows = static_cast<Engine::RowTable*>(v);
  if (hipHostMalloc(reinterpret_cast<void**>(&e.host_rows), sizeof(Engine::RowTable)) != hipSuccess)
    return MX_ENOMEM;
  std::memset(e.host_rows, 0, sizeof(Engine::RowTable));
  e.offsets.assign(c.max_slots, 0);
  e.failed.assign(c.max_slots, 0);
  if (hipStreamSynchronize(e.stream) != hipSuccess) return MX_EHIP;
  return MX_OK;
}

size_t qw_bytes(const QWeight& w) {
  return size_t(w.n) * w.k * w.bits / 8 + size_t(w.n) * (w.k / w.group_size) * 4;
}

bool experts_fast(const Engine& e, const LayerW& L) {
  const QWeight g{L.gate.codes, L.gate.scales, L.gate.biases, L.gate.n, L.gate.k, L.gate.bits,
                  L.gate.group_size};
  const QWeight d{L.down.codes, L.down.scales, L.down.biases, L.down.n, L.down.k, L.down.bits,
                  L.down.group_size};
  return !ex(e, kExMoe) && skinny_supported(g) && skinny_supported(d) && skinny_supported(L.sgate) &&
         skinny_supported(L.sdown);
}

int experts_gate_up(Engine& e, const LayerW& L, int rows) {
  const auto& c = e.cfg;
  if (experts_fast(e, L))
    return skinny_gate_up(e.mixed, e.ids, rows, c.top_k, L.gate, L.up, L.sgate, L.sup, e.moe_h,
                          e.stream);
  return xq_gate_up(e.mixed, mixed_plane(e, rows), e.moe_plan_buf, rows, c.top_k, L.gate, L.up,
                    L.sgate, L.sup, e.moe_h, e.stream);
}

int experts_down(Engine& e, const LayerW& L, int rows) {
  const auto& c = e.cfg;
  if (experts_fast(e, L))
    return skinny_down(e.moe_h, e.ids, e.scores, rows, c.top_k, L.gate.n, L.sgate.n, L.down,
                       L.sdown, e.moe_p, e.stream);
  return xq_down(e.moe_h, e.moe_plan_buf, e.scores, rows, c.top_k, L.gate.n, L.sgate.n, L.down,
                 L.sdown, e.moe_p, e.stream);
}

// Profiled (eager) steps: count the layer's distinct routed experts and time
// the gate/up and down expert kernels with events on the engine stream.
int profile_experts(Engine& e, const LayerW& L, int rows) {
  const auto& c = e.cfg;
  std::vector<uint32_t> ids(size_t(rows) * c.top_k);
  MX_HIP(hipMemcpyAsync(ids.data(), e.ids, ids.size() * 4, hipMemcpyDeviceToHost, e.stream));
  MX_HIP(hipStreamSynchronize(e.stream));
  std::vector<char> seen(c.experts, 0);
  int distinct = 0;
  for (uint32_t v : ids)
    if (v < uint32_t(c.experts) && !seen[v]) {
      seen[v] = 1;
      ++distinct;
    }
  if (!experts_fast(e, L)) MX_TRY(moe_plan(e.ids, rows, c.top_k, e.moe_plan_buf, e.stream));
  MX_HIP(hipEventRecord(e.ev[0], e.stream));
  MX_TRY(experts_gate_up(e, L, rows));
  MX_HIP(hipEventRecord(e.ev[1], e.stream));
  MX_TRY(experts_down(e, L, rows));
  MX_HIP(hipEventRecord(e.ev[2], e.stream));
  MX_HIP(hipEventSynchronize(e.ev[2]));
  float a = 0.0f, b = 0.0f;
  MX_HIP(hipEventElapsedTime(&a, e.ev[0], e.ev[1]));
  MX_HIP(hipEventElapsedTime(&b, e.ev[1], e.ev[2]));
  mx_step_profile& p = *e.prof;
  p.layers += 1;
  p.distinct_experts += distinct;
  p.gate_up_ms += a;
  p.down_ms += b;
  const QWeight g{L.gate.codes, L.gate.scales, L.gate.biases, L.gate.n, L.gate.k, L.gate.bits,
                  L.gate.group_size};
  const QWeight d{L.down.codes, L.down.scales, L.down.biases, L.down.n, L.down.k, L.down.bits,
                  L.down.group_size};
  p.gate_up_bytes += double(distinct) * 2.0 * double(qw_bytes(g)) +
                     double(qw_bytes(L.sgate) + qw_bytes(L.sup));
  p.down_bytes += double(distinct) * double(qw_bytes(d)) + double(qw_bytes(L.sdown));
  e.prof_routed += double(distinct) * (2.0 * double(qw_bytes(g)) + double(qw_bytes(d)));
  return MX_OK;
}

// Projection on the matrix cores (fast mode) or the exact kernels.
// Exact components take the exact-integer projection (bit for bit the CPU
// oracle's); a weight it does not cover is an error, never another path.
int project(Engine& e, const QWeight& w, const uint16_t* x, int64_t xs, int rows,
            const ProjEpilogue& ep, int part, const char* plane = nullptr) {
  if (ex(e, part)) return xq_dense(w, x, xs, rows, ep, e.stream, plane);
  if (rows <= 8 && skinny_supported(w)) return skinny_dense(w, x, xs, rows, ep, e.stream);
  if (qmm_supported(w)) {
    ProjEpilogue ek = ep;  // prefill rows may split k across workgroups
    ek.part = e.gemm_part;
    ek.part_floats = e.gemm_part_floats;
    return qmm(w, x, xs, rows, ek, e.stream);
  }
  return xq_dense(w, x, xs, rows, ep, e.stream);
}

int hc_forward(Engine& e, const HcW& w, int rows, uint16_t* mixed_out, uint16_t* inj_out) {
  const auto& c = e.cfg;
  if (!ex(e, kExHc) && rows <= 8 && hc_fused_supported(w.down, w.up, c.hc, c.hidden, c.hc_rank))
    return hc_fused(w.down, w.up, e.h, w.scale, rows, c.hc, c.hidden, c.hc_rank, c.rms_eps,
                    e.hc_part, mixed_out, inj_out, e.stream);
  // exact: the norm writes the down projection's operand plane, and the
  // up-projection + mix writes the plane of `mixed` for its consumers
  const bool exact = ex(e, kExHc) && rows <= 8;
  if (e.xn_ready)
    e.xn_ready = false;  // the slot sum before normed the streams with this scale
  else
    MX_TRY(hc_norm(e.h, w.scale, rows, c.hc, c.hidden, c.rms_eps, e.xn, e.stream,
                   exact ? e.xn_plane : nullptr));
  ProjEpilogue d{};
  d.mode = kHcDown;
  d.y = e.lo;
  d.y_stride = c.hc_rank;
  d.aux = inj_out;
  d.aux_stride = c.hc;
  d.rank = c.hc_rank;
  d.hc = c.hc;
  MX_TRY(project(e, w.down, e.xn, int64_t(c.hc) * c.hidden, rows, d, kExHc,
                 exact ? e.xn_plane : nullptr));
  if (exact && mixed_out == e.mixed)
    return xq_upmix(w.up, e.lo, rows, e.xn, c.hidden, mixed_out, e.mixed_plane, e.stream);
  ProjEpilogue u{};
  u.mode = kHcUpMix;
  u.y = mixed_out;
  u.y_stride = c.hidden;
  u.xn = e.xn;
  u.xn_stride = int64_t(c.hc) * c.hidden;
  u.hc = c.hc;
  u.hidden = c.hidden;
  MX_TRY(project(e, w.up, e.lo, c.hc_rank, rows, u, kExHc));
  return MX_OK;
}

// Records the kernels of one step for `rows` rows arranged as `groups`
// sequences of `t` tokens.  Row metadata is read from e.dev_rows.
// Records one layer (attention or GDN sublayer, then the MoE sublayer) on the
// hc streams e.h of `rows` rows arranged as `groups` sequences of `t` tokens.
// next_scale (nullable): the norm scale of the hyper-connection that follows
// the layer, which the exact slot sum then applies in the same launch.
int record_layer(Engine& e, const LayerW& L, int rows, int groups, int t, bool history,
                 const uint16_t* next_scale = nullptr) {
  const auto& c = e.cfg;
  Engine::RowTable* rt = e.dev_rows;
  {
    MX_TRY(hc_forward(e, L.attn_hc, rows, e.mixed, e.inj));
    ProjEpilogue wr{};
    wr.mode = kHcWrite;
    wr.y = e.h;
    wr.y_stride = int64_t(c.hc) * c.hidden;
    wr.aux = e.inj;
    wr.aux_stride = c.hc;
    wr.hc = c.hc;
    if (!L.attn) {
      const int gi = L.cache_index;
      ProjEpilogue pl{};
      pl.mode = kPlain;
      pl.y = e.pbuf;
      pl.y_stride = e.P;
      const size_t conv_per = size_t(c.conv_k - 1) * e.cd;
      const size_t state_per = size_t(c.gdn_hv) * c.gdn_dk * c.gdn_dv;
      // cache layout [slot][gdn layer]: slot index s -> s * n_gdn + gi
      const bool exact_in = ex(e, kExGdnProj);
      if (t == 1 && !history && rows <= 8 && L.gdn_in.bits == 4 && c.conv_k <= kConvMaxTaps &&
          (exact_in ? xq_supported(L.gdn_in) : skinny_supported(L.gdn_in))) {
        // the conv runs in the projection's epilogue
        pl.mode = kConv;
        pl.conv_state = e.conv_state + gi * conv_per;
        pl.conv_w = L.conv_w;
        pl.slots = rt->gdn_slots;
        pl.conv_out = e.conv_out;
        pl.conv_stride = e.cd;
        pl.conv_ch = int(e.cd);
        pl.taps = c.conv_k;
        if (exact_in)
          MX_TRY(xq_dense(L.gdn_in, e.mixed, c.hidden, rows, pl, e.stream, mixed_plane(e, rows)));
        else
          MX_TRY(skinny_dense(L.gdn_in, e.mixed, c.hidden, rows, pl, e.stream));
      } else {
        MX_TRY(project(e, L.gdn_in, e.mixed, c.hidden, rows, pl, kExGdnProj, mixed_plane(e, rows)));
        MX_TRY(gdn_conv(e.pbuf, e.P, groups, t, rt->gdn_slots, e.conv_state + gi * conv_per,
                        L.conv_w, e.cd, c.conv_k, e.conv_out, e.cd,
                        history ? e.hist_conv + size_t(gi) * (c.conv_k - 1 + c.max_verify) * e.cd
                                : nullptr,
                        e.stream));
      }
      float* hist = history ? e.hist_state + size_t(gi) * c.max_verify * state_per : nullptr;
      if (!ex(e, kExGdn) && rows > 8) {
        // a prefill chunk: the chunked scan (64-token chunks on the matrix
        // cores) in place of the token-by-token step
        MX_TRY(gdn_chunk_fast(e.conv_out, e.cd, e.pbuf + e.cd, e.pbuf + e.cd + e.vd,
                              e.pbuf + e.cd + e.vd + c.gdn_hv, e.P, L.a_log, L.dt_bias,
                              L.gdn_norm, c.rms_eps, e.gd, groups, t, rt->gdn_slots,
                              e.gdn_state + gi * state_per, e.y, e.gdn_io, e.gdn_ws, e.stream));
      } else if (!ex(e, kExGdn)) {
        // decode, verify and prefill blocks alike: a verify block's tokens
        // get the bits of one-token decode steps (lossless speculation)
        MX_TRY(gdn_recurrence_fast(e.conv_out, e.cd, e.pbuf + e.cd, e.pbuf + e.cd + e.vd,
                                   e.pbuf + e.cd + e.vd + c.gdn_hv, e.P, L.a_log, L.dt_bias,
                                   L.gdn_norm, c.rms_eps, e.gd, groups, t, rt->gdn_slots,
                                   e.gdn_state + gi * state_per, hist, e.y, e.stream));
      }
      // exact recurrence + exact projection: the recurrence writes the
      // projection's operand plane
      char* yp = ex(e, kExGdn) && ex(e, kExGdnProj) && rows <= 8 ? e.y_plane : nullptr;
      if (ex(e, kExGdn))
        MX_TRY(gdn_recurrence(e.conv_out, e.cd, e.pbuf + e.cd, e.pbuf + e.cd + e.vd,
                              e.pbuf + e.cd + e.vd + c.gdn_hv, e.P, L.a_log, L.dt_bias,
                              L.gdn_norm, c.rms_eps, e.gd, groups, t, rt->gdn_slots,
                              e.gdn_state + gi * state_per, hist, e.y, e.stream, yp));
      MX_TRY(project(e, L.gdn_out, e.y, e.vd, rows, wr, kExGdnProj, yp));
    } else {
      const int ai = L.cache_index;
      ProjEpilogue pl{};
      pl.mode = kPlain;
      pl.y = e.pbuf;
      pl.y_stride = e.Q;
      MX_TRY(project(e, L.attn_in, e.mixed, c.hidden, rows, pl, kExAttnProj, mixed_plane(e, rows)));
      const size_t layer_off = size_t(ai) * c.kv_heads * c.max_context * c.head_dim;
      MX_TRY(attn_prep(e.pbuf, e.Q, rows, rt->slots, rt->pos, L.q_norm, L.k_norm, c.rms_eps,
                       e.rope_cos, e.rope_sin, e.ad, e.qrot, e.k_cache + layer_off,
                       e.v_cache + layer_off, e.stream));
      const bool fast_attn = !ex(e, kExAttn) && attn_fast_supported(e.ad);
      char* yp = !fast_attn && ex(e, kExAttnProj) && rows <= 8 ? e.y_plane : nullptr;
      const size_t qd = size_t(c.heads) * c.head_dim;
      // more than 8 rows in fast mode: the rows of one slot's chunk in one
      // launch, their query blocks sharing each key tile; otherwise rows go
      // through in blocks of kAttnRows, so the per-chunk partials stay sized
      // for kAttnRows rows
      const bool prefill = rows > 8 && fast_attn && attn_prefill_supported(e.ad);
      if (prefill) {
        const int splits = attn_prefill_splits(c.max_context);
        MX_TRY(attn_prefill(e.qrot, rows, rt->slots, rt->pos, e.k_cache + layer_off,
                            e.v_cache + layer_off, e.ad, splits, e.o_part, e.ml_part, e.stream));
        MX_TRY(attn_combine_splits(e.o_part, e.ml_part, e.pbuf, e.Q, rows, rt->pos, e.ad, splits,
                                   e.y, e.stream));
      }
      for (int r0 = 0; r0 < rows && !prefill; r0 += kAttnRows) {
        const int n = rows - r0 < kAttnRows ? rows - r0 : kAttnRows;
        MX_TRY(attn_decode(e.qrot + r0 * qd, n, rt->slots + r0, rt->pos + r0,
                           e.k_cache + layer_off, e.v_cache + layer_off, e.ad, e.max_chunks,
                           fast_attn, e.o_part, e.ml_part, e.stream));
        MX_TRY(attn_combine(e.o_part, e.ml_part, e.pbuf + size_t(r0) * e.Q, e.Q, n,
                            rt->pos + r0, e.ad, e.max_chunks, fast_attn, e.y + r0 * qd,
                            e.stream, yp));
      }
      MX_TRY(project(e, L.attn_out, e.y, int64_t(c.heads) * c.head_dim, rows, wr, kExAttnProj,
                     yp));
    }
    // MoE sublayer
    MX_TRY(hc_forward(e, L.mlp_hc, rows, e.mixed, e.inj));
    ProjEpilogue rl{};
    rl.mode = kPlain;
    rl.y = e.logits_r;
    rl.y_stride = c.experts + 1;
    MX_TRY(project(e, L.router, e.mixed, c.hidden, rows, rl, kExMoe, mixed_plane(e, rows)));
    bool summed = false;  // slots summed and the streams written
    if (rows > 8) {
      // a prefill chunk: the routes grouped by expert, on the matrix cores
      MX_TRY(moe_route(e.logits_r, c.experts + 1, e.logits_r + c.experts, c.experts + 1, rows,
                       c.experts, c.top_k, e.ids, e.scores, e.factor, e.stream));
      MX_TRY(chunk_plan(e.ids, rows, c.experts, c.top_k, e.chunk_plan, e.stream));
      MX_TRY(qmm_chunk_gate_up(e.mixed, e.chunk_plan, rows, c.experts, c.top_k, L.gate, L.up,
                               L.sgate, L.sup, e.moe_h, e.stream));
      MX_TRY(qmm_chunk_down(e.moe_h, e.chunk_plan, e.scores, rows, c.experts, c.top_k, L.gate.n,
                            L.sgate.n, L.down, L.sdown, e.moe_p, e.stream));
    } else if (!e.prof && experts_fast(e, L)) {
      // the expert gate/up kernel routes the rows itself
      const RouteIO ro{e.logits_r, c.experts + 1, e.logits_r + c.experts, c.experts + 1,
                       e.ids, e.scores, e.factor};
      MX_TRY(skinny_route_gate_up(ro, c.experts, e.mixed, rows, c.top_k, L.gate, L.up, L.sgate,
                                  L.sup, e.moe_h, e.stream));
      // 512-deep experts: the down kernel sums the slots and writes the
      // residual streams itself
      if (skinny_down_hc_supported(rows, c.top_k, c.hc, L.down, L.sdown)) {
        MX_TRY(skinny_down_hc(e.moe_h, e.ids, e.scores, e.factor, e.inj, rows, c.top_k, c.hc,
                              L.gate.n, L.sgate.n, L.down, L.sdown, e.h, e.stream));
        summed = true;
      } else {
        MX_TRY(experts_down(e, L, rows));
      }
    } else {
      if (e.prof) {
        MX_TRY(moe_route(e.logits_r, c.experts + 1, e.logits_r + c.experts, c.experts + 1, rows,
                         c.experts, c.top_k, e.ids, e.scores, e.factor, e.stream));
        MX_TRY(profile_experts(e, L, rows));
      } else {
        MX_TRY(moe_route_plan(e.logits_r, c.experts + 1, e.logits_r + c.experts, c.experts + 1,
                              rows, c.experts, c.top_k, e.ids, e.scores, e.factor,
                              e.moe_plan_buf, e.stream));
        MX_TRY(experts_gate_up(e, L, rows));
        MX_TRY(experts_down(e, L, rows));
      }
    }
    if (!summed) {
      if (next_scale && ex(e, kExHc) && moe_reduce_norm_supported(rows, c.top_k, c.hc, c.hidden)) {
        MX_TRY(moe_reduce_norm(e.moe_p, e.factor, e.h, e.inj, rows, c.top_k, c.hc, c.hidden,
                               next_scale, c.rms_eps, e.xn, e.xn_plane, e.stream));
        e.xn_ready = true;
      } else {
        MX_TRY(moe_reduce_hc_epilogue(e.moe_p, e.factor, e.h, e.inj, rows, c.top_k, c.hc,
                                      c.hidden, e.h, e.stream));
      }
    }
  }
  return MX_OK;
}

// Greedy head over rows first_row .. first_row + rows - 1 of e.mixed: next
// tokens into the device row table (from entry 0); with `logits`, the bf16
// logits too.
int record_head(Engine& e, int rows, bool logits, int first_row = 0);

int record_step(Engine& e, int rows, int groups, int t, bool history, bool logits) {
  const auto& c = e.cfg;
  Engine::RowTable* rt = e.dev_rows;
  MX_TRY(embed(e.embed, rt->tokens, rows, c.hc, e.h, e.stream));
  int launched = 0;
  e.xn_ready = false;
  for (size_t i = 0; i < e.layers.size(); ++i) {
    const LayerW& L = e.layers[i];
    const uint16_t* next = i + 1 < e.layers.size() ? e.layers[i + 1].attn_hc.scale : e.mixer.scale;
    MX_TRY(record_layer(e, L, rows, groups, t, history, next));
    if (e.fail_after > 0 && ++launched == e.fail_after) {
      // the injected failure: the launched layers run, then the step stops
      // as a failed launch would
      // (under graph capture nothing has run yet: the capture is dropped)
      e.fail_after = 0;
      if (!e.use_graphs) (void)hipStreamSynchronize(e.stream);
      return MX_EHIP;
    }
  }
  // mixer + greedy head
  MX_TRY(hc_forward(e, e.mixer, rows, e.mixed, nullptr));
  return record_head(e, rows, logits);
}

int record_head(Engine& e, int rows, bool logits, int first_row) {
  const auto& c = e.cfg;
  Engine::RowTable* rt = e.dev_rows;
  const uint16_t* x = e.mixed + size_t(first_row) * c.hidden;
  int parts = 0;
  float* maxima = static_cast<float*>(e.head_ws);
  uint32_t* indices = reinterpret_cast<uint32_t*>(maxima + size_t(head_parts(c.vocab, c.hidden)) * 8);
  // either head writes the bf16 logits it ranks when they are wanted; heads
  // the matrix-core kernel does not cover take the exact-integer one
  if (!ex(e, kExHead) && skinny_supported(e.head) && e.head.k % 512 == 0 && e.head.k <= 2048)
    MX_TRY(skinny_head(e.head, x, rows, maxima, indices, &parts, e.stream,
                       logits ? e.logits : nullptr));
  else
    MX_TRY(xq_head(e.head, x, first_row == 0 ? mixed_plane(e, rows) : nullptr, rows, maxima,
                   indices, logits ? e.logits : nullptr, &parts, e.stream));
  return argmax_reduce(maxima, indices, rows, parts, rt->next, e.stream);
}

int graph_key(int rows, int groups, int t, bool history, bool logits) {
  return ((rows * 16 + groups) * 16 + t) * 4 + (history ? 2 : 0) + (logits ? 1 : 0);
}

// Runs one step: copies the row table in, replays (or captures) the graph and
// reads back the next tokens.  Synchronises once, like the reference's eval.
int run_step(Engine& e, int rows, int groups, int t, bool history, uint32_t* next) {
  if (hipMemcpyAsync(e.dev_rows, e.host_rows, sizeof(Engine::RowTable), hipMemcpyHostToDevice,
                     e.stream) != hipSuccess)
    return MX_EHIP;
  const int key = graph_key(rows, groups, t, history, e.want_logits);
  if (e.use_graphs) {
    auto it = e.graphs.find(key);
    if (it == e.graphs.end()) {
      hipGraph_t g = nullptr;
      MX_HIP(hipStreamBeginCapture(e.stream, hipStreamCaptureModeThreadLocal));
      const int rc = record_step(e, rows, groups, t, history, e.want_logits);
      hipGraph_t captured = nullptr;
      const hipError_t end = hipStreamEndCapture(e.stream, &captured);
      if (rc != MX_OK) {
        if (captured) hipGraphDestroy(captured);
        return rc;
      }
      MX_HIP(end);
      g = captured;
      hipGraphExec_t exec = nullptr;
      const hipError_t inst = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
      hipGraphDestroy(g);
      MX_HIP(inst);
      it = e.graphs.emplace(key, exec).first;
    }
    MX_HIP(hipGraphLaunch(it->second, e.stream));
  } else {
    MX_TRY(record_step(e, rows, groups, t, history, e.want_logits));
  }
  MX_HIP(hipMemcpyAsync(e.host_rows->next, e.dev_rows->next, sizeof(uint32_t) * rows,
                        hipMemcpyDeviceToHost, e.stream));
  MX_HIP(hipStreamSynchronize(e.stream));
  if (next) std::memcpy(next, e.host_rows->next, sizeof(uint32_t) * rows);
  e.last_rows = rows;
  return MX_OK;
}

// MTP forward (Mtp::forward, src/mtp.rs:72-127) over `rows` rows of one slot:
// the token ids (the token after each MTP position) and positions come from
// the row table, the previous hidden streams from e.mtp_prev; the draft
// tokens go to the row table's `next` and the new hidden streams stay in e.h.
//   e = fc_embedding(norm(embedding, pre_fc_norm_embedding))
//   h = fc_hidden(norm(previous hidden over all hc streams)) per stream
//   h = bf16(e + h) -> attention layer + MoE layer -> mixer -> greedy head
// Both norms are compiled::norm (src/compiled.rs:22-28), run by the
// hyper-connection norm kernel with one stream of H or hc * H values.
int record_mtp(Engine& e, int rows) {
  const auto& c = e.cfg;
  Engine::RowTable* rt = e.dev_rows;
  const int H = c.hidden, hc = c.hc;
  MX_TRY(embed(e.embed, rt->tokens, rows, 1, e.mtp_emb, e.stream));
  MX_TRY(hc_norm(e.mtp_emb, e.mtp.norm_emb, rows, 1, H, c.rms_eps, e.mtp_a, e.stream));
  ProjEpilogue pe{};
  pe.mode = kPlain;
  pe.y = e.mtp_e;
  pe.y_stride = H;
  MX_TRY(project(e, e.mtp.fc_emb, e.mtp_a, H, rows, pe, kExAttnProj));
  MX_TRY(hc_norm(e.mtp_prev, e.mtp.norm_hid, rows, 1, hc * H, c.rms_eps, e.mtp_hn, e.stream));
  const int piece = e.chunk ? kQmmMaxRows : 8;  // stream rows per projection
  for (int r0 = 0; r0 < rows * hc; r0 += piece) {
    const int n = rows * hc - r0 < piece ? rows * hc - r0 : piece;
    ProjEpilogue ph{};
    ph.mode = kPlain;
    ph.y = e.mtp_f + size_t(r0) * H;
    ph.y_stride = H;
    MX_TRY(project(e, e.mtp.fc_hid, e.mtp_hn + size_t(r0) * H, H, n, ph, kExAttnProj));
  }
  MX_TRY(mtp_combine(e.mtp_e, e.mtp_f, rows, hc, H, e.h, e.stream));
  e.xn_ready = false;
  MX_TRY(record_layer(e, e.mtp.layer, rows, 1, rows, false, e.mtp.mixer.scale));
  MX_TRY(hc_forward(e, e.mtp.mixer, rows, e.mixed, nullptr));
  // a prompt chunk's pass needs only its last row's draft (into entry 0)
  return rows > 8 ? record_head(e, 1, false, rows - 1) : record_head(e, rows, false);
}

// One eager MTP pass over `rows` rows of `slot` at MTP positions pos0 + r.
// chunk: a prompt chunk's pass on the matrix-core kernels (rows up to
// kPrefillChunk); beyond eight rows only next[rows - 1] is written.
int mtp_step(Engine& e, int slot, const uint32_t* tokens, int rows, int pos0, uint32_t* next,
             bool chunk = false) {
  for (int r = 0; r < rows; ++r) {
    e.host_rows->tokens[r] = tokens[r];
    e.host_rows->slots[r] = slot;
    e.host_rows->pos[r] = pos0 + r;
    e.host_rows->gdn_slots[r] = slot * e.n_gdn;
  }
  MX_HIP(hipMemcpyAsync(e.dev_rows, e.host_rows, sizeof(Engine::RowTable), hipMemcpyHostToDevice,
                        e.stream));
  e.chunk = chunk;
  const int rc = record_mtp(e, rows);
  e.chunk = false;
  MX_TRY(rc);
  const int got = rows > 8 ? 1 : rows;
  MX_HIP(hipMemcpyAsync(e.host_rows->next, e.dev_rows->next, sizeof(uint32_t) * got,
                        hipMemcpyDeviceToHost, e.stream));
  MX_HIP(hipStreamSynchronize(e.stream));
  if (rows > 8)
    next[rows - 1] = e.host_rows->next[0];
  else
    std::memcpy(next, e.host_rows->next, sizeof(uint32_t) * rows);
  return MX_OK;
}

size_t state_per(const Engine& e) {
  return size_t(e.cfg.gdn_hv) * e.cfg.gdn_dk * e.cfg.gdn_dv;
}
size_t conv_per(const Engine& e) { return size_t(e.cfg.conv_k - 1) * e.cd; }

}  // namespace

// ---- engine operations used by the C ABI --------------------------------
int engine_create(const mx_model_config& cfg, Engine** out) {
  auto e = std::make_unique<Engine>();
  e->cfg = cfg;
  MX_HIP(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking));
  MX_TRY(build(*e));
  // caches start empty (zero state, zero conv window)
  for (int s = 0; s < cfg.max_slots; ++s) MX_TRY(engine_reset_slot(*e, s));
  MX_HIP(hipStreamSynchronize(e->stream));
  *out = e.release();
  return MX_OK;
}

void engine_destroy(Engine* e) { delete e; }

int engine_reset_slot(Engine& e, int slot) {
  const size_t sp = state_per(e), cp = conv_per(e);
  MX_HIP(hipMemsetAsync(e.gdn_state + size_t(slot) * e.n_gdn * sp, 0, e.n_gdn * sp * 4, e.stream));
  MX_HIP(hipMemsetAsync(e.conv_state + size_t(slot) * e.n_gdn * cp, 0, e.n_gdn * cp * 2, e.stream));
  MX_HIP(hipStreamSynchronize(e.stream));
  e.offsets[slot] = 0;
  e.failed[slot] = 0;
  if (e.verify_slot == slot) e.verify_slot = -1;
  return MX_OK;
}

int engine_clone_slot(Engine& e, int src, int dst) {
  if (e.failed[src]) return MX_ESTATE;  // nothing intact to copy
  const size_t sp = state_per(e), cp = conv_per(e);
  const int64_t kv = e.ad.slot_stride;
  MX_HIP(hipMemcpyAsync(e.gdn_state + size_t(dst) * e.n_gdn * sp,
                        e.gdn_state + size_t(src) * e.n_gdn * sp, e.n_gdn * sp * 4,
                        hipMemcpyDeviceToDevice, e.stream));
  MX_HIP(hipMemcpyAsync(e.conv_state + size_t(dst) * e.n_gdn * cp,
                        e.conv_state + size_t(src) * e.n_gdn * cp, e.n_gdn * cp * 2,
                        hipMemcpyDeviceToDevice, e.stream));
  // only the filled positions of each (layer, kv head) need copying
  const int used = e.offsets[src];
  if (used > 0) {
    const size_t row_bytes = size_t(used) * e.cfg.head_dim * 2;
    const size_t pitch = size_t(e.cfg.max_context) * e.cfg.head_dim * 2;
    const size_t planes = size_t(e.n_attn) * e.cfg.kv_heads;
    for (uint16_t* cache : {e.k_cache, e.v_cache})
      MX_HIP(hipMemcpy2DAsync(cache + size_t(dst) * kv, pitch, cache + size_t(src) * kv, pitch,
                              row_bytes, planes, hipMemcpyDeviceToDevice, e.stream));
  }
  MX_HIP(hipStreamSynchronize(e.stream));
  e.offsets[dst] = e.offsets[src];
  e.failed[dst] = 0;
  // the copy replaces the caches a pending verify block of dst would roll back
  if (dst == e.verify_slot) e.verify_slot = -1;
  return MX_OK;
}

int engine_offset(const Engine& e, int slot) { return e.offsets[slot]; }

// A step that fails after its first launch leaves the GDN state and conv
// windows of its slots partly advanced (they are updated in place; the
// reference's lazy evaluation never writes a cache before the whole step has
// succeeded, src/batching.rs:136-137).  Those slots are marked failed and
// refused until reset_slot or clone_slot replaces their caches, so no later
// step reads them as if they were intact; their offsets do not advance.
int step_failed(Engine& e, const int32_t* slots, int n, int rc, std::string* err) {
  for (int r = 0; r < n; ++r) e.failed[slots[r]] = 1;
  for (int r = 0; r < n; ++r)
    if (slots[r] == e.verify_slot) e.verify_slot = -1;
  if (err->empty())
    *err = "the step failed after updating its slots' caches in place; reset or clone over "
           "those slots before using them again";
  return rc;
}

int slots_usable(const Engine& e, const int32_t* slots, int n, std::string* err) {
  for (int r = 0; r < n; ++r)
    if (e.failed[slots[r]]) {
      *err = "slot " + std::to_string(slots[r]) +
             " was left partly updated by a failed step; reset it or clone a prefix into it";
      return MX_ESTATE;
    }
  return MX_OK;
}

int engine_slot_failed(const Engine& e, int slot) { return e.failed[slot]; }
void engine_inject_failure(Engine& e, int after_layers) { e.fail_after = after_layers; }

int engine_decode_rows(Engine& e, const int32_t* slots, const uint32_t* tokens, int rows,
                       uint32_t* next, std::string* err) {
  MX_TRY(slots_usable(e, slots, rows, err));
  for (int r = 0; r < rows; ++r) {
    for (int q = 0; q < r; ++q)
      if (slots[q] == slots[r]) {
        *err = "a slot appears twice in one step";
        return MX_EINVAL;
      }
    if (e.offsets[slots[r]] >= e.cfg.max_context) {
      *err = "slot context is full";
      return MX_ESTATE;
    }
    e.host_rows->tokens[r] = tokens[r];
    e.host_rows->slots[r] = slots[r];
    e.host_rows->gdn_slots[r] = slots[r] * e.n_gdn;
    e.host_rows->pos[r] = e.offsets[slots[r]];
  }
  const int rc = run_step(e, rows, rows, 1, false, next);
  if (rc != MX_OK) return step_failed(e, slots, rows, rc, err);
  for (int r = 0; r < rows; ++r) e.offsets[slots[r]] += 1;
  // a decode step invalidates any pending verify block of these slots
  for (int r = 0; r < rows; ++r)
    if (slots[r] == e.verify_slot) e.verify_slot = -1;
  return MX_OK;
}

// decode_rows, then the step's logits (bf16 [rows, vocab]) and final hidden
// streams (bf16 [rows, hc * hidden]) into caller device buffers (either may be
// null), as HybridModel::decode_batch returns them (src/batching.rs:34-170).
int engine_decode_outputs(Engine& e, const int32_t* slots, const uint32_t* tokens, int rows,
                          uint32_t* next, uint16_t* logits, uint16_t* hidden, std::string* err) {
  const auto& c = e.cfg;
  const bool saved = e.want_logits;
  e.want_logits = saved || logits != nullptr;
  const int rc = engine_decode_rows(e, slots, tokens, rows, next, err);
  e.want_logits = saved;
  MX_TRY(rc);
  if (logits)
    MX_HIP(hipMemcpyAsync(logits, e.logits, size_t(rows) * c.vocab * 2, hipMemcpyDeviceToDevice,
                          e.stream));
  if (hidden)
    MX_HIP(hipMemcpyAsync(hidden, e.h, size_t(rows) * c.hc * c.hidden * 2,
                          hipMemcpyDeviceToDevice, e.stream));
  MX_HIP(hipStreamSynchronize(e.stream));
  return MX_OK;
}

// Teacher-forced decode step (a test hook): each layer i runs eagerly on the
// given input streams h_in[i] (host bf16 [layers + 1][rows][hc * hidden])
// instead of the previous layer's output; its output streams go to h_out[i]
// and its routing to ids_out[i] ([layers][rows][top_k]); the mixer and head
// run on h_in[layers].  Caches are updated and offsets advance as in a step.
int engine_decode_forced(Engine& e, const int32_t* slots, const uint32_t* tokens, int rows,
                         const uint16_t* h_in, uint16_t* h_out, uint32_t* ids_out,
                         uint32_t* next, std::string* err) {
  const auto& c = e.cfg;
  MX_TRY(slots_usable(e, slots, rows, err));
  for (int r = 0; r < rows; ++r) {
    for (int q = 0; q < r; ++q)
      if (slots[q] == slots[r]) {
        *err = "a slot appears twice in one step";
        return MX_EINVAL;
      }
    if (e.offsets[slots[r]] >= c.max_context) {
      *err = "slot context is full";
      return MX_ESTATE;
    }
    e.host_rows->tokens[r] = tokens[r];
    e.host_rows->slots[r] = slots[r];
    e.host_rows->gdn_slots[r] = slots[r] * e.n_gdn;
    e.host_rows->pos[r] = e.offsets[slots[r]];
  }
  const size_t HS = size_t(rows) * c.hc * c.hidden;
  MX_HIP(hipMemcpyAsync(e.dev_rows, e.host_rows, sizeof(Engine::RowTable), hipMemcpyHostToDevice,
                        e.stream));
  e.xn_ready = false;
  for (size_t i = 0; i < e.layers.size(); ++i) {
    MX_HIP(hipMemcpyAsync(e.h, h_in + i * HS, HS * 2, hipMemcpyHostToDevice, e.stream));
    MX_TRY(record_layer(e, e.layers[i], rows, rows, 1, false));
    MX_HIP(hipMemcpyAsync(h_out + i * HS, e.h, HS * 2, hipMemcpyDeviceToHost, e.stream));
    MX_HIP(hipMemcpyAsync(ids_out + i * size_t(rows) * c.top_k, e.ids,
                          size_t(rows) * c.top_k * 4, hipMemcpyDeviceToHost, e.stream));
    MX_HIP(hipStreamSynchronize(e.stream));
  }
  MX_HIP(hipMemcpyAsync(e.h, h_in + e.layers.size() * HS, HS * 2, hipMemcpyHostToDevice,
                        e.stream));
  MX_TRY(hc_forward(e, e.mixer, rows, e.mixed, nullptr));
  MX_TRY(record_head(e, rows, e.want_logits));
  MX_HIP(hipMemcpyAsync(e.host_rows->next, e.dev_rows->next, sizeof(uint32_t) * rows,
                        hipMemcpyDeviceToHost, e.stream));
  MX_HIP(hipStreamSynchronize(e.stream));
  std::memcpy(next, e.host_rows->next, sizeof(uint32_t) * rows);
  e.last_rows = rows;
  for (int r = 0; r < rows; ++r) {
    e.offsets[slots[r]] += 1;
    if (slots[r] == e.verify_slot) e.verify_slot = -1;
  }
  return MX_OK;
}

// One chunk of up to 8 consecutive tokens of one slot (prefill or verify).
int engine_block(Engine& e, int slot, const uint32_t* tokens, int count, bool history,
                 uint32_t* next, std::string* err) {
  MX_TRY(slots_usable(e, &slot, 1, err));
  if (e.offsets[slot] + count > e.cfg.max_context) {
    *err = "slot context is full";
    return MX_ESTATE;
  }
  for (int r = 0; r < count; ++r) {
    e.host_rows->tokens[r] = tokens[r];
    e.host_rows->slots[r] = slot;
    e.host_rows->pos[r] = e.offsets[slot] + r;
  }
  e.host_rows->gdn_slots[0] = slot * e.n_gdn;
  // a prefill block (no history) moves the caches past any pending verify
  // block of this slot, whose snapshot and history no longer apply
  if (!history && slot == e.verify_slot) e.verify_slot = -1;
  const int rc = run_step(e, count, 1, count, history, next);
  if (rc != MX_OK) return step_failed(e, &slot, 1, rc, err);
  e.offsets[slot] += count;
  return MX_OK;
}

// One prefill chunk of `rows` consecutive tokens of one slot (rows from the
// row table): every layer on the matrix-core kernels with `rows` activation
// rows (a GDN layer scans the chunk's tokens in order), then the greedy head
// on the chunk's last row only (its next token lands in entry 0 of `next`).
static int record_chunk(Engine& e, int rows) {
  const auto& c = e.cfg;
  MX_TRY(embed(e.embed, e.dev_rows->tokens, rows, c.hc, e.h, e.stream));
  e.xn_ready = false;
  for (const LayerW& L : e.layers) MX_TRY(record_layer(e, L, rows, 1, rows, false));
  MX_TRY(hc_forward(e, e.mixer, rows, e.mixed, nullptr));
  return record_head(e, 1, false, rows - 1);
}

// Whether every layer of the model has a matrix-core kernel for a prefill
// chunk (checked before any launch, so an unsupported model is refused
// without touching a slot): projections and expert banks of group size 64
// and depth <= 8192, at most 1023 experts with a routing width the routing
// kernel covers, top-k <= 16, 128-wide GDN heads and a conv of <= 8 taps.
static bool chunk_supported(const Engine& e, std::string* err) {
  const auto& c = e.cfg;
  auto bank = [](const QBank& b) {
    return qmm_supported(QWeight{b.codes, b.scales, b.biases, b.n, b.k, b.bits, b.group_size});
  };
  const int per = c.experts / 64;
  bool ok = c.experts <= kChunkMaxExperts && c.experts % 64 == 0 &&
            (per == 1 || per == 2 || per == 4 || per == 8 || per == 16) && c.top_k <= 16 &&
            c.gdn_dk == 128 && c.gdn_dv == 128 && c.conv_k >= 2 && c.conv_k <= 8 &&
            qmm_supported(e.mixer.down) && qmm_supported(e.mixer.up);
  auto layer_ok = [&](const LayerW& L) {
    bool r = qmm_supported(L.attn_hc.down) && qmm_supported(L.attn_hc.up) &&
             qmm_supported(L.mlp_hc.down) && qmm_supported(L.mlp_hc.up) &&
             qmm_supported(L.router) && bank(L.gate) && bank(L.up) && bank(L.down) &&
             qmm_supported(L.sgate) && qmm_supported(L.sup) && qmm_supported(L.sdown);
    return r && (L.attn ? qmm_supported(L.attn_in) && qmm_supported(L.attn_out)
                        : qmm_supported(L.gdn_in) && qmm_supported(L.gdn_out));
  };
  for (const LayerW& L : e.layers) ok = ok && layer_ok(L);
  if (e.has_mtp)
    ok = ok && layer_ok(e.mtp.layer) && qmm_supported(e.mtp.fc_emb) &&
         qmm_supported(e.mtp.fc_hid) && qmm_supported(e.mtp.mixer.down) &&
         qmm_supported(e.mtp.mixer.up);
  if (!ok)
    *err = "the model has no matrix-core prefill kernel for some layer (group size 64, depth "
           "<= 8192, <= 1023 experts in 64..1024 steps of powers of two, top-k <= 16, 128-wide "
           "GDN heads needed); use mx_engine_prefill";
  return ok;
}

// Prefill in chunks of up to kPrefillChunk tokens (speculative::prepare,
// src/speculative.rs:38-68, which runs the model's forward over each chunk):
// the projections and experts of a whole chunk on the matrix cores (expert
// weights read once per 16 of an expert's routes in the chunk instead of once
// per eight tokens), the GDN layers through the chunked scan.  The chunk's
// arithmetic is the matrix-core kernels' (fp32 sums in hardware order), so the
// caches agree with a block-by-block exact prefill to those kernels'
// tolerance, not bit for bit.  Eager launches (no graph).
int engine_prefill_chunked(Engine& e, int slot, const uint32_t* tokens, int count,
                           uint32_t* next, std::string* err) {
  MX_TRY(slots_usable(e, &slot, 1, err));
  if (int64_t(e.offsets[slot]) + count > e.cfg.max_context) {
    *err = "slot context is full";
    return MX_ESTATE;
  }
  if (!chunk_supported(e, err)) return MX_EUNSUPPORTED;
  if (slot == e.verify_slot) e.verify_slot = -1;
  for (int a = 0; a < count; a += kPrefillChunk) {
    const int n = count - a < kPrefillChunk ? count - a : kPrefillChunk;
    for (int r = 0; r < n; ++r) {
      e.host_rows->tokens[r] = tokens[a + r];
      e.host_rows->slots[r] = slot;
      e.host_rows->pos[r] = e.offsets[slot] + r;
    }
    e.host_rows->gdn_slots[0] = slot * e.n_gdn;
    int rc = MX_OK;
    if (hipMemcpyAsync(e.dev_rows, e.host_rows, sizeof(Engine::RowTable), hipMemcpyHostToDevice,
                       e.stream) != hipSuccess)
      rc = MX_EHIP;
    if (rc == MX_OK) {
      e.chunk = true;
      rc = record_chunk(e, n);
      e.chunk = false;
    }
    if (rc == MX_OK &&
        (hipMemcpyAsync(e.host_rows->next, e.dev_rows->next, sizeof(uint32_t),
                        hipMemcpyDeviceToHost, e.stream) != hipSuccess ||
         hipStreamSynchronize(e.stream) != hipSuccess))
      rc = MX_EHIP;
    if (rc != MX_OK) return step_failed(e, &slot, 1, rc, err);
    e.offsets[slot] += n;
    *next = e.host_rows->next[0];
  }
  e.last_rows = 0;  // the activation buffers hold no step's rows
  return MX_OK;
}

int engine_verify(Engine& e, int slot, const uint32_t* tokens, int count, uint32_t* next,
                  std::string* err) {
  // a failed slot is refused before its (partly updated) caches are
  // snapshotted, so a failure below always comes from this block's own step
  MX_TRY(slots_usable(e, &slot, 1, err));
  // snapshot the recurrent state so that keep = 0 can restore it
  const size_t sp = state_per(e), cp = conv_per(e);
  MX_HIP(hipMemcpyAsync(e.snap_state, e.gdn_state + size_t(slot) * e.n_gdn * sp, e.n_gdn * sp * 4,
                        hipMemcpyDeviceToDevice, e.stream));
  MX_HIP(hipMemcpyAsync(e.snap_conv, e.conv_state + size_t(slot) * e.n_gdn * cp, e.n_gdn * cp * 2,
                        hipMemcpyDeviceToDevice, e.stream));
  const int base = e.offsets[slot];
  const int rc = engine_block(e, slot, tokens, count, true, next, err);
  if (rc != MX_OK) {
    // a failed verify block puts back the snapshot it took: the state and
    // conv window return to the block's start, the offset never moved, and
    // the KV rows past it are overwritten before they are read
    if (e.failed[slot] &&
        hipMemcpyAsync(e.gdn_state + size_t(slot) * e.n_gdn * sp, e.snap_state, e.n_gdn * sp * 4,
                       hipMemcpyDeviceToDevice, e.stream) == hipSuccess &&
        hipMemcpyAsync(e.conv_state + size_t(slot) * e.n_gdn * cp, e.snap_conv, e.n_gdn * cp * 2,
                       hipMemcpyDeviceToDevice, e.stream) == hipSuccess &&
        hipStreamSynchronize(e.stream) == hipSuccess) {
      e.failed[slot] = 0;
      *err += " (the verify block's snapshot restored the slot)";
    }
    return rc;
  }
  e.verify_slot = slot;
  e.verify_count = count;
  e.verify_base = base;
  return MX_OK;
}

// Accept the first `keep` tokens of the last verify block
// (HybridCache::commit_verified, src/hybrid.rs:699-759): the GDN state after
// token keep-1 comes from the history, the conv window is re-sliced, and the
// attention offset is trimmed (later positions are overwritten by later steps).
int engine_commit(Engine& e, int slot, int keep, std::string* err) {
  if (slot != e.verify_slot) {
    *err = "no verify block pending on this slot";
    return MX_ESTATE;
  }
  if (keep < 0 || keep > e.verify_count) {
    *err = "keep outside the verify block";
    return MX_EINVAL;
  }
  const auto& c = e.cfg;
  const size_t sp = state_per(e), cp = conv_per(e);
  float* st = e.gdn_state + size_t(slot) * e.n_gdn * sp;
  uint16_t* cv = e.conv_state + size_t(slot) * e.n_gdn * cp;
  if (keep == 0) {
    MX_HIP(hipMemcpyAsync(st, e.snap_state, e.n_gdn * sp * 4, hipMemcpyDeviceToDevice, e.stream));
    MX_HIP(hipMemcpyAsync(cv, e.snap_conv, e.n_gdn * cp * 2, hipMemcpyDeviceToDevice, e.stream));
  } else if (keep < e.verify_count) {
    for (int g = 0; g < e.n_gdn; ++g) {
      MX_HIP(hipMemcpyAsync(st + g * sp, e.hist_state + (size_t(g) * c.max_verify + keep - 1) * sp,
                            sp * 4, hipMemcpyDeviceToDevice, e.stream));
      // window rows keep .. keep + K - 2 are the conv state after `keep` tokens
      MX_HIP(hipMemcpyAsync(cv + g * cp,
                            e.hist_conv + size_t(g) * (c.conv_k - 1 + c.max_verify) * e.cd +
                                size_t(keep) * e.cd,
                            cp * 2, hipMemcpyDeviceToDevice, e.stream));
    }
  }
  MX_HIP(hipStreamSynchronize(e.stream));
  e.offsets[slot] = e.verify_base + keep;
  e.verify_slot = -1;
  return MX_OK;
}

// Greedy generation from an empty slot (speculative::generate_prepared,
// src/speculative.rs:225-483, with its default policies: full-vocabulary
// greedy draft head, fixed depth, no EOS).  depth 0: prefill, then one decode
// step per token.  depth k >= 1: the MTP layer drafts k tokens (the first from
// the previous pass), a (k + 1)-token verify block checks them, the accepted
// prefix and the target's next token are emitted, the block is committed, and
// the draft layer is resynchronised on the target's hidden states of the
// accepted positions.  The MTP KV positions past the kept ones are
// overwritten before they are read again, so a snapshot is just a length.
int engine_generate(Engine& e, int slot, const uint32_t* prompt, int n_prompt, int max_tokens,
                    int depth, uint32_t* out, int* n_out, mx_generate_stats* stats,
                    uint32_t* drafts_out, std::string* err) {
  const auto& c = e.cfg;
  if (e.offsets[slot] != 0) {
    *err = "generate needs an empty slot";
    return MX_ESTATE;
  }
  if (n_prompt < 1 || max_tokens < 1) {
    *err = "empty prompt or no tokens requested";
    return MX_EINVAL;
  }
  if (depth < 0 || depth > 7 || depth + 1 > c.max_verify) {
    *err = "depth must be in 0..min(7, max_verify - 1)";
    return MX_EINVAL;
  }
  if (depth > 0 && !e.has_mtp) {
    *err = "the model has no MTP layer (mtp = 0)";
    return MX_EUNSUPPORTED;
  }
  if (int64_t(n_prompt) + max_tokens + depth + 1 > c.max_context) {
    *err = "prompt + tokens exceed max_context";
    return MX_EINVAL;
  }
  const size_t HS = size_t(c.hc) * c.hidden;
  mx_generate_stats st{};
  uint32_t nxt[8], drafts[kPrefillChunk], toks[kPrefillChunk];
  uint32_t bonus = 0, seed = 0;
  // prefill in blocks of 8 (or matrix-core chunks); with a draft layer, each
  // block's MTP pass follows it (MTP position i reads token i + 1 and the
  // target's hidden state at i; the last position reads the target's first
  // greedy token)
  const bool chunked = e.chunked_generate;
  const int block = chunked ? kPrefillChunk : 8;
  for (int a = 0; a < n_prompt; a += block) {
    const int cnt = n_prompt - a < block ? n_prompt - a : block;
    if (chunked) {
      MX_TRY(engine_prefill_chunked(e, slot, prompt + a, cnt, &bonus, err));
    } else {
      MX_TRY(engine_block(e, slot, prompt + a, cnt, false, nxt, err));
      bonus = nxt[cnt - 1];
    }
    if (depth > 0) {
      MX_HIP(hipMemcpyAsync(e.mtp_prev, e.h, cnt * HS * 2, hipMemcpyDeviceToDevice, e.stream));
      for (int r = 0; r < cnt; ++r) toks[r] = a + r + 1 < n_prompt ? prompt[a + r + 1] : bonus;
      MX_TRY(mtp_step(e, slot, toks, cnt, a, drafts, chunked));
      seed = drafts[cnt - 1];
      MX_HIP(hipMemcpyAsync(e.mtp_dh, e.h + (cnt - 1) * HS, HS * 2, hipMemcpyDeviceToDevice,
                            e.stream));
    }
  }
  int emitted = 0;
  out[emitted++] = bonus;
  if (depth == 0) {
    while (emitted < max_tokens) {
      const int32_t sl = slot;
      const uint32_t tok = out[emitted - 1];
      MX_TRY(engine_decode_rows(e, &sl, &tok, 1, nxt, err));
      out[emitted++] = nxt[0];
    }
  } else {
    int mtp_len = n_prompt;
    while (emitted < max_tokens) {
      const int k = depth < max_tokens - emitted ? depth : max_tokens - emitted;
      uint32_t drafted[8], block[8], pred[8];
      drafted[0] = seed;
      const int base = mtp_len;
      for (int i = 1; i < k; ++i) {
        MX_HIP(hipMemcpyAsync(e.mtp_prev, e.mtp_dh, HS * 2, hipMemcpyDeviceToDevice, e.stream));
        MX_TRY(mtp_step(e, slot, &drafted[i - 1], 1, base + i - 1, &drafted[i]));
        MX_HIP(hipMemcpyAsync(e.mtp_dh, e.h, HS * 2, hipMemcpyDeviceToDevice, e.stream));
      }
      block[0] = bonus;
      for (int i = 0; i < k; ++i) block[i + 1] = drafted[i];
      if (drafts_out)
        for (int i = 0; i < k; ++i) drafts_out[st.drafted + i] = drafted[i];
      MX_TRY(engine_verify(e, slot, block, k + 1, pred, err));
      int accepted = 0;
      while (accepted < k && drafted[accepted] == pred[accepted]) ++accepted;
      const uint32_t next = pred[accepted];
      int emitted_now = 0;
      bool ending = false;
      for (int i = 0; i <= accepted; ++i) {
        if (emitted == max_tokens) {
          ending = true;
          break;
        }
        out[emitted++] = i < accepted ? drafted[i] : next;
        ++emitted_now;
      }
      const int committed = ending ? (emitted_now < accepted ? emitted_now : accepted) + 1
                                   : accepted + 1;
      MX_TRY(engine_commit(e, slot, committed, err));
      st.rounds += 1;
      st.drafted += k;
      st.accepted += accepted;
      if (ending || emitted == max_tokens) break;
      bonus = next;
      // resynchronise: keep the draft positions of the first `kept` drafts,
      // then run the accepted tokens and the next one on the target's hidden
      // states (verify rows kept .. accepted, still in e.h after the commit)
      const int kept = accepted < k - 1 ? accepted : k - 1;
      mtp_len = base + kept;
      const int sync = accepted - kept + 1;
      for (int i = 0; i < sync - 1; ++i) toks[i] = drafted[kept + i];
      toks[sync - 1] = next;
      MX_HIP(hipMemcpyAsync(e.mtp_prev, e.h + size_t(kept) * HS, sync * HS * 2,
                            hipMemcpyDeviceToDevice, e.stream));
      MX_TRY(mtp_step(e, slot, toks, sync, mtp_len, drafts));
      seed = drafts[sync - 1];
      MX_HIP(hipMemcpyAsync(e.mtp_dh, e.h + size_t(sync - 1) * HS, HS * 2,
                            hipMemcpyDeviceToDevice, e.stream));
      mtp_len += sync;
    }
  }
  *n_out = emitted;
  if (stats) *stats = st;
  return MX_OK;
}

int engine_read(Engine& e, const char* what, void* host, size_t bytes, std::string* err) {
  const std::string w(what);
  const void* src = nullptr;
  size_t avail = 0;
  if (w == "hidden") {
    src = e.h;
    avail = size_t(e.last_rows) * e.cfg.hc * e.cfg.hidden * 2;
  } else if (w == "logits") {
    src = e.logits;
    avail = size_t(e.last_rows) * e.cfg.vocab * 2;
  } else {
    auto it = e.tensors.find(w);
    if (it == e.tensors.end()) {
      *err = "unknown tensor " + w;
      return MX_EINVAL;
    }
    src = it->second.p;
    avail = it->second.bytes;
  }
  if (bytes > avail) {
    *err = "read larger than the tensor";
    return MX_EINVAL;
  }
  MX_HIP(hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, e.stream));
  MX_HIP(hipStreamSynchronize(e.stream));
  return MX_OK;
}

// Algorithmic bytes of one step over the given rows (each distinct byte once):
// every weight outside the expert banks, the distinct experts' weights, the
// embedding rows, GDN state and conv window read + write, and the KV
// positions each row attends to.
// Bytes of the tensors under `prefix` outside the routed expert banks.
double dense_bytes(const Engine& e, const char* prefix) {
  double dense = 0.0;
  for (const auto& kv : e.tensors) {
    const std::string& n = kv.first;
    if (n.rfind(prefix, 0) != 0) continue;
    if (n.find(".moe.gate.") != std::string::npos || n.find(".moe.up.") != std::string::npos ||
        n.find(".moe.down.") != std::string::npos)
      continue;
    dense += double(kv.second.bytes);
  }
  return dense;
}

double step_bytes(const Engine& e, int rows, const int32_t* pos, double distinct_sum) {
  const auto& c = e.cfg;
  const double dense = dense_bytes(e, "layers.") + dense_bytes(e, "mixer.") + dense_bytes(e, "head.");
  double experts = 0.0;
  if (!e.layers.empty()) {
    const LayerW& L = e.layers[0];
    const QWeight g{L.gate.codes, L.gate.scales, L.gate.biases, L.gate.n, L.gate.k, L.gate.bits,
                    L.gate.group_size};
    const QWeight d{L.down.codes, L.down.scales, L.down.biases, L.down.n, L.down.k, L.down.bits,
                    L.down.group_size};
    experts = distinct_sum * double(2 * qw_bytes(g) + qw_bytes(d));
  }
  const double embed_rows = double(rows) * double(c.hidden) * (c.embed_bits / 8.0 + 4.0 / c.group_size);
  const double state = double(rows) * e.n_gdn *
                       (double(c.gdn_hv) * c.gdn_dk * c.gdn_dv * 4.0 + double(c.conv_k - 1) * e.cd * 2.0) * 2.0;
  double kv = 0.0;
  for (int r = 0; r < rows; ++r)
    kv += double(pos[r] + 1) * e.n_attn * c.kv_heads * c.head_dim * 2.0 * 2.0;
  return dense + experts + embed_rows + state + kv;
}

int engine_profile_step(Engine& e, const int32_t* slots, const uint32_t* tokens, int rows,
                        uint32_t* next, mx_step_profile* out, std::string* err) {
  std::memset(out, 0, sizeof(*out));
  out->rows = rows;
  int32_t pos[8];
  for (int r = 0; r < rows; ++r) pos[r] = e.offsets[slots[r]];
  for (auto& ev : e.ev)
    if (!ev) MX_HIP(hipEventCreate(&ev));
  hipEvent_t t0, t1;
  MX_HIP(hipEventCreate(&t0));
  MX_HIP(hipEventCreate(&t1));
  const bool graphs = e.use_graphs;
  e.use_graphs = false;
  e.prof = out;
  MX_HIP(hipEventRecord(t0, e.stream));
  const int rc = engine_decode_rows(e, slots, tokens, rows, next, err);
  e.prof = nullptr;
  e.use_graphs = graphs;
  MX_HIP(hipEventRecord(t1, e.stream));
  MX_HIP(hipEventSynchronize(t1));
  float ms = 0.0f;
  MX_HIP(hipEventElapsedTime(&ms, t0, t1));
  hipEventDestroy(t0);
  hipEventDestroy(t1);
  if (rc != MX_OK) return rc;
  out->step_ms = ms;
  out->step_bytes = step_bytes(e, rows, pos, out->distinct_experts);
  return MX_OK;
}

// Algorithmic bytes of one verify block of `count` tokens of one slot that
// starts at position `base` (each distinct byte once): every weight outside
// the expert banks, the routed experts the block touches (`routed`), the
// embedding rows, the GDN state read once and written after every token (the
// verify history), the conv window read and written, and the KV positions up
// to the block's last.
double verify_bytes(const Engine& e, int count, int base, double routed) {
  const auto& c = e.cfg;
  const double dense = dense_bytes(e, "layers.") + dense_bytes(e, "mixer.") + dense_bytes(e, "head.");
  const double embed_rows = double(count) * double(c.hidden) * (c.embed_bits / 8.0 + 4.0 / c.group_size);
  const double state = double(e.n_gdn) * (double(c.gdn_hv) * c.gdn_dk * c.gdn_dv * 4.0 * (1 + count) +
                                          double(c.conv_k - 1) * e.cd * 2.0 * 2.0);
  const double kv = double(base + count) * e.n_attn * c.kv_heads * c.head_dim * 2.0 * 2.0;
  return dense + routed + embed_rows + state + kv;
}

// Algorithmic bytes of one MTP draft step of one row at position `pos`: the
// draft layer's weights outside its expert banks, top_k routed experts of its
// bank, the embedding row, the shared greedy head and the draft layer's KV
// positions.
double draft_bytes(const Engine& e, int pos) {
  const auto& c = e.cfg;
  const LayerW& L = e.mtp.layer;
  const QWeight g{L.gate.codes, L.gate.scales, L.gate.biases, L.gate.n, L.gate.k, L.gate.bits,
                  L.gate.group_size};
  const QWeight d{L.down.codes, L.down.scales, L.down.biases, L.down.n, L.down.k, L.down.bits,
                  L.down.group_size};
  const double layer = dense_bytes(e, "mtp.layer.") + dense_bytes(e, "mtp.norm_") +
                       dense_bytes(e, "mtp.fc_") + dense_bytes(e, "mtp.mixer.");
  const double experts = double(c.top_k) * (2.0 * double(qw_bytes(g)) + double(qw_bytes(d)));
  const double embed_row = double(c.hidden) * (c.embed_bits / 8.0 + 4.0 / c.group_size);
  const double kv = double(pos + 1) * c.kv_heads * c.head_dim * 2.0 * 2.0;
  return layer + experts + embed_row + dense_bytes(e, "head.") + kv;
}

int engine_profile_verify(Engine& e, int slot, const uint32_t* tokens, int count, uint32_t* next,
                          mx_step_profile* out, std::string* err) {
  std::memset(out, 0, sizeof(*out));
  out->rows = count;
  const int base = e.offsets[slot];
  for (auto& ev : e.ev)
    if (!ev) MX_HIP(hipEventCreate(&ev));
  hipEvent_t t0, t1;
  MX_HIP(hipEventCreate(&t0));
  MX_HIP(hipEventCreate(&t1));
  const bool graphs = e.use_graphs;
  e.use_graphs = false;
  e.prof = out;
  e.prof_routed = 0.0;
  MX_HIP(hipEventRecord(t0, e.stream));
  const int rc = engine_verify(e, slot, tokens, count, next, err);
  e.prof = nullptr;
  e.use_graphs = graphs;
  MX_HIP(hipEventRecord(t1, e.stream));
  MX_HIP(hipEventSynchronize(t1));
  float ms = 0.0f;
  MX_HIP(hipEventElapsedTime(&ms, t0, t1));
  hipEventDestroy(t0);
  hipEventDestroy(t1);
  if (rc != MX_OK) return rc;
  out->step_ms = ms;
  out->step_bytes = verify_bytes(e, count, base, e.prof_routed);
  return MX_OK;
}

int engine_draft_bytes(const Engine& e, int pos, double* bytes, std::string* err) {
  if (!e.has_mtp) {
    *err = "the model has no MTP layer (mtp = 0)";
    return MX_EUNSUPPORTED;
  }
  *bytes = draft_bytes(e, pos);
  return MX_OK;
}

// Times the expert kernels of every MoE layer back to back on the routing
// and activations of the last step: all gate/up launches between two events,
// then all down launches.  Each launch reads its own layer's weights, so the
// weights come from HBM as in a step; back-to-back launches keep the events'
// own dispatch overhead out of the per-launch average.  Caches are untouched.
int engine_time_experts(Engine& e, int rows, mx_expert_timing* out, std::string* err) {
  const auto& c = e.cfg;
  std::memset(out, 0, sizeof(*out));
  if (rows < 1 || rows > 8) {
    *err = "rows must be in 1..8";
    return MX_EINVAL;
  }
  std::vector<uint32_t> ids(size_t(rows) * c.top_k);
  MX_HIP(hipMemcpyAsync(ids.data(), e.ids, ids.size() * 4, hipMemcpyDeviceToHost, e.stream));
  MX_HIP(hipStreamSynchronize(e.stream));
  std::vector<char> seen(c.experts, 0);
  int distinct = 0;
  for (uint32_t v : ids)
    if (v < uint32_t(c.experts) && !seen[v]) {
      seen[v] = 1;
      ++distinct;
    }
  for (auto& ev : e.ev)
    if (!ev) MX_HIP(hipEventCreate(&ev));
  if (!e.layers.empty() && !experts_fast(e, e.layers[0]))
    MX_TRY(moe_plan(e.ids, rows, c.top_k, e.moe_plan_buf, e.stream));
  MX_HIP(hipEventRecord(e.ev[0], e.stream));
  for (const LayerW& L : e.layers) MX_TRY(experts_gate_up(e, L, rows));
  MX_HIP(hipEventRecord(e.ev[1], e.stream));
  for (const LayerW& L : e.layers) MX_TRY(experts_down(e, L, rows));
  MX_HIP(hipEventRecord(e.ev[2], e.stream));
  MX_HIP(hipEventSynchronize(e.ev[2]));
  float a = 0.0f, b = 0.0f;
  MX_HIP(hipEventElapsedTime(&a, e.ev[0], e.ev[1]));
  MX_HIP(hipEventElapsedTime(&b, e.ev[1], e.ev[2]));
  out->launches = int32_t(e.layers.size());
  out->distinct_experts = distinct;
  out->gate_up_ms = a;
  out->down_ms = b;
  for (const LayerW& L : e.layers) {
    const QWeight g{L.gate.codes, L.gate.scales, L.gate.biases, L.gate.n, L.gate.k, L.gate.bits,
                    L.gate.group_size};
    const QWeight d{L.down.codes, L.down.scales, L.down.biases, L.down.n, L.down.k, L.down.bits,
                    L.down.group_size};
    out->gate_up_bytes += double(distinct) * 2.0 * double(qw_bytes(g)) +
                          double(qw_bytes(L.sgate) + qw_bytes(L.sup));
    out->down_bytes += double(distinct) * double(qw_bytes(d)) + double(qw_bytes(L.sdown));
  }
  return MX_OK;
}

// Gives a slot a synthetic context of `length` positions: random K/V for
// those positions, random GDN state and conv window (decode cost depends on
// the context length only, so this stands in for a prefill when measuring).
int engine_fill_slot(Engine& e, int slot, int length, uint64_t seed, std::string* err) {
  const auto& c = e.cfg;
  if (length < 0 || length > c.max_context) {
    *err = "length outside 0..max_context";
    return MX_EINVAL;
  }
  const size_t sp = state_per(e), cp = conv_per(e);
  MX_TRY(fill_f32(e.gdn_state + size_t(slot) * e.n_gdn * sp, e.n_gdn * sp, seed, -0.05f, 0.05f,
                  e.stream));
  MX_TRY(fill_bf16(e.conv_state + size_t(slot) * e.n_gdn * cp, e.n_gdn * cp, seed + 1, 1, 1.0f,
                   0.0f, e.stream));
  const size_t plane = size_t(c.max_context) * c.head_dim;
  for (int p = 0; p < e.n_attn * c.kv_heads; ++p) {
    uint16_t* kb = e.k_cache + size_t(slot) * e.ad.slot_stride + p * plane;
    uint16_t* vb = e.v_cache + size_t(slot) * e.ad.slot_stride + p * plane;
    MX_TRY(fill_bf16(kb, size_t(length) * c.head_dim, seed + 2 + 2 * p, 1, 1.0f, 0.0f, e.stream));
    MX_TRY(fill_bf16(vb, size_t(length) * c.head_dim, seed + 3 + 2 * p, 1, 1.0f, 0.0f, e.stream));
  }
  MX_HIP(hipStreamSynchronize(e.stream));
  e.offsets[slot] = length;
  e.failed[slot] = 0;
  if (e.verify_slot == slot) e.verify_slot = -1;
  return MX_OK;
}

int engine_tensor(Engine& e, const char* name, void** ptr, size_t* bytes) {
  auto it = e.tensors.find(name);
  if (it == e.tensors.end()) return MX_EINVAL;
  *ptr = it->second.p;
  *bytes = it->second.bytes;
  return MX_OK;
}

void engine_set_flags(Engine& e, int want_logits, int use_graphs, int exact, int exact_parts,
                      int chunked_generate) {
  e.want_logits = want_logits != 0;
  e.chunked_generate = chunked_generate != 0;
  e.use_graphs = use_graphs != 0;
  if (e.exact != (exact != 0) || e.exact_parts != exact_parts) {
    // captured graphs bake in the kernel choice
    for (auto& g : e.graphs) hipGraphExecDestroy(g.second);
    e.graphs.clear();
  }
  e.exact = exact != 0;
  e.exact_parts = exact_parts;
}

// ---------------------------------------------------------------------------
// Checkpoint loading: MLX tensor names (the reference's Weights / HybridModel
// loaders, src/weights.rs:22-99, src/hybrid.rs:56-66, 130-142, 335-352,
// 529-567, src/mtp.rs:39-70) onto the engine's matrices, several of which fuse
// reference modules: the GDN input projection is qkv | z | a | b, the router
// carries the shared-expert gate as its last row, a hyper-connection's down
// projection carries the block-inject rows after the low-rank rows, and the
// attention input projection is q_proj (query and gate per head) | k | v.
namespace {

bool take(std::string& s, const char* prefix) {
  const size_t n = std::strlen(prefix);
  if (s.compare(0, n, prefix) != 0) return false;
  s.erase(0, n);
  return true;
}

}  // namespace

// Where one MLX tensor goes, from the model configuration alone: rows
// [row0, row0 + rows) of the engine matrix `tensor` (its codes, scales or
// biases), or the whole bf16 / fp32 vector `tensor`, or the GDN conv weight
// (fp32 [taps][channels] from MLX's [channels][taps][1]).
int checkpoint_target(const mx_model_config& c, std::string name, CheckpointTarget* t) {
  using T = CheckpointTarget;
  auto quant = [&](const std::string& tensor, int n, int k, int bits, int row0, int rows,
                   const std::string& rest) -> int {
    t->kind = T::kQuant;
    t->tensor = tensor;
    t->n = n;
    t->k = k;
    t->bits = bits;
    t->row0 = row0;
    t->rows = rows;
    if (rest == "weight") t->part = 0;
    else if (rest == "scales") t->part = 1;
    else if (rest == "biases") t->part = 2;
    else return MX_EINVAL;
    return MX_OK;
  };
  auto vec = [&](const std::string& tensor, T::Kind kind, size_t count) -> int {
    t->kind = kind;
    t->tensor = tensor;
    t->count = count;
    return MX_OK;
  };
  const int H = c.hidden, hc = c.hc, r = c.hc_rank;
  const int cd = 2 * c.gdn_hk * c.gdn_dk + c.gdn_hv * c.gdn_dv, vd = c.gdn_hv * c.gdn_dv;
  const int P = cd + vd + 2 * c.gdn_hv;
  const int qr = c.heads * 2 * c.head_dim, kv = c.kv_heads * c.head_dim, Q = qr + 2 * kv;
  auto hcw = [&](const std::string& e, int layer, bool inject, std::string rest) -> int {
    const int bits = layer_bits(c, layer, 0), nd = r + (inject ? hc : 0);
    if (rest == "hc_norm.weight") return vec(e + ".scale", T::kBf16, size_t(hc) * H);
    if (take(rest, "input_mix_weight_down.")) return quant(e + ".down", nd, hc * H, bits, 0, r, rest);
    if (inject && take(rest, "block_inject_weight.")) return quant(e + ".down", nd, hc * H, bits, r, hc, rest);
    if (take(rest, "input_mix_weight_up.")) return quant(e + ".up", hc * H, r, bits, 0, hc * H, rest);
    return int(MX_EINVAL);
  };
  auto layer = [&](const std::string& e, int i, bool attn, std::string rest) -> int {
    const int bits = layer_bits(c, i, 0), db = layer_bits(c, i, 1);
    if (take(rest, "attn_hyper_connection.")) return hcw(e + ".attn_hc", i, true, rest);
    if (take(rest, "mlp_hyper_connection.")) return hcw(e + ".mlp_hc", i, true, rest);
    if (take(rest, "ple.")) return int(MX_EUNSUPPORTED);  // per-layer n-gram embeddings: not built
    if (!attn && take(rest, "linear_attn.")) {
      const std::string g = e + ".gdn.in";
      if (take(rest, "in_proj_qkv.")) return quant(g, P, H, bits, 0, cd, rest);
      if (take(rest, "in_proj_z.")) return quant(g, P, H, bits, cd, vd, rest);
      if (take(rest, "in_proj_a.")) return quant(g, P, H, bits, cd + vd, c.gdn_hv, rest);
      if (take(rest, "in_proj_b.")) return quant(g, P, H, bits, cd + vd + c.gdn_hv, c.gdn_hv, rest);
      if (take(rest, "out_proj.")) return quant(e + ".gdn.out", H, vd, bits, 0, H, rest);
      if (rest == "conv1d.weight") {
        t->conv_ch = cd;
        t->taps = c.conv_k;
        return vec(e + ".gdn.conv_w", T::kConvW, size_t(cd) * c.conv_k);
      }
      if (rest == "A_log") return vec(e + ".gdn.a_log", T::kF32, size_t(c.gdn_hv));
      if (rest == "dt_bias") return vec(e + ".gdn.dt_bias", T::kBf16, size_t(c.gdn_hv));
      if (rest == "norm.weight") return vec(e + ".gdn.norm", T::kBf16, size_t(c.gdn_dv));
      return int(MX_EINVAL);
    }
    if (attn && take(rest, "self_attn.")) {
      if (take(rest, "indexer.")) return int(MX_EUNSUPPORTED);  // sparse-attention indexer: not built
      const std::string a = e + ".attn.in";
      if (take(rest, "q_proj.")) return quant(a, Q, H, bits, 0, qr, rest);
      if (take(rest, "k_proj.")) return quant(a, Q, H, bits, qr, kv, rest);
      if (take(rest, "v_proj.")) return quant(a, Q, H, bits, qr + kv, kv, rest);
      if (take(rest, "o_proj.")) return quant(e + ".attn.out", H, c.heads * c.head_dim, bits, 0, H, rest);
      if (rest == "q_norm.weight") return vec(e + ".attn.q_norm", T::kBf16, size_t(c.head_dim));
      if (rest == "k_norm.weight") return vec(e + ".attn.k_norm", T::kBf16, size_t(c.head_dim));
      return int(MX_EINVAL);
    }
    if (take(rest, "mlp.")) {
      const std::string m = e + ".moe.";
      const int E = c.experts, I = c.moe_inter, SI = c.shared_inter;
      if (take(rest, "gate.")) return quant(m + "router", E + 1, H, bits, 0, E, rest);
      if (take(rest, "shared_expert_gate.")) return quant(m + "router", E + 1, H, bits, E, 1, rest);
      if (take(rest, "switch_mlp.gate_proj.")) return quant(m + "gate", E * I, H, bits, 0, E * I, rest);
      if (take(rest, "switch_mlp.up_proj.")) return quant(m + "up", E * I, H, bits, 0, E * I, rest);
      if (take(rest, "switch_mlp.down_proj.")) return quant(m + "down", E * H, I, db, 0, E * H, rest);
      if (take(rest, "shared_expert.gate_proj.")) return quant(m + "shared_gate", SI, H, bits, 0, SI, rest);
      if (take(rest, "shared_expert.up_proj.")) return quant(m + "shared_up", SI, H, bits, 0, SI, rest);
      if (take(rest, "shared_expert.down_proj.")) return quant(m + "shared_down", H, SI, db, 0, H, rest);
      return int(MX_EINVAL);
    }
    return int(MX_EINVAL);
  };
  take(name, "language_model.");
  if (take(name, "model.embed_tokens.")) return quant("embed", c.vocab, H, c.embed_bits, 0, c.vocab, name);
  if (take(name, "lm_head.")) return quant("head", c.vocab, H, c.head_bits, 0, c.vocab, name);
  if (take(name, "model.hyper_connection_mixer.")) return hcw("mixer", -1, false, name);
  if (take(name, "model.layers.")) {
    const size_t dot = name.find('.');
    if (dot == std::string::npos || dot == 0) return MX_EINVAL;
    const int i = std::atoi(name.substr(0, dot).c_str());
    if (i < 0 || i >= c.layers) return MX_EINVAL;
    const bool attn = i % c.attn_every == c.attn_every - 1;
    return layer("layers." + std::to_string(i), i, attn, name.substr(dot + 1));
  }
  if (take(name, "mtp.")) {
    if (!c.mtp) return MX_EUNSUPPORTED;  // configuration without the draft layer
    const int m = c.layers, bits = layer_bits(c, m, 0);
    if (take(name, "layers.0.")) return layer("mtp.layer", m, true, name);
    if (name == "pre_fc_norm_embedding.weight") return vec("mtp.norm_emb", T::kBf16, size_t(H));
    if (name == "pre_fc_norm_hidden.weight") return vec("mtp.norm_hidden", T::kBf16, size_t(hc) * H);
    if (take(name, "fc_embedding.")) return quant("mtp.fc_emb", H, H, bits, 0, H, name);
    if (take(name, "fc_hidden.")) return quant("mtp.fc_hidden", H, H, bits, 0, H, name);
    if (take(name, "hyper_connection_mixer.")) return hcw("mtp.mixer", m, false, name);
    return MX_EINVAL;
  }
  return MX_EINVAL;
}

namespace {

float load_value(const void* data, int dtype, size_t i) {
  switch (dtype) {
    case MX_DT_BF16: return bf16_to_f32(static_cast<const uint16_t*>(data)[i]);
    case MX_DT_F16: {
      _Float16 h;
      std::memcpy(&h, static_cast<const uint16_t*>(data) + i, 2);
      return float(h);
    }
    default: return static_cast<const float*>(data)[i];
  }
}

bool float_dtype(int dtype) { return dtype == MX_DT_BF16 || dtype == MX_DT_F16 || dtype == MX_DT_F32; }

// The first value of an F16 / F32 tensor that bf16 cannot hold exactly, or -1.
int64_t first_inexact_bf16(const void* data, int dtype, size_t count) {
  if (dtype == MX_DT_BF16) return -1;
  for (size_t i = 0; i < count; ++i) {
    const float v = load_value(data, dtype, i);
    uint32_t u;
    std::memcpy(&u, &v, 4);
    if (u & 0xffffu) return int64_t(i);
  }
  return -1;
}

std::vector<uint16_t> to_bf16(const void* data, int dtype, size_t count) {
  std::vector<uint16_t> v(count);
  for (size_t i = 0; i < count; ++i) {
    if (dtype == MX_DT_BF16) {
      v[i] = static_cast<const uint16_t*>(data)[i];
    } else {
      const float f = load_value(data, dtype, i);
      uint32_t u;
      std::memcpy(&u, &f, 4);
      v[i] = uint16_t(u >> 16);  // exact: first_inexact_bf16 passed
    }
  }
  return v;
}

// Every check of one tensor that needs no engine: its target, rank, dims,
// byte count, dtype, width, group count and (with data) exact float values.
int plan_tensor(const mx_model_config& c, const char* name, int dtype, const int64_t* shape,
                int ndim, const void* data, size_t bytes, CheckpointTarget* t, size_t* count_out,
                std::string* err) {
  const int rc = checkpoint_target(c, name, t);
  if (rc == MX_EUNSUPPORTED) {
    *err = std::string("the engine has no module for tensor ") + name;
    return MX_EUNSUPPORTED;
  }
  if (rc != MX_OK) {
    *err = std::string("unknown tensor name ") + name;
    return MX_EINVAL;
  }
  if (ndim < 1 || ndim > 4) {
    *err = std::string(name) + ": bad rank";
    return MX_EINVAL;
  }
  size_t count = 1;
  for (int i = 0; i < ndim; ++i) {
    if (shape[i] <= 0 || shape[i] > (int64_t(1) << 40)) {
      *err = std::string(name) + ": dim " + std::to_string(i) + " is " + std::to_string(shape[i]);
      return MX_EINVAL;
    }
    if (count > (size_t(1) << 42) / size_t(shape[i])) {
      *err = std::string(name) + ": shape too large";
      return MX_EINVAL;
    }
    count *= size_t(shape[i]);
  }
  const size_t esize = dtype == MX_DT_F32 || dtype == MX_DT_U32 ? 4 : 2;
  if (bytes != count * esize) {
    *err = std::string(name) + ": byte count does not match shape and dtype";
    return MX_EINVAL;
  }
  *count_out = count;
  if (t->kind != CheckpointTarget::kQuant) {
    if (!float_dtype(dtype) || count != t->count) {
      *err = std::string(name) + ": expected " + std::to_string(t->count) + " float values";
      return MX_EINVAL;
    }
    if (t->kind == CheckpointTarget::kConvW && shape[0] != t->conv_ch) {
      *err = std::string(name) + ": conv channels differ from the engine's";
      return MX_EINVAL;
    }
  } else {
    // quantised matrix rows: leading dims flatten into rows (an expert bank
    // is [experts, n, width]), the last dim is the packed or per-group width
    const int64_t width = shape[ndim - 1];
    const int64_t rows = int64_t(count / size_t(width));
    if (rows != t->rows) {
      *err = std::string(name) + ": " + std::to_string(rows) + " rows, the engine's matrix takes " +
             std::to_string(t->rows);
      return MX_EINVAL;
    }
    const int gs = c.group_size;
    const int64_t words = int64_t(t->k) * t->bits / 32, groups = t->k / gs;
    if (t->part == 0) {
      if (dtype != MX_DT_U32) {
        *err = std::string(name) + ": packed codes must be U32 (unquantised matrices are not supported)";
        return MX_EUNSUPPORTED;
      }
      if (width != words) {
        *err = std::string(name) + ": " + std::to_string(width * 32 / t->k) +
               "-bit codes, the engine's matrix is " + std::to_string(t->bits) + "-bit";
        return MX_EUNSUPPORTED;
      }
      return MX_OK;
    }
    if (!float_dtype(dtype) || width != groups) {
      *err = std::string(name) + ": " + std::to_string(width) +
             " groups per row, the engine's matrix has " + std::to_string(groups) +
             " (group size " + std::to_string(gs) + ")";
      return MX_EUNSUPPORTED;
    }
  }
  // bf16 targets keep values exactly or refuse them (never a silent rounding)
  const bool to_bf16_target = t->kind == CheckpointTarget::kQuant || t->kind == CheckpointTarget::kBf16;
  if (data && to_bf16_target) {
    const int64_t bad = first_inexact_bf16(data, dtype, count);
    if (bad >= 0) {
      char v[64];
      std::snprintf(v, sizeof v, "%.9g", double(load_value(data, dtype, size_t(bad))));
      *err = std::string(name) + ": value " + v + " at index " + std::to_string(bad) +
             " is not a bf16 value (the engine keeps this tensor in bf16 and does not round it)";
      return MX_EUNSUPPORTED;
    }
  }
  return MX_OK;
}

}  // namespace

int engine_load_tensor(Engine& e, const char* name, int dtype, const int64_t* shape, int ndim,
                       const void* data, size_t bytes, std::string* err) {
  CheckpointTarget t;
  size_t count = 0;
  MX_TRY(plan_tensor(e.cfg, name, dtype, shape, ndim, data, bytes, &t, &count, err));
  auto ptr = [&](const std::string& n) -> void* {
    auto it = e.tensors.find(n);
    return it == e.tensors.end() ? nullptr : it->second.p;
  };
  const char* suffix = t.kind != CheckpointTarget::kQuant ? ""
                       : t.part == 0                      ? ".codes"
                       : t.part == 1                      ? ".scales"
                                                          : ".biases";
  char* dst = static_cast<char*>(ptr(t.tensor + suffix));
  if (!dst) {
    *err = "engine tensor " + t.tensor + " missing";
    return MX_EINVAL;
  }
  auto put = [&](const void* src, size_t n) {
    return hipMemcpy(dst, src, n, hipMemcpyHostToDevice) == hipSuccess ? MX_OK : MX_EHIP;
  };
  switch (t.kind) {
    case CheckpointTarget::kBf16: {
      const std::vector<uint16_t> v = to_bf16(data, dtype, count);
      return put(v.data(), count * 2);
    }
    case CheckpointTarget::kF32: {
      std::vector<float> v(count);
      for (size_t i = 0; i < count; ++i) v[i] = load_value(data, dtype, i);
      return put(v.data(), count * 4);
    }
    case CheckpointTarget::kConvW: {  // MLX conv1d weight [channels, taps, 1] -> [taps][channels]
      std::vector<float> v(count);
      for (int ch = 0; ch < t.conv_ch; ++ch)
        for (int j = 0; j < t.taps; ++j)
          v[size_t(j) * t.conv_ch + ch] = load_value(data, dtype, size_t(ch) * t.taps + j);
      return put(v.data(), count * 4);
    }
    case CheckpointTarget::kQuant:
      break;
  }
  const int64_t words = int64_t(t.k) * t.bits / 32, groups = t.k / e.cfg.group_size;
  if (t.part == 0) {
    dst += size_t(t.row0) * words * 4;
    return put(data, bytes);
  }
  dst += size_t(t.row0) * groups * 2;
  const std::vector<uint16_t> v = to_bf16(data, dtype, count);
  return put(v.data(), count * 2);
}

namespace {

// A minimal JSON reader for safetensors headers: objects of names to
// {"dtype": str, "shape": [int...], "data_offsets": [int, int]}, plus
// "__metadata__" (skipped).
struct JsonIn {
  const char* p;
  const char* end;
  void ws() { while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p; }
  bool eat(char ch) {
    ws();
    if (p < end && *p == ch) { ++p; return true; }
    return false;
  }
  bool str(std::string* out) {
    ws();
    if (p >= end || *p != '"') return false;
    ++p;
    out->clear();
    while (p < end && *p != '"') {
      if (*p == '\\' && p + 1 < end) {
        ++p;
        const char ch = *p;
        out->push_back(ch == 'n' ? '\n' : ch == 't' ? '\t' : ch);
      } else {
        out->push_back(*p);
      }
      ++p;
    }
    if (p >= end) return false;
    ++p;
    return true;
  }
  bool num(int64_t* v) {
    ws();
    if (p >= end || !(*p == '-' || (*p >= '0' && *p <= '9'))) return false;
    int64_t x = 0;
    bool neg = false;
    if (*p == '-') { neg = true; ++p; }
    const char* first = p;
    while (p < end && *p >= '0' && *p <= '9') {
      if (x > (INT64_MAX - 9) / 10) return false;  // out of range
      x = x * 10 + (*p - '0');
      ++p;
    }
    if (p == first) return false;
    *v = neg ? -x : x;
    return true;
  }
  bool skip(int depth = 0) {  // any value
    ws();
    if (p >= end || depth > 64) return false;
    if (*p == '"') { std::string s; return str(&s); }
    if (*p == '{' || *p == '[') {
      const char open = *p, close = open == '{' ? '}' : ']';
      ++p;
      if (eat(close)) return true;
      do {
        if (open == '{') {
          std::string k;
          if (!str(&k) || !eat(':')) return false;
        }
        if (!skip(depth + 1)) return false;
      } while (eat(','));
      return eat(close);
    }
    while (p < end && *p != ',' && *p != '}' && *p != ']') ++p;
    return true;
  }
};

struct StEntry {
  std::string name, dtype;
  std::vector<int64_t> shape;
  int64_t begin = -1, end = -1;
};

bool parse_header(const char* p, size_t n, std::vector<StEntry>* out) {
  JsonIn in{p, p + n};
  if (!in.eat('{')) return false;
  if (in.eat('}')) return true;
  do {
    StEntry en;
    if (!in.str(&en.name) || !in.eat(':')) return false;
    if (en.name == "__metadata__") {
      if (!in.skip()) return false;
      continue;
    }
    if (!in.eat('{')) return false;
    do {
      std::string key;
      if (!in.str(&key) || !in.eat(':')) return false;
      if (key == "dtype") {
        if (!in.str(&en.dtype)) return false;
      } else if (key == "shape" || key == "data_offsets") {
        std::vector<int64_t> v;
        if (!in.eat('[')) return false;
        if (!in.eat(']')) {
          do {
            int64_t x;
            if (!in.num(&x) || v.size() >= 8) return false;
            v.push_back(x);
          } while (in.eat(','));
          if (!in.eat(']')) return false;
        }
        if (key == "shape") {
          en.shape = v;
        } else {
          if (v.size() != 2) return false;
          en.begin = v[0];
          en.end = v[1];
        }
      } else if (!in.skip()) {
        return false;
      }
    } while (in.eat(','));
    if (!in.eat('}')) return false;
    out->push_back(std::move(en));
  } while (in.eat(','));
  return in.eat('}');
}

// Reads a .safetensors file and calls fn(name, dtype, shape, ndim, data, bytes)
// for each tensor the reference's loader keeps (it skips vision towers and
// the n-gram tables' row shards, src/weights.rs:48-54), stopping at the first
// nonzero status.  Offsets are checked against the file before any read.
template <class Fn>
int read_safetensors(const char* path, int* done, std::string* err, Fn fn) {
  *done = 0;
  FILE* f = std::fopen(path, "rb");
  if (!f) {
    *err = std::string("cannot open ") + path;
    return MX_EINVAL;
  }
  std::unique_ptr<FILE, int (*)(FILE*)> guard(f, std::fclose);
  if (std::fseek(f, 0, SEEK_END) != 0) {
    *err = std::string(path) + ": cannot seek";
    return MX_EINVAL;
  }
  const long fsize = std::ftell(f);
  std::rewind(f);
  uint64_t hlen = 0;
  if (fsize < 8 || std::fread(&hlen, 8, 1, f) != 1 || hlen > (100ull << 20) ||
      hlen > uint64_t(fsize) - 8) {
    *err = std::string(path) + ": not a safetensors file";
    return MX_EINVAL;
  }
  std::string header(size_t(hlen), '\0');
  if (std::fread(&header[0], 1, header.size(), f) != header.size()) {
    *err = std::string(path) + ": truncated header";
    return MX_EINVAL;
  }
  std::vector<StEntry> entries;
  if (!parse_header(header.data(), header.size(), &entries)) {
    *err = std::string(path) + ": unreadable header";
    return MX_EINVAL;
  }
  const int64_t base = int64_t(8 + hlen), data_size = int64_t(fsize) - base;
  std::vector<char> buf;
  for (const StEntry& en : entries) {
    if (en.name.rfind("visual.", 0) == 0 || en.name.rfind("vision_tower.", 0) == 0 ||
        en.name.find(".ngram_embedding.shards.") != std::string::npos)
      continue;
    int dt;
    if (en.dtype == "U32") dt = MX_DT_U32;
    else if (en.dtype == "BF16") dt = MX_DT_BF16;
    else if (en.dtype == "F16") dt = MX_DT_F16;
    else if (en.dtype == "F32") dt = MX_DT_F32;
    else {
      *err = en.name + ": unsupported dtype " + en.dtype;
      return MX_EUNSUPPORTED;
    }
    if (en.begin < 0 || en.end < en.begin || en.end > data_size) {
      *err = en.name + ": data_offsets [" + std::to_string(en.begin) + ", " +
             std::to_string(en.end) + "] outside the file's " + std::to_string(data_size) +
             " data bytes";
      return MX_EINVAL;
    }
    if (en.shape.empty()) {
      *err = en.name + ": empty shape";
      return MX_EINVAL;
    }
    for (int64_t d : en.shape)
      if (d <= 0) {
        *err = en.name + ": dim " + std::to_string(d);
        return MX_EINVAL;
      }
    buf.resize(size_t(en.end - en.begin));
    if (std::fseek(f, long(base + en.begin), SEEK_SET) != 0 ||
        std::fread(buf.data(), 1, buf.size(), f) != buf.size()) {
      *err = en.name + ": truncated data";
      return MX_EINVAL;
    }
    const int rc = fn(en.name.c_str(), dt, en.shape.data(), int(en.shape.size()), buf.data(),
                      buf.size());
    if (rc != MX_OK) return rc;
    ++*done;
  }
  return MX_OK;
}

}  // namespace

int engine_load_safetensors(Engine& e, const char* path, int* loaded, std::string* err) {
  return read_safetensors(path, loaded, err,
                          [&](const char* name, int dt, const int64_t* shape, int ndim,
                              const void* data, size_t bytes) {
                            return engine_load_tensor(e, name, dt, shape, ndim, data, bytes, err);
                          });
}

int checkpoint_check(const mx_model_config& c, const char* path, int* checked, std::string* err) {
  return read_safetensors(path, checked, err,
                          [&](const char* name, int dt, const int64_t* shape, int ndim,
                              const void* data, size_t bytes) {
                            CheckpointTarget t;
                            size_t count = 0;
                            return plan_tensor(c, name, dt, shape, ndim, data, bytes, &t, &count,
                                               err);
                          });
}

const mx_model_config& engine_config(const Engine& e) { return e.cfg; }
int engine_gdn_layers(const Engine& e) { return e.n_gdn; }
int engine_attn_layers(const Engine& e) { return e.n_attn; }
hipStream_t engine_stream(const Engine& e) { return e.stream; }

}  // namespace mx
