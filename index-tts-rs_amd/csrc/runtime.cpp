// libitts_hip runtime: the C ABI of include/itts_hip.h over the gfx950 kernels.
//
// Mirrors the reference's decoder interface (crates/core/src/models/gpt.rs and
// sampler.rs): Gpt::from_weights -> itts_gpt_create, KvCache::new -> itts_kv_create,
// prefill / prefill_after / step, sample_next_token and generate_codes_after.
// Everything here is host orchestration; all arithmetic runs in the HIP kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/itts_hip.h"
#include "kernels.h"

using namespace itts;

namespace {

thread_local std::string g_last_error;

itts_status set_error(itts_status st, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

}  // namespace

// Error text from other translation units of the library (the safetensors loader).
namespace itts {
itts_status set_error_text(itts_status st, const char *msg) {
  g_last_error = msg;
  return st;
}
}  // namespace itts

namespace {

#define HIP_TRY(expr)                                                                    \
  do {                                                                                   \
    hipError_t e_ = (expr);                                                              \
    if (e_ != hipSuccess)                                                                \
      return set_error(ITTS_E_DEVICE, "HIP error %s at %s:%d: %s", hipGetErrorName(e_), \
                       __FILE__, __LINE__, #expr);                                       \
  } while (0)

struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  hipError_t ensure(size_t n) {
    if (n <= bytes) return hipSuccess;
    if (p) {
      hipError_t e = hipFree(p);
      if (e != hipSuccess) return e;
      p = nullptr;
      bytes = 0;
    }
    hipError_t e = hipMalloc(&p, n);
    if (e == hipSuccess) bytes = n;
    return e;
  }
  template <class T>
  T *as() const {
    return static_cast<T *>(p);
  }
};

// Activation rows in the prefill GEMM's split form (bf16 hi/lo planes + group sums).
// Pinned host staging for asynchronous uploads: the copies that read it are followed by
// `ready`, and the next rewrite waits for that event first, so a call returns without
// waiting for its uploads to land.
struct HostStage {
  void *p = nullptr;
  size_t bytes = 0;
  hipEvent_t ready = nullptr;
  ~HostStage() {
    if (ready) (void)hipEventDestroy(ready);
    if (p) (void)hipHostFree(p);
  }
  // room for n bytes, once the previous uploads from here have landed
  hipError_t acquire(size_t n) {
    hipError_t e = ready ? hipEventSynchronize(ready) : hipEventCreateWithFlags(&ready, hipEventDisableTiming);
    if (e != hipSuccess || n <= bytes) return e;
    if (p) {
      e = hipHostFree(p);
      p = nullptr;
      bytes = 0;
      if (e != hipSuccess) return e;
    }
    e = hipHostMalloc(&p, n, hipHostMallocDefault);
    if (e == hipSuccess) bytes = n;
    return e;
  }
  hipError_t release(hipStream_t s) { return hipEventRecord(ready, s); }
  template <class T>
  T *as() const {
    return static_cast<T *>(p);
  }
};

struct SplitBuf {
  DevBuf hi, lo, gs;
  hipError_t ensure(size_t M, int K) {
    hipError_t e = hi.ensure(sizeof(uint16_t) * M * K);
    if (e == hipSuccess) e = lo.ensure(sizeof(uint16_t) * M * K);
    if (e == hipSuccess) e = gs.ensure(sizeof(float) * M * (K / 64));
    return e;
  }
  SplitOut out() const { return SplitOut{hi.as<uint16_t>(), lo.as<uint16_t>(), gs.as<float>()}; }
  SplitAct act() const { return out().act(); }
};

bool valid_config(const itts_config &c, std::string &why) {
  char b[256];
  auto fail = [&](const char *m) {
    why = m;
    return false;
  };
  if (c.n_layer <= 0) return fail("config: n_layer must be >= 1");
  if (c.n_head <= 0 || c.d_model != c.n_head * 64) return fail("config: d_model must equal n_head * 64");
  if (c.d_ffn <= 0 || c.d_ffn % 64 != 0) return fail("config: d_ffn must be a positive multiple of 64");
  if (c.quant_bits != 8 && c.quant_bits != 4) return fail("config: quant_bits must be 8 or 4");
  if (c.param_dtype != ITTS_F16 && c.param_dtype != ITTS_F32) return fail("config: param_dtype must be F16 or F32");
  const int epc = c.quant_bits == 8 ? 16 : 32;
  if (c.d_model / epc > 512 || c.d_ffn / epc > 512) return fail("config: K too large for the decode GEMV");
  if (c.mel_vocab < 3 || c.mel_vocab > 9216) return fail("config: mel_vocab must be in 3..=9216");
  if (c.text_vocab < 2 || c.lang_vocab < 1) return fail("config: text_vocab >= 2 and lang_vocab >= 1");
  if (c.mel_pos_len < 3 || c.text_pos_len < 3) return fail("config: positional tables too short");
  (void)b;
  return true;
}

}  // namespace

// ------------------------------------------------------------------------------------
// Handles
// ------------------------------------------------------------------------------------

struct QLHost {
  DevBuf codes, params, bias;
  DevQL dev() const { return DevQL{codes.as<uint8_t>(), params.p, bias.as<float>(), N, K}; }
  int N = 0, K = 0;
};

// A decoder is shared by its KV caches: each cache holds a reference, so destroying the
// decoder while caches are alive (in any order) never leaves a cache pointing at freed
// memory; the object goes when the last of them is released.
struct itts_gpt {
  itts_config cfg{};
  hipStream_t stream = nullptr;
  int refs = 1;
  bool user_released = false;
  // Decode iterations replay a captured graph; ITTS_NO_GRAPH=1 enqueues the same
  // kernels directly (for tools that cannot follow graph launches).
  bool use_graph = true;
  int max_cond = 64;
  DevBuf text_emb, lang_emb, mel_emb, mel_pos, text_pos;
  std::vector<DevBuf> ln;  // ln1_w, ln1_b, ln2_w, ln2_b per layer, then ln_f, final_norm
  std::vector<QLHost> qls; // 4 per layer, then mel_head
  std::vector<DevLayer> layers;
  DevBuf ln_f_w, ln_f_b, fn_w, fn_b;
  DevQL head{};
  // persistent decode step: device copy of `layers`; the folded LayerNorm rows
  // (fold_floats(d, F) per layer, int8 and int4 codes; the batched step's products use
  // them too); blocks (one per compute unit)
  DevBuf dlayers, fold;
  int n_cu = 0;
  int device = 0;
  bool persist_ok = false;  // kernels set up (int8 or int4 codes)
  itts_decode_path path = ITTS_DECODE_AUTO;
  // decode workspace
  DevBuf x, q, a, f, logits;
  // prefill workspace (grown on demand): residual stream and q (fp32), GEMM inputs in
  // split form (LN output, attention output, GELU output), split-K partials and counters
  DevBuf px, pq, rows, conds;
  HostStage h_rows, h_conds;  // their pinned host staging
  SplitBuf ph, pa, pf;
  // the folded LayerNorms' group statistics of the residual rows [M][d/64] (mean, M2)
  DevBuf pst;
  DevBuf gws, gcnt;
  // replay / all-row forward: per-layer scratch K/V (fp32 [n_head][M][64]), key starts,
  // head logits, probe maps, codes and log-probabilities
  DevBuf rk, rv, kstart, plog, pmap, pcodes, plp, pkvs;
  int align_pairs[2][2] = {{4, 10}, {5, 10}};  // (layer, head), align/mod.rs:37
  int n_align = 2;
  // batched decode: residual rows, q rows, split-form rows, attention partials, logits,
  // the per-sequence descriptors and sampling parameters
  DevBuf bx, bq, blog, bseqs, bps;
  SplitBuf bh, ba, bf;
  // sampler API scratch
  DevBuf s_logits, s_seen, s_rng, s_tok;
  int ptype() const { return cfg.param_dtype == ITTS_F32 ? kParamF32 : kParamF16; }
};

struct itts_kv {
  itts_gpt *gpt = nullptr;
  int max_seq = 0;
  int kvt = kKvBf16;
  int valid_len = 0;
  DevBuf k, v;         // [n_layer][n_head][max_seq][64]
  DevBuf ctl;          // DecodeCtl
  DevBuf part;         // attention split partials [n_head][splits][66]
  DevBuf codes;        // generate output
  DecodeCtl *host_ctl = nullptr;  // pinned staging, 2 slots, then the error word's copy
  uint32_t *host_err() const { return reinterpret_cast<uint32_t *>(host_ctl + 2); }
  int splits = 0;
  // persistent decode step: exchange words, split counters + error word, arguments
  bool persist = false;
  DevBuf xch, sync;
  PersistArgs pa{};
  // captured decode iteration (sampler + step), keyed by the sampling parameters
  hipGraphExec_t gexec = nullptr;
  hipGraph_t graph = nullptr;
  DevSampling gkey{};
  bool have_graph = false;
  // timing of the last generate call
  hipEvent_t ev_t[3] = {nullptr, nullptr, nullptr};
  itts_timing timing{};
  bool timing_valid = false;
  size_t layer_elems() const { return (size_t)gpt->cfg.n_head * max_seq * 64; }
  void *k_layer(int l) const {
    return static_cast<char *>(k.p) + layer_elems() * l * (kvt == kKvBf16 ? 2 : 4);
  }
  void *v_layer(int l) const {
    return static_cast<char *>(v.p) + layer_elems() * l * (kvt == kKvBf16 ? 2 : 4);
  }
  ~itts_kv() {
    for (hipEvent_t e : ev_t)
      if (e) (void)hipEventDestroy(e);
    if (gexec) (void)hipGraphExecDestroy(gexec);
    if (graph) (void)hipGraphDestroy(graph);
    if (host_ctl) (void)hipHostFree(host_ctl);
  }
};

namespace {

hipError_t upload(DevBuf &b, const void *src, size_t bytes) {
  hipError_t e = b.ensure(bytes);
  if (e != hipSuccess) return e;
  return hipMemcpy(b.p, src, bytes, hipMemcpyHostToDevice);
}

// Packs scales/biases [N][G] into the device's interleaved (scale, bias) pairs.
std::vector<uint8_t> pack_params(const void *scales, const void *biases, size_t count, bool f32) {
  std::vector<uint8_t> out(count * (f32 ? 8 : 4));
  if (f32) {
    const float *s = static_cast<const float *>(scales), *b = static_cast<const float *>(biases);
    float *o = reinterpret_cast<float *>(out.data());
    for (size_t i = 0; i < count; i++) {
      o[2 * i] = s[i];
      o[2 * i + 1] = b[i];
    }
  } else {
    const uint16_t *s = static_cast<const uint16_t *>(scales), *b = static_cast<const uint16_t *>(biases);
    uint32_t *o = reinterpret_cast<uint32_t *>(out.data());
    for (size_t i = 0; i < count; i++) o[i] = (uint32_t)s[i] | ((uint32_t)b[i] << 16);
  }
  return out;
}

itts_status upload_ql(QLHost &dst, const itts_qlinear &src, int N, int K, int bits, bool f32,
                      const char *name) {
  if (!src.codes || !src.scales || !src.biases || !src.bias)
    return set_error(ITTS_E_WEIGHT, "weight load error in `%s`: missing tensor", name);
  dst.N = N;
  dst.K = K;
  const size_t G = (size_t)K / 64;
  HIP_TRY(upload(dst.codes, src.codes, (size_t)N * K * bits / 8));
  std::vector<uint8_t> pk = pack_params(src.scales, src.biases, (size_t)N * G, f32);
  HIP_TRY(upload(dst.params, pk.data(), pk.size()));
  HIP_TRY(upload(dst.bias, src.bias, sizeof(float) * N));
  return ITTS_OK;
}

itts_status check_vec(const float *p, const char *name) {
  if (!p) return set_error(ITTS_E_WEIGHT, "weight load error in `%s`: missing tensor", name);
  return ITTS_OK;
}

DevSampling to_dev_sampling(const itts_sampling &p, int n) {
  DevSampling d{};
  d.greedy = p.greedy ? 1 : 0;
  d.inv_temp = 1.0f / p.temperature;
  d.top_p = p.top_p;
  d.top_k = p.top_k == 0 ? n : std::min<int>((int)p.top_k, n);
  d.penalty = p.repetition_penalty;
  d.apply_penalty = std::fabs(p.repetition_penalty - 1.0f) <= 1.1920928955078125e-7f ? 0 : 1;
  return d;
}

// Prompts up to this many rows use the per-row attention kernel, longer ones the MFMA
// flash kernel (measured crossover on MI355X at 24 layers x 20 heads).
constexpr int kFlashMinRows = 384;

// GEMM arguments over M rows with the decoder's split-K workspace.
GemmArgs gemm_args(const itts_gpt *g, const DevQL &ql, SplitAct x, int M) {
  GemmArgs ga{};
  ga.ql = ql;
  ga.x = x;
  ga.M = M;
  ga.ws = g->gws.as<float>();
  ga.ws_floats = g->gws.bytes / sizeof(float);
  ga.cnt = g->gcnt.as<uint32_t>();
  ga.cnt_words = kGemmCounters;
  ga.n_cu = g->n_cu;
  return ga;
}

// Grows the per-row buffers of a multi-row forward to M rows.
itts_status ensure_rows(itts_gpt *g, int M) {
  const int d = g->cfg.d_model;
  HIP_TRY(g->px.ensure(sizeof(float) * (size_t)M * d));
  HIP_TRY(g->ph.ensure(M, d));
  HIP_TRY(g->pq.ensure(sizeof(float) * (size_t)M * d));
  HIP_TRY(g->pa.ensure(M, d));
  HIP_TRY(g->pf.ensure(M, g->cfg.d_ffn));
  HIP_TRY(g->pst.ensure(sizeof(float2) * (size_t)M * (d / kGroup)));
  return ITTS_OK;
}

// LayerNorms of the multi-row stacks after layer 0's ln_1 folded into the products: each
// residual product writes gamma * x of the next LayerNorm in split form with the group
// statistics of x (TileFoldOut), and the QKV / c_fc product applies them (TileFoldIn).
// Layer 0's ln_1 input comes from the embeddings and keeps its row kernel.  Used on the
// 64 x 64 tiles (235-row prefill 2.42 -> 2.35 ms on MI355X); on 128 x 128 tiles the fold's
// epilogues cost more than the row kernels (4 x 547 rows: 11.05 -> 11.32 ms), and d <= 2048
// (the statistics' reduction holds at most 32 groups a row).
struct StackFold {
  bool on;
  size_t per;
  const float *fold;
  float2 *st;
  int d, F;
  StackFold(const itts_gpt *g, int M) {
    d = g->cfg.d_model;
    F = g->cfg.d_ffn;
    on = g->fold.p != nullptr && d % kGroup == 0 && d <= 32 * kGroup && M <= kGemmSmallTileRows;
    per = fold_floats(d, F);
    fold = g->fold.as<float>();
    st = g->pst.as<float2>();
  }
  TileFoldIn qkv(int l) const { return TileFoldIn{st, fold + per * l, fold + per * l + 3 * d}; }
  TileFoldIn fc(int l) const { return TileFoldIn{st, fold + per * l + 6 * d, fold + per * l + 6 * d + F}; }
  TileFoldOut out(const SplitBuf &b, const float *gamma) const { return TileFoldOut{b.out(), gamma, st}; }
};

itts_status validate_prefix(const itts_config &c, const int32_t *text, int32_t n_text,
                            const float *conds, int32_t n_cond, int32_t max_cond, int32_t lang,
                            const int32_t *prior, int32_t n_prior);

// Embeds prompts into consecutive row ranges of gpt->px (gpt.rs:535-627 per prompt):
// prompt b occupies rows row0[b] .. row0[b] + T[b] - 1.  Prompts are validated first.
itts_status embed_prompts(itts_gpt *g, const itts_code_prompt *ps, int B, std::vector<int> &row0,
                          std::vector<int> &T, int *M_out) {
  const itts_config &c = g->cfg;
  const int d = c.d_model;
  int M = 0, n_cond_all = 0;
  row0.assign(B, 0);
  T.assign(B, 0);
  for (int b = 0; b < B; b++) {
    const itts_code_prompt &p = ps[b];
    if (itts_status st = validate_prefix(c, p.text_tokens, p.n_text, p.conds, p.n_cond, g->max_cond, p.lang_id,
                                         p.prior_codes, p.n_prior))
      return st;
    row0[b] = M;
    T[b] = p.n_cond + p.n_text + 3 + p.n_prior;
    M += T[b];
    n_cond_all += p.n_cond;
  }
  std::vector<EmbedRow> rows;
  rows.reserve(M);
  int cbase = 0;
  for (int b = 0; b < B; b++) {
    const itts_code_prompt &p = ps[b];
    for (int i = 0; i < p.n_cond; i++) rows.push_back({0, cbase + i, 0});
    for (int j = 0; j < p.n_text + 2; j++) {
      const int u = j == 0 ? 0 : (j == p.n_text + 1 ? 1 : p.text_tokens[j - 1]);
      rows.push_back({1, u, j});
    }
    rows.push_back({2, c.mel_vocab - 2, 0});
    for (int i = 0; i < p.n_prior; i++) rows.push_back({2, p.prior_codes[i], i + 2});
    cbase += p.n_cond;
  }
  if (itts_status st = ensure_rows(g, M)) return st;
  HIP_TRY(g->rows.ensure(sizeof(EmbedRow) * (size_t)M));
  HIP_TRY(g->conds.ensure(sizeof(float) * (size_t)std::max(1, n_cond_all) * d));
  // through pinned staging, so that the copies are asynchronous and the call need not wait
  // for them before it enqueues the stack
  HIP_TRY(g->h_rows.acquire(sizeof(EmbedRow) * (size_t)M));
  HIP_TRY(g->h_conds.acquire(sizeof(float) * (size_t)std::max(1, n_cond_all) * d));
  memcpy(g->h_rows.p, rows.data(), sizeof(EmbedRow) * M);
  HIP_TRY(hipMemcpyAsync(g->rows.p, g->h_rows.p, sizeof(EmbedRow) * M, hipMemcpyHostToDevice, g->stream));
  cbase = 0;
  for (int b = 0; b < B; b++) {
    const itts_code_prompt &p = ps[b];
    if (p.n_cond > 0) {
      float *hc = g->h_conds.as<float>() + (size_t)cbase * d;
      memcpy(hc, p.conds, sizeof(float) * (size_t)p.n_cond * d);
      HIP_TRY(hipMemcpyAsync(g->conds.as<float>() + (size_t)cbase * d, hc, sizeof(float) * (size_t)p.n_cond * d,
                             hipMemcpyHostToDevice, g->stream));
    }
    HIP_TRY(launch_embed_rows(g->rows.as<EmbedRow>() + row0[b], T[b], g->conds.as<float>(), g->text_emb.as<float>(),
                              g->lang_emb.as<float>() + (size_t)p.lang_id * d, g->text_pos.as<float>(),
                              g->mel_emb.as<float>(), g->mel_pos.as<float>(), d,
                              g->px.as<float>() + (size_t)row0[b] * d, g->stream));
    cbase += p.n_cond;
  }
  HIP_TRY(g->h_rows.release(g->stream));
  HIP_TRY(g->h_conds.release(g->stream));
  *M_out = M;
  return ITTS_OK;
}

// Enqueues the stack over the rows already embedded in gpt->px (prefill, T rows at
// cache positions 0..T-1) and the head of the last row into gpt->logits.
itts_status enqueue_prefill_stack(itts_gpt *g, itts_kv *kv, int T) {
  const itts_config &c = g->cfg;
  const int d = c.d_model, bits = c.quant_bits, pt = g->ptype();
  hipStream_t s = g->stream;
  float *X = g->px.as<float>(), *Q = g->pq.as<float>();
  auto gemm = [&](const DevQL &ql, SplitAct x) { return gemm_args(g, ql, x, T); };
  const StackFold sf(g, T);
  for (int l = 0; l < c.n_layer; l++) {
    const DevLayer &L = g->layers[l];
    if (!sf.on || l == 0) HIP_TRY(launch_ln_rows(X, L.ln1_w, L.ln1_b, T, d, g->ph.out(), s));
    GemmArgs ga = gemm(L.attn, g->ph.act());
    if (sf.on && l > 0) ga.tfi = sf.qkv(l);
    ga.qkv = QkvDst{Q, kv->k_layer(l), kv->v_layer(l), kv->max_seq, 0, d};
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiQKV, kv->kvt, s));
    if (T <= kFlashMinRows) {  // few query tiles: one block per (head, row) spreads wider
      HIP_TRY(launch_attn_prefill(Q, T, 0, kv->k_layer(l), kv->v_layer(l), c.n_head, kv->max_seq, g->pa.out(),
                                  kv->kvt, s));
    } else {
      HIP_TRY(launch_attn_flash(Q, T, 0, nullptr, kv->k_layer(l), kv->v_layer(l), kv->max_seq, c.n_head,
                                g->pa.out(), kv->kvt, s));
    }
    ga = gemm(L.proj, g->pa.act());
    ga.y = X;
    if (sf.on) ga.tfo = sf.out(g->ph, L.ln2_w);
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiResid, kv->kvt, s));
    if (!sf.on) HIP_TRY(launch_ln_rows(X, L.ln2_w, L.ln2_b, T, d, g->ph.out(), s));
    ga = gemm(L.fc, g->ph.act());
    if (sf.on) ga.tfi = sf.fc(l);
    ga.xo = g->pf.out();
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiGelu, kv->kvt, s));
    ga = gemm(L.mproj, g->pf.act());
    ga.y = X;
    if (sf.on && l + 1 < c.n_layer) ga.tfo = sf.out(g->ph, g->layers[l + 1].ln1_w);
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiResid, kv->kvt, s));
  }
  GemvArgs ha{};
  ha.ql = g->head;
  ha.x = X + (size_t)(T - 1) * d;
  ha.ln_w = g->ln_f_w.as<float>();
  ha.ln_b = g->ln_f_b.as<float>();
  ha.ln2_w = g->fn_w.as<float>();
  ha.ln2_b = g->fn_b.as<float>();
  ha.y = g->logits.as<float>();
  HIP_TRY(launch_gemv(ha, bits, pt, kProLNLN, kEpiStore, kv->kvt, s));
  return ITTS_OK;
}

// Enqueues one decode step driven by kv->ctl (token, position and cache length read on
// the device): logits land in gpt->logits and ctl->valid_len advances.
// Persistent decode steps of different decoders must not run at the same time.  A step's
// blocks wait for each other's exchange words and assume that together they hold every
// compute unit; two steps dispatched together from two streams could each get part of the
// chip and wait for blocks that cannot start before the other step ends (the bounded waits
// would then fail both).  Persistent launches are therefore chained per device: a launch on
// a stream other than the previous launch's first waits for that launch's completion
// event, and every launch records the event.  Steps of one decoder share its stream and
// are ordered by it already.
struct PersistChain {
  std::mutex mu;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
};
PersistChain g_persist_chain[kMaxDevices];

// Runs launch() (work on g->stream that contains persistent launches) ordered after every
// earlier persistent launch of another decoder on the device.
template <class F>
itts_status persist_chained(itts_gpt *g, F launch) {
  PersistChain &ch = g_persist_chain[g->device];
  std::lock_guard<std::mutex> lock(ch.mu);
  if (!ch.done) HIP_TRY(hipEventCreateWithFlags(&ch.done, hipEventDisableTiming));
  if (ch.last && ch.last != g->stream) HIP_TRY(hipStreamWaitEvent(g->stream, ch.done, 0));
  HIP_TRY(launch());
  HIP_TRY(hipEventRecord(ch.done, g->stream));
  ch.last = g->stream;
  return ITTS_OK;
}

itts_status launch_persist_chained(itts_gpt *g, itts_kv *kv) {
  return persist_chained(g, [&] { return launch_decode_persist(kv->pa, g->cfg.quant_bits, g->ptype(), g->stream); });
}

itts_status enqueue_decode_step(itts_gpt *g, itts_kv *kv) {
  if (kv->persist) return launch_persist_chained(g, kv);
  const itts_config &c = g->cfg;
  const int d = c.d_model, bits = c.quant_bits, pt = g->ptype();
  hipStream_t s = g->stream;
  DecodeCtl *ctl = kv->ctl.as<DecodeCtl>();
  float *x = g->x.as<float>(), *q = g->q.as<float>(), *f = g->f.as<float>();
  for (int l = 0; l < c.n_layer; l++) {
    const DevLayer &L = g->layers[l];
    GemvArgs ga{};
    ga.ql = L.attn;
    ga.x = x;
    ga.ln_w = L.ln1_w;
    ga.ln_b = L.ln1_b;
    ga.qkv = QkvDst{q, kv->k_layer(l), kv->v_layer(l), kv->max_seq, 0, d};
    ga.ctl = ctl;
    if (l == 0) {  // the step embedding is the prologue of layer 0's QKV projection
      ga.emb_tok = g->mel_emb.as<float>();
      ga.emb_pos = g->mel_pos.as<float>();
      ga.x_out = x;
    }
    HIP_TRY(launch_gemv(ga, bits, pt, l == 0 ? kProEmbedLN : kProLN, kEpiQKV, kv->kvt, s));
    HIP_TRY(launch_attn_decode(q, kv->k_layer(l), kv->v_layer(l), c.n_head, kv->max_seq, ctl, 0,
                               kv->part.as<float>(), kv->kvt, s));
    ga = GemvArgs{};
    ga.ql = L.proj;
    ga.attn = AttnPartials{kv->part.as<float>(), c.n_head, kv->splits, 0};
    ga.y = x;
    ga.ctl = ctl;
    HIP_TRY(launch_gemv(ga, bits, pt, kProAttn, kEpiResid, kv->kvt, s));
    ga = GemvArgs{};
    ga.ql = L.fc;
    ga.x = x;
    ga.ln_w = L.ln2_w;
    ga.ln_b = L.ln2_b;
    ga.y = f;
    ga.ctl = ctl;
    HIP_TRY(launch_gemv(ga, bits, pt, kProLN, kEpiGelu, kv->kvt, s));
    ga = GemvArgs{};
    ga.ql = L.mproj;
    ga.x = f;
    ga.y = x;
    ga.ctl = ctl;
    HIP_TRY(launch_gemv(ga, bits, pt, kProNone, kEpiResid, kv->kvt, s));
  }
  GemvArgs ha{};
  ha.ql = g->head;
  ha.x = x;
  ha.ln_w = g->ln_f_w.as<float>();
  ha.ln_b = g->ln_f_b.as<float>();
  ha.ln2_w = g->fn_w.as<float>();
  ha.ln2_b = g->fn_b.as<float>();
  ha.y = g->logits.as<float>();
  ha.ctl = ctl;
  ha.finish = ctl;
  HIP_TRY(launch_gemv(ha, bits, pt, kProLNLN, kEpiStore, kv->kvt, s));
  return ITTS_OK;
}

itts_status validate_prefix(const itts_config &c, const int32_t *text, int32_t n_text,
                            const float *conds, int32_t n_cond, int32_t max_cond, int32_t lang,
                            const int32_t *prior, int32_t n_prior) {
  // gpt.rs:536-560 (prefix_embedding) and 605-613 (sequence_embedding), in that order
  if (n_prior < 0 || n_prior + 3 > c.mel_pos_len)
    return set_error(ITTS_E_VALIDATION, "codes: %d codes exceed the Mel positional capacity", n_prior);
  if (n_text <= 0 || !text) return set_error(ITTS_E_VALIDATION, "text_tokens: text_tokens must not be empty");
  if (n_text + 2 > c.text_pos_len)
    return set_error(ITTS_E_VALIDATION, "text_tokens: text sequence length %d exceeds %d", n_text + 2,
                     c.text_pos_len);
  if (n_cond < 0 || n_cond > max_cond || (n_cond > 0 && !conds))
    return set_error(ITTS_E_VALIDATION, "conds: expected 0..=%d rows of %d, got %d", max_cond, c.d_model,
                     n_cond);
  if (lang < 0 || lang >= c.lang_vocab)
    return set_error(ITTS_E_VALIDATION, "lang_id: lang_id %d out of range 0..%d", lang, c.lang_vocab);
  for (int i = 0; i < n_text; i++)
    if (text[i] < 0 || text[i] >= c.text_vocab)
      return set_error(ITTS_E_VALIDATION, "text_tokens: id %d out of range 0..%d", text[i], c.text_vocab);
  if (n_prior > 0 && !prior) return set_error(ITTS_E_VALIDATION, "codes: null prior codes");
  for (int i = 0; i < n_prior; i++)
    if (prior[i] < 0 || prior[i] >= c.mel_vocab)
      return set_error(ITTS_E_VALIDATION, "codes: id %d out of range 0..%d", prior[i], c.mel_vocab);
  return ITTS_OK;
}

// Embeds the prefill rows into gpt->px and runs the stack; on success the cache holds T
// rows and gpt->logits the next-token logits.  The cache is reset first (gpt.rs:664).
itts_status run_prefill(itts_gpt *g, itts_kv *kv, const int32_t *text, int32_t n_text,
                        const float *conds, int32_t n_cond, int32_t lang, const int32_t *prior,
                        int32_t n_prior, int *T_out) {
  const itts_config &c = g->cfg;
  itts_status st = validate_prefix(c, text, n_text, conds, n_cond, g->max_cond, lang, prior, n_prior);
  if (st) return st;
  const int T = n_cond + n_text + 3 + n_prior;
  kv->valid_len = 0;
  if (T > kv->max_seq)
    return set_error(ITTS_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d", T,
                     kv->max_seq);
  const itts_code_prompt p{text, n_text, conds, n_cond, lang, prior, n_prior, 0};
  std::vector<int> row0, Tb;
  int M = 0;
  if ((st = embed_prompts(g, &p, 1, row0, Tb, &M))) return st;
  st = enqueue_prefill_stack(g, kv, T);
  if (st) return st;
  kv->valid_len = T;
  *T_out = T;
  return ITTS_OK;
}

// A requested attention export: probabilities of (layer, head) for the query rows q0..
// over the key columns [k0, k1), into device memory.
struct ProbeSpec {
  int layer, head, q0, k0, k1;
  float *out;
};

// Runs n_layers blocks over the M rows in gpt->px (row r attends to keys kstart[r]..r)
// with fp32 scratch K/V for one layer at a time, filling the probes on the way.
itts_status forward_rows_stack(itts_gpt *g, int M, const std::vector<int> &kstart, int n_layers,
                               const std::vector<ProbeSpec> &probes) {
  const itts_config &c = g->cfg;
  const int d = c.d_model, bits = c.quant_bits, pt = g->ptype();
  hipStream_t s = g->stream;
  HIP_TRY(g->rk.ensure(sizeof(float) * (size_t)M * d));
  HIP_TRY(g->pkvs.ensure(sizeof(uint16_t) * attn_kv_split_halves(c.n_head, M)));
  HIP_TRY(g->rv.ensure(sizeof(float) * (size_t)M * d));
  // kstart, then the attention's query tiles (64 rows) ordered by their key count, most first
  const int n_tiles = (M + 63) / 64;
  std::vector<int> ks_order(kstart);
  ks_order.resize((size_t)M + n_tiles);
  {
    std::vector<int> keys(n_tiles);
    for (int i = 0; i < n_tiles; i++) keys[i] = std::min(M - 1, 64 * i + 63) - kstart[64 * i] + 1;
    int *order = ks_order.data() + M;
    for (int i = 0; i < n_tiles; i++) order[i] = i;
    std::stable_sort(order, order + n_tiles, [&](int a, int b) { return keys[a] > keys[b]; });
  }
  HIP_TRY(g->kstart.ensure(sizeof(int) * ks_order.size()));
  HIP_TRY(hipMemcpyAsync(g->kstart.p, ks_order.data(), sizeof(int) * ks_order.size(), hipMemcpyHostToDevice, s));
  float *X = g->px.as<float>(), *Q = g->pq.as<float>();
  const StackFold sf(g, M);
  for (int l = 0; l < n_layers; l++) {
    const DevLayer &L = g->layers[l];
    if (!sf.on || l == 0) HIP_TRY(launch_ln_rows(X, L.ln1_w, L.ln1_b, M, d, g->ph.out(), s));
    GemmArgs ga = gemm_args(g, L.attn, g->ph.act(), M);
    if (sf.on && l > 0) ga.tfi = sf.qkv(l);
    ga.qkv = QkvDst{Q, g->rk.p, g->rv.p, M, 0, d};
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiQKV, kKvF32, s));
    for (const ProbeSpec &p : probes)  // read-only exports of this layer's attention
      if (p.layer == l)
        HIP_TRY(launch_attn_probe(Q, M, g->kstart.as<int>(), g->rk.p, g->rv.p, c.n_head,
                                  AttnProbe{p.head, p.q0, p.k0, p.k1, p.out}, kKvF32, s));
    HIP_TRY(launch_attn_flash(Q, M, 0, g->kstart.as<int>(), g->rk.p, g->rv.p, M, c.n_head, g->pa.out(), kKvF32, s,
                              g->pkvs.as<uint16_t>(), g->kstart.as<int>() + M));
    ga = gemm_args(g, L.proj, g->pa.act(), M);
    ga.y = X;
    if (sf.on) ga.tfo = sf.out(g->ph, L.ln2_w);
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiResid, kKvF32, s));
    if (!sf.on) HIP_TRY(launch_ln_rows(X, L.ln2_w, L.ln2_b, M, d, g->ph.out(), s));
    ga = gemm_args(g, L.fc, g->ph.act(), M);
    if (sf.on) ga.tfi = sf.fc(l);
    ga.xo = g->pf.out();
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiGelu, kKvF32, s));
    ga = gemm_args(g, L.mproj, g->pf.act(), M);
    ga.y = X;
    if (sf.on && l + 1 < n_layers) ga.tfo = sf.out(g->ph, g->layers[l + 1].ln1_w);
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiResid, kKvF32, s));
  }
  return ITTS_OK;
}

// Head logits of R rows of gpt->px from row0: ln_f, final_norm, mel_head (gpt.rs:838-846)
// into gpt->plog [R][mel_vocab].
itts_status head_rows(itts_gpt *g, int row0, int R) {
  const itts_config &c = g->cfg;
  const int d = c.d_model;
  HIP_TRY(g->plog.ensure(sizeof(float) * (size_t)R * c.mel_vocab));
  HIP_TRY(launch_ln_rows(g->px.as<float>() + (size_t)row0 * d, g->ln_f_w.as<float>(), g->ln_f_b.as<float>(), R, d,
                         g->ph.out(), g->stream, g->fn_w.as<float>(), g->fn_b.as<float>()));
  GemmArgs ga = gemm_args(g, g->head, g->ph.act(), R);
  ga.y = g->plog.as<float>();
  HIP_TRY(launch_gemm(ga, c.quant_bits, g->ptype(), kEpiStore, kKvF32, g->stream));
  return ITTS_OK;
}

// Shared part of teacher_forced / code_log_probs / alignment_attention (gpt.rs:797-915):
// embeds the prompt with `fed` as prior codes, runs n_layers blocks with the alignment
// probes of queries q0.. over the text columns, and averages the maps into attention_out.
itts_status replay(itts_gpt *g, itts_kv *kv, const int32_t *text, int32_t n_text, const float *conds,
                   int32_t n_cond, int32_t lang, const std::vector<int32_t> &fed, int32_t q0, int n_layers,
                   int n_codes, float *attention_out, int *T_out) {
  const itts_config &c = g->cfg;
  const int T = n_cond + n_text + 3 + (int)fed.size();
  kv->valid_len = 0;  // the cache is scratch (gpt.rs:819, 836)
  const itts_code_prompt p{text, n_text, conds, n_cond, lang, fed.empty() ? nullptr : fed.data(), (int32_t)fed.size(),
                           0};
  if (itts_status st = validate_prefix(c, text, n_text, conds, n_cond, g->max_cond, lang, p.prior_codes, p.n_prior))
    return st;
  if (T > kv->max_seq)
    return set_error(ITTS_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d", T, kv->max_seq);
  std::vector<int> row0, Tb;
  int M = 0;
  if (itts_status st = embed_prompts(g, &p, 1, row0, Tb, &M)) return st;
  const int text_lo = n_cond, text_hi = n_cond + n_text + 2, W = n_text + 2;
  std::vector<ProbeSpec> probes;
  if (attention_out) {
    HIP_TRY(g->pmap.ensure(sizeof(float) * (size_t)g->n_align * n_codes * W));
    for (int i = 0; i < g->n_align; i++)
      probes.push_back({g->align_pairs[i][0], g->align_pairs[i][1], q0, text_lo, text_hi,
                        g->pmap.as<float>() + (size_t)i * n_codes * W});
  }
  if (itts_status st = forward_rows_stack(g, M, std::vector<int>(M, 0), n_layers, probes)) return st;
  if (attention_out) {
    std::vector<float> maps((size_t)g->n_align * n_codes * W);
    HIP_TRY(hipMemcpyAsync(maps.data(), g->pmap.p, sizeof(float) * maps.size(), hipMemcpyDeviceToHost, g->stream));
    HIP_TRY(hipStreamSynchronize(g->stream));
    const size_t n = (size_t)n_codes * W;
    for (size_t i = 0; i < n; i++) {  // mean over the stacked maps (gpt.rs:849-851)
      float acc = maps[i];
      for (int k = 1; k < g->n_align; k++) acc += maps[k * n + i];
      attention_out[i] = acc / (float)g->n_align;
    }
  }
  *T_out = T;
  return ITTS_OK;
}

itts_status check_replay_args(itts_gpt *g, itts_kv *kv, const int32_t *codes, int32_t n_codes) {
  if (!g || !kv || kv->gpt != g) return set_error(ITTS_E_VALIDATION, "kv_cache: cache belongs to another decoder");
  if (n_codes <= 0 || !codes) return set_error(ITTS_E_VALIDATION, "codes: codes must not be empty");
  for (int i = 0; i < n_codes; i++)
    if (codes[i] < 0 || codes[i] >= g->cfg.mel_vocab)
      return set_error(ITTS_E_VALIDATION, "codes: id %d out of range 0..%d", codes[i], g->cfg.mel_vocab);
  return ITTS_OK;
}

// Checks a batch of caches and uploads their descriptors; grows the batch workspace.
itts_status prepare_batch(itts_gpt *g, itts_kv *const *caches, int B) {
  const itts_config &c = g->cfg;
  if (!caches || B <= 0 || B > 64) return set_error(ITTS_E_VALIDATION, "caches: 1..64 caches expected");
  std::vector<BatchSeq> seqs(B);
  for (int b = 0; b < B; b++) {
    itts_kv *kv = caches[b];
    if (!kv || kv->gpt != g) return set_error(ITTS_E_VALIDATION, "kv_cache: cache belongs to another decoder");
    if (kv->max_seq != caches[0]->max_seq || kv->kvt != caches[0]->kvt)
      return set_error(ITTS_E_VALIDATION, "kv_cache: a batch needs caches of one capacity and dtype");
    for (int j = 0; j < b; j++)
      if (caches[j] == kv) return set_error(ITTS_E_VALIDATION, "kv_cache: a cache appears twice in the batch");
    seqs[b] = BatchSeq{kv->ctl.as<DecodeCtl>(), kv->k.p, kv->v.p, kv->codes.as<int32_t>()};
  }
  const int d = c.d_model;
  HIP_TRY(g->bx.ensure(sizeof(float) * (size_t)B * d));
  HIP_TRY(g->bq.ensure(sizeof(float) * (size_t)B * d));
  HIP_TRY(g->bh.ensure(B, d));
  HIP_TRY(g->ba.ensure(B, d));
  HIP_TRY(g->bf.ensure(B, c.d_ffn));
  HIP_TRY(g->blog.ensure(sizeof(float) * (size_t)B * c.mel_vocab));
  HIP_TRY(g->bseqs.ensure(sizeof(BatchSeq) * B));
  HIP_TRY(hipMemcpyAsync(g->bseqs.p, seqs.data(), sizeof(BatchSeq) * B, hipMemcpyHostToDevice, g->stream));
  HIP_TRY(hipStreamSynchronize(g->stream));
  return ITTS_OK;
}

// Enqueues one decode step of the B sequences described in gpt->bseqs (tokens, positions
// and cache lengths read from their control blocks): logits land in gpt->blog [B][V] and
// every unfinished sequence's cache length advances.  The linears run as M = B GEMMs, so
// each weight byte is read once per step for the whole batch.
itts_status enqueue_step_batch(itts_gpt *g, int B, int max_seq, int kvt) {
  const itts_config &c = g->cfg;
  const int d = c.d_model, bits = c.quant_bits, pt = g->ptype();
  hipStream_t s = g->stream;
  const BatchSeq *seqs = g->bseqs.as<BatchSeq>();
  float *X = g->bx.as<float>();
  HIP_TRY(launch_embed_batch(seqs, B, g->mel_emb.as<float>(), g->mel_pos.as<float>(), d, X, s));
  const size_t layer_elems = (size_t)c.n_head * max_seq * 64;
  // ln_1 and ln_2 folded into the products that follow them (no row kernels) where the
  // few-row products take them: up to 8 rows, d a multiple of 256 up to 2048
  const bool fold = g->fold.p && B <= 8 && d % 256 == 0 && d <= 2048;
  const size_t per = fold_floats(d, c.d_ffn);
  for (int l = 0; l < c.n_layer; l++) {
    const DevLayer &L = g->layers[l];
    const float *fo = fold ? g->fold.as<float>() + per * l : nullptr;
    GemmArgs ga = gemm_args(g, L.attn, g->bh.act(), B);
    if (fold)
      ga.fold = FoldIn{X, L.ln1_w, fo, fo + 3 * d};
    else
      HIP_TRY(launch_ln_rows(X, L.ln1_w, L.ln1_b, B, d, g->bh.out(), s));
    ga.qkv = QkvDst{g->bq.as<float>(), nullptr, nullptr, max_seq, 0, d, seqs, layer_elems * l};
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiQKV, kvt, s));
    HIP_TRY(launch_decode_batch_rows(g->bq.as<float>(), seqs, B, layer_elems * l, c.n_head, max_seq, g->ba.out(),
                                     kvt, s));
    ga = gemm_args(g, L.proj, g->ba.act(), B);
    ga.y = X;
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiResid, kvt, s));
    ga = gemm_args(g, L.fc, g->bh.act(), B);
    if (fold)
      ga.fold = FoldIn{X, L.ln2_w, fo + 6 * d, fo + 6 * d + c.d_ffn};
    else
      HIP_TRY(launch_ln_rows(X, L.ln2_w, L.ln2_b, B, d, g->bh.out(), s));
    ga.xo = g->bf.out();
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiGelu, kvt, s));
    ga = gemm_args(g, L.mproj, g->bf.act(), B);
    ga.y = X;
    HIP_TRY(launch_gemm(ga, bits, pt, kEpiResid, kvt, s));
  }
  HIP_TRY(launch_ln_rows(X, g->ln_f_w.as<float>(), g->ln_f_b.as<float>(), B, d, g->bh.out(), s, g->fn_w.as<float>(),
                         g->fn_b.as<float>()));
  GemmArgs ga = gemm_args(g, g->head, g->bh.act(), B);
  ga.y = g->blog.as<float>();
  HIP_TRY(launch_gemm(ga, bits, pt, kEpiStore, kvt, s));
  HIP_TRY(launch_advance_batch(seqs, B, s));
  return ITTS_OK;
}

// Writes the host-known fields of the decode control block (the device-owned step
// counter that follows them is left alone).
itts_status write_ctl(itts_kv *kv, const DecodeCtl &h) {
  *kv->host_ctl = h;
  HIP_TRY(hipMemcpyAsync(kv->ctl.p, kv->host_ctl, offsetof(DecodeCtl, xstep), hipMemcpyHostToDevice,
                         kv->gpt->stream));
  return ITTS_OK;
}

// After the stream has drained: a persistent step whose exchange wait timed out leaves
// the error word set and its step unfinished.  The exchange state is cleared so that the
// cache stays usable, and the call reports a device error.
// The persistent step's error word: its copy to pinned memory enqueued, then read after the
// caller's next synchronisation (persist_err_check).
hipError_t persist_err_enqueue(itts_kv *kv) {
  if (!kv->persist) return hipSuccess;
  return hipMemcpyAsync(kv->host_err(), kv->pa.err, sizeof(uint32_t), hipMemcpyDeviceToHost, kv->gpt->stream);
}
itts_status persist_err_check(itts_kv *kv) {
  if (!kv->persist || *kv->host_err() == 0) return ITTS_OK;
  hipStream_t s = kv->gpt->stream;
  HIP_TRY(hipMemsetAsync(kv->xch.p, 0, kv->xch.bytes, s));
  HIP_TRY(hipMemsetAsync(kv->sync.p, 0, kv->sync.bytes, s));
  // epochs restart with the cleared words (an exchange word keeps 16 epoch bits, so a
  // cleared word must never meet an epoch that is 0 in those bits)
  HIP_TRY(hipMemsetAsync(static_cast<char *>(kv->ctl.p) + offsetof(DecodeCtl, xstep), 0, sizeof(int32_t), s));
  HIP_TRY(hipStreamSynchronize(s));
  return set_error(ITTS_E_DEVICE, "decode step: a persistent-kernel exchange wait timed out");
}
itts_status check_persist(itts_kv *kv) {
  HIP_TRY(persist_err_enqueue(kv));
  HIP_TRY(hipStreamSynchronize(kv->gpt->stream));
  return persist_err_check(kv);
}

// Sets up the persistent decode step for a new cache when the decoder and the cache
// shape allow it.  *used reports whether the cache takes that path.
itts_status setup_persist(itts_gpt *g, itts_kv *kv, bool *used) {
  *used = false;
  const itts_config &c = g->cfg;
  int S = 0;
  const bool shape_ok = g->persist_ok &&
                        persist_supported(c.d_model, c.d_ffn, c.mel_vocab, c.n_head, c.n_layer, kv->max_seq,
                                          g->n_cu, c.quant_bits, &S);
  PersistArgs a{};
  const int d = c.d_model, F = c.d_ffn, H = c.n_head, V = c.mel_vocab, B = g->n_cu;
  if (shape_ok) {
    a.n_layer = c.n_layer;
    a.d = d;
    a.H = H;
    a.F = F;
    a.V = V;
    a.S = S;
    a.B = B;
    auto r4 = [](int n) { return (n + 3) & ~3; };
    auto rows = [&](int N) { return (N + B - 1) / B; };
    const int rq = rows(3 * d), rp = rows(d), rf = rows(F), rh = rows(V);
    const int epc = c.quant_bits == 8 ? 16 : 32;  // codes per 16-byte chunk
    auto padded = [&](int n) { return r4(n + n / epc * 4); };  // 4 floats after each chunk's values
    a.xin_len = padded(std::max(d, F));
    a.xn_len = padded(d);
    a.part_len = r4(std::max({rq * (d / epc), rp * (d / epc), rf * (d / epc), rp * (F / epc), rh * (d / epc)}));
    a.own_len = r4(rp);
    a.out_len = r4(std::max({rq, rp, rf, rh}));
    a.pp_len = r4(S * 66);
    a.lp_len = r4(std::max(2 * d + 2 * rq + rp + 2 * rf + rp, 4 * d + rh));  // stage_params_dma
    a.kvt = kv->kvt;
    // f32 rows: V of a split is staged over the input row, normalised row and partials
    if (kv->kvt == kKvF32)
      a.part_len = std::max(a.part_len, r4(persist_f32_v_floats(kv->max_seq, S) - a.xin_len - a.xn_len));
  }
  bool ok = shape_ok && persist_lds_bytes(a) <= kPersistMaxLds;
  if (ok) HIP_TRY(persist_fits(c.quant_bits, g->ptype(), kv->kvt, persist_lds_bytes(a), &ok));  // one block per CU
  if (g->path == ITTS_DECODE_PERSISTENT && !ok)
    return set_error(ITTS_E_VALIDATION,
                     "decode_path: the persistent decode step does not support this cache (%s rows, "
                     "max_seq %d, %d compute units)",
                     kv->kvt == kKvBf16 ? "bf16" : "f32", kv->max_seq, B);
  if (!ok || g->path == ITTS_DECODE_MULTI) return ITTS_OK;
  size_t off[6];
  const size_t words = persist_exchange_words(d, F, H, S, B, off);
  const size_t sync_words = (size_t)H * kCntStride + 64;
  HIP_TRY(kv->xch.ensure(words * 16));
  HIP_TRY(kv->sync.ensure(sync_words * sizeof(uint32_t)));
  HIP_TRY(hipMemsetAsync(kv->xch.p, 0, kv->xch.bytes, g->stream));
  HIP_TRY(hipMemsetAsync(kv->sync.p, 0, kv->sync.bytes, g->stream));
  char *x = static_cast<char *>(kv->xch.p);
  a.x_x = x + off[0] * 16;
  a.x_qkv = x + off[1] * 16;
  a.x_part = x + off[2] * 16;
  a.x_attn = x + off[3] * 16;
  a.x_mid = x + off[4] * 16;
  a.x_f = x + off[5] * 16;
  a.cnt = kv->sync.as<uint32_t>();
  a.err = a.cnt + (size_t)H * kCntStride;
  a.layers = g->dlayers.as<DevLayer>();
  a.head = g->head;
  a.ln_f_w = g->ln_f_w.as<float>();
  a.ln_f_b = g->ln_f_b.as<float>();
  a.fn_w = g->fn_w.as<float>();
  a.fn_b = g->fn_b.as<float>();
  a.fold = g->fold.as<float>();
  a.mel_emb = g->mel_emb.as<float>();
  a.mel_pos = g->mel_pos.as<float>();
  a.kc = kv->k.p;
  a.vc = kv->v.p;
  a.max_seq = kv->max_seq;
  a.ctl = kv->ctl.as<DecodeCtl>();
  a.logits = g->logits.as<float>();
  a.ep_stride = 8u * (uint32_t)(c.n_layer + 1);
  kv->pa = a;
  *used = true;
  return ITTS_OK;
}

}  // namespace

// ------------------------------------------------------------------------------------
// C ABI
// ------------------------------------------------------------------------------------

extern "C" {

const char *itts_version(void) { return "libitts_hip 0.1.0 (gfx950)"; }

const char *itts_last_error(void) { return g_last_error.c_str(); }

itts_config itts_config_default(void) {
  itts_config c{};
  c.n_layer = 24;
  c.d_model = 1280;
  c.n_head = 20;
  c.d_ffn = 5120;
  c.mel_vocab = 8194;
  c.text_vocab = 60510;
  c.lang_vocab = 107;
  c.mel_pos_len = 1818;
  c.text_pos_len = 602;
  c.quant_bits = 8;
  c.param_dtype = ITTS_F16;
  return c;
}

itts_sampling itts_sampling_default(void) {
  itts_sampling p{};
  p.greedy = 0;
  p.temperature = 0.8f;
  p.top_p = 0.8f;
  p.top_k = 3;
  p.repetition_penalty = 10.0f;
  p.max_mel_tokens = 1500;
  return p;
}

itts_status itts_sampling_validate(const itts_sampling *p) {
  if (!p) return set_error(ITTS_E_VALIDATION, "sampling: null");
  if (!std::isfinite(p->temperature) || !(p->temperature >= 0.05f && p->temperature <= 2.0f))
    return set_error(ITTS_E_VALIDATION, "temperature: must be finite and in 0.05..=2.0, got %g",
                     (double)p->temperature);
  if (!std::isfinite(p->top_p) || !(p->top_p >= 0.01f && p->top_p <= 1.0f))
    return set_error(ITTS_E_VALIDATION, "top_p: must be finite and in 0.01..=1.0, got %g", (double)p->top_p);
  if (p->top_k > 8194) return set_error(ITTS_E_VALIDATION, "top_k: must be <= 8194, got %u", p->top_k);
  if (!std::isfinite(p->repetition_penalty) ||
      !(p->repetition_penalty >= 1.0f && p->repetition_penalty <= 50.0f))
    return set_error(ITTS_E_VALIDATION, "repetition_penalty: must be finite and in 1.0..=50.0, got %g",
                     (double)p->repetition_penalty);
  if (p->max_mel_tokens < 1 || p->max_mel_tokens > 1815)
    return set_error(ITTS_E_VALIDATION, "max_mel_tokens: must be in 1..=1815, got %u", p->max_mel_tokens);
  return ITTS_OK;
}

itts_status itts_gpt_create(const itts_weights *w, itts_gpt **out) {
  if (!w || !out) return set_error(ITTS_E_VALIDATION, "weights: null argument");
  std::string why;
  if (!valid_config(w->config, why)) return set_error(ITTS_E_WEIGHT, "weight load error in `config`: %s", why.c_str());
  auto *g = new itts_gpt();
  g->cfg = w->config;
  const itts_config &c = g->cfg;
  const int d = c.d_model, F = c.d_ffn, bits = c.quant_bits;
  const bool f32 = c.param_dtype == ITTS_F32;
  auto fail = [&](itts_status st) {
    delete g;
    return st;
  };
  if (hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking) != hipSuccess)
    return fail(set_error(ITTS_E_DEVICE, "hipStreamCreate failed"));
  if (sampler_init() != hipSuccess) return fail(set_error(ITTS_E_DEVICE, "sampler LDS attribute failed"));
  if (const char *ng = getenv("ITTS_NO_GRAPH")) g->use_graph = !(ng[0] == '1' && ng[1] == '\0');
  struct {
    const float *p;
    const char *name;
    DevBuf *dst;
    size_t n;
  } tabs[] = {
      {w->text_embedding, "text_embedding.weight", &g->text_emb, (size_t)c.text_vocab * d},
      {w->lang_embedding, "lang_embedding.weight", &g->lang_emb, (size_t)c.lang_vocab * d},
      {w->mel_embedding, "mel_embedding.weight", &g->mel_emb, (size_t)c.mel_vocab * d},
      {w->mel_pos_embedding, "mel_pos_embedding.emb.weight", &g->mel_pos, (size_t)c.mel_pos_len * d},
      {w->text_pos_embedding, "text_pos_embedding.emb.weight", &g->text_pos, (size_t)c.text_pos_len * d},
      {w->ln_f_w, "gpt.ln_f.weight", &g->ln_f_w, (size_t)d},
      {w->ln_f_b, "gpt.ln_f.bias", &g->ln_f_b, (size_t)d},
      {w->final_norm_w, "final_norm.weight", &g->fn_w, (size_t)d},
      {w->final_norm_b, "final_norm.bias", &g->fn_b, (size_t)d},
  };
  for (auto &t : tabs) {
    if (itts_status st = check_vec(t.p, t.name)) return fail(st);
    if (upload(*t.dst, t.p, sizeof(float) * t.n) != hipSuccess)
      return fail(set_error(ITTS_E_DEVICE, "upload of `%s` failed", t.name));
  }
  if (!w->layers) return fail(set_error(ITTS_E_WEIGHT, "weight load error in `gpt.h`: missing layers"));
  g->ln.resize((size_t)c.n_layer * 4);
  g->qls.resize((size_t)c.n_layer * 4 + 1);
  g->layers.resize(c.n_layer);
  char name[128];
  for (int l = 0; l < c.n_layer; l++) {
    const itts_layer_weights &L = w->layers[l];
    const float *lnp[4] = {L.ln1_w, L.ln1_b, L.ln2_w, L.ln2_b};
    const char *lnn[4] = {"ln_1.weight", "ln_1.bias", "ln_2.weight", "ln_2.bias"};
    for (int i = 0; i < 4; i++) {
      snprintf(name, sizeof name, "gpt.h.%d.%s", l, lnn[i]);
      if (itts_status st = check_vec(lnp[i], name)) return fail(st);
      if (upload(g->ln[l * 4 + i], lnp[i], sizeof(float) * d) != hipSuccess)
        return fail(set_error(ITTS_E_DEVICE, "upload of `%s` failed", name));
    }
    const itts_qlinear *qs[4] = {&L.c_attn, &L.c_proj, &L.c_fc, &L.mlp_c_proj};
    const int Ns[4] = {3 * d, d, F, d}, Ks[4] = {d, d, d, F};
    const char *qn[4] = {"attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"};
    for (int i = 0; i < 4; i++) {
      snprintf(name, sizeof name, "gpt.h.%d.%s", l, qn[i]);
      if (itts_status st = upload_ql(g->qls[l * 4 + i], *qs[i], Ns[i], Ks[i], bits, f32, name)) return fail(st);
    }
    DevLayer &D = g->layers[l];
    D.ln1_w = g->ln[l * 4].as<float>();
    D.ln1_b = g->ln[l * 4 + 1].as<float>();
    D.ln2_w = g->ln[l * 4 + 2].as<float>();
    D.ln2_b = g->ln[l * 4 + 3].as<float>();
    D.attn = g->qls[l * 4].dev();
    D.proj = g->qls[l * 4 + 1].dev();
    D.fc = g->qls[l * 4 + 2].dev();
    D.mproj = g->qls[l * 4 + 3].dev();
  }
  QLHost &hq = g->qls[(size_t)c.n_layer * 4];
  if (itts_status st = upload_ql(hq, w->mel_head, c.mel_vocab, d, bits, f32, "mel_head")) return fail(st);
  g->head = hq.dev();
  if (upload(g->dlayers, g->layers.data(), sizeof(DevLayer) * c.n_layer) != hipSuccess)
    return fail(set_error(ITTS_E_DEVICE, "upload of the layer table failed"));
  {
    int dev = 0, coop = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices ||
        hipDeviceGetAttribute(&g->n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev) != hipSuccess)
      return fail(set_error(ITTS_E_DEVICE, "device attribute query failed"));
    g->device = dev;
    g->persist_ok = (bits == 8 || bits == 4) && coop != 0 && persist_init() == hipSuccess;
    if (bits == 8 || bits == 4) {  // G and c of the products that follow ln_1 and ln_2
      const size_t per = fold_floats(d, F);
      if (g->fold.ensure(sizeof(float) * per * c.n_layer) != hipSuccess)
        return fail(set_error(ITTS_E_DEVICE, "fold buffer allocation failed"));
      for (int l = 0; l < c.n_layer; l++) {
        const DevLayer &D = g->layers[l];
        float *fo = g->fold.as<float>() + per * l;
        if (launch_ln_fold(D.attn, bits, g->ptype(), D.ln1_w, D.ln1_b, fo, fo + 3 * d, g->stream) != hipSuccess ||
            launch_ln_fold(D.fc, bits, g->ptype(), D.ln2_w, D.ln2_b, fo + 6 * d, fo + 6 * d + F, g->stream) !=
                hipSuccess)
          return fail(set_error(ITTS_E_DEVICE, "LayerNorm fold launch failed"));
      }
      if (hipStreamSynchronize(g->stream) != hipSuccess)
        return fail(set_error(ITTS_E_DEVICE, "LayerNorm fold failed"));
    }
    if (sampler_stage_init(dev) != hipSuccess)
      return fail(set_error(ITTS_E_DEVICE, "sampler staging area lookup failed"));
  }
  if (g->gws.ensure(sizeof(float) * gemm_ws_floats(g->n_cu)) || g->gcnt.ensure(sizeof(uint32_t) * kGemmCounters) ||
      hipMemset(g->gcnt.p, 0, sizeof(uint32_t) * kGemmCounters) || gemm_init() != hipSuccess)
    return fail(set_error(ITTS_E_DEVICE, "GEMM workspace allocation failed"));
  if (g->x.ensure(sizeof(float) * d) || g->q.ensure(sizeof(float) * d) || g->a.ensure(sizeof(float) * d) ||
      g->f.ensure(sizeof(float) * F) || g->logits.ensure(sizeof(float) * c.mel_vocab))
    return fail(set_error(ITTS_E_DEVICE, "workspace allocation failed"));
  *out = g;
  return ITTS_OK;
}

static void gpt_release(itts_gpt *gpt) {
  if (--gpt->refs > 0) return;
  if (gpt->stream) {
    (void)hipStreamSynchronize(gpt->stream);
    {
      // a later decoder's stream may reuse this handle value: forget it as the last
      // persistent launcher (its work has drained)
      PersistChain &ch = g_persist_chain[gpt->device];
      std::lock_guard<std::mutex> lock(ch.mu);
      if (ch.last == gpt->stream) ch.last = nullptr;
    }
    (void)hipStreamDestroy(gpt->stream);
  }
  delete gpt;
}

void itts_gpt_destroy(itts_gpt *gpt) {
  if (!gpt || gpt->user_released) return;
  gpt->user_released = true;
  gpt_release(gpt);
}

int32_t itts_gpt_num_layers(const itts_gpt *gpt) { return gpt ? gpt->cfg.n_layer : 0; }
itts_config itts_gpt_config(const itts_gpt *gpt) { return gpt ? gpt->cfg : itts_config{}; }
int32_t itts_gpt_max_cond(const itts_gpt *gpt) { return gpt ? gpt->max_cond : 0; }
void *itts_gpt_stream(const itts_gpt *gpt) { return gpt ? (void *)gpt->stream : nullptr; }

itts_status itts_gpt_set_decode_path(itts_gpt *gpt, itts_decode_path path) {
  if (!gpt) return set_error(ITTS_E_VALIDATION, "decode_path: null decoder");
  if (path != ITTS_DECODE_AUTO && path != ITTS_DECODE_MULTI && path != ITTS_DECODE_PERSISTENT)
    return set_error(ITTS_E_VALIDATION, "decode_path: unknown path %d", (int)path);
  if (path == ITTS_DECODE_PERSISTENT && !gpt->persist_ok)
    return set_error(ITTS_E_VALIDATION,
                     "decode_path: the persistent decode step needs 8-bit codes and cooperative launch");
  gpt->path = path;
  return ITTS_OK;
}

itts_status itts_kv_create(itts_gpt *gpt, int32_t max_seq, itts_dtype kv_dtype, itts_kv **out) {
  if (!gpt || !out) return set_error(ITTS_E_VALIDATION, "kv_cache: null argument");
  if (max_seq <= 0) return set_error(ITTS_E_VALIDATION, "max_seq: KV cache max_seq must be >= 1");
  if (kv_dtype != ITTS_BF16 && kv_dtype != ITTS_F32)
    return set_error(ITTS_E_VALIDATION, "kv_dtype: must be BF16 or F32");
  auto *kv = new itts_kv();
  kv->gpt = gpt;
  kv->max_seq = max_seq;
  kv->kvt = kv_dtype == ITTS_BF16 ? kKvBf16 : kKvF32;
  const size_t es = kv->kvt == kKvBf16 ? 2 : 4;
  const size_t n = (size_t)gpt->cfg.n_layer * kv->layer_elems();
  kv->splits = attn_decode_max_splits(max_seq);
  if (kv->k.ensure(n * es) || kv->v.ensure(n * es) || kv->ctl.ensure(sizeof(DecodeCtl)) ||
      kv->part.ensure(sizeof(float) * (size_t)gpt->cfg.n_head * kv->splits * 66) ||
      kv->codes.ensure(sizeof(int32_t) * 2048) ||
      hipHostMalloc((void **)&kv->host_ctl, 2 * sizeof(DecodeCtl) + 64, hipHostMallocDefault) != hipSuccess) {
    delete kv;
    return set_error(ITTS_E_DEVICE, "KV cache allocation of %zu bytes failed", 2 * n * es);
  }
  if (hipMemsetAsync(kv->k.p, 0, n * es, gpt->stream) != hipSuccess ||
      hipMemsetAsync(kv->v.p, 0, n * es, gpt->stream) != hipSuccess ||
      hipMemsetAsync(kv->ctl.p, 0, sizeof(DecodeCtl), gpt->stream) != hipSuccess) {
    delete kv;
    return set_error(ITTS_E_DEVICE, "KV cache initialisation failed");
  }
  if (itts_status st = setup_persist(gpt, kv, &kv->persist)) {
    (void)hipStreamSynchronize(gpt->stream);
    delete kv;
    return st;
  }
  if (hipStreamSynchronize(gpt->stream) != hipSuccess) {
    delete kv;
    return set_error(ITTS_E_DEVICE, "KV cache initialisation failed");
  }
  gpt->refs += 1;
  *out = kv;
  return ITTS_OK;
}

void itts_kv_destroy(itts_kv *kv) {
  if (!kv) return;
  itts_gpt *gpt = kv->gpt;
  (void)hipStreamSynchronize(gpt->stream);
  delete kv;
  gpt_release(gpt);
}

void itts_kv_reset(itts_kv *kv) {
  if (kv) kv->valid_len = 0;
}
int32_t itts_kv_valid_len(const itts_kv *kv) { return kv ? kv->valid_len : 0; }
int32_t itts_kv_max_seq(const itts_kv *kv) { return kv ? kv->max_seq : 0; }
itts_decode_path itts_kv_decode_path(const itts_kv *kv) {
  return kv && kv->persist ? ITTS_DECODE_PERSISTENT : ITTS_DECODE_MULTI;
}

itts_status itts_kv_read(const itts_kv *kv, int32_t layer, int32_t which_v, float *out) {
  if (!kv || !out) return set_error(ITTS_E_VALIDATION, "kv_cache: null argument");
  const itts_config &c = kv->gpt->cfg;
  if (layer < 0 || layer >= c.n_layer) return set_error(ITTS_E_VALIDATION, "layer: out of range");
  HIP_TRY(hipStreamSynchronize(kv->gpt->stream));
  const size_t es = kv->kvt == kKvBf16 ? 2 : 4;
  std::vector<uint8_t> tmp((size_t)kv->valid_len * 64 * es);
  for (int h = 0; h < c.n_head; h++) {
    const char *src = static_cast<const char *>(which_v ? kv->v_layer(layer) : kv->k_layer(layer)) +
                      (size_t)h * kv->max_seq * 64 * es;
    if (kv->valid_len == 0) continue;
    HIP_TRY(hipMemcpy(tmp.data(), src, tmp.size(), hipMemcpyDeviceToHost));
    float *dst = out + (size_t)h * kv->valid_len * 64;
    for (size_t i = 0; i < (size_t)kv->valid_len * 64; i++) {
      if (es == 2) {
        uint32_t b = (uint32_t)reinterpret_cast<const uint16_t *>(tmp.data())[i] << 16;
        memcpy(&dst[i], &b, 4);
      } else {
        dst[i] = reinterpret_cast<const float *>(tmp.data())[i];
      }
    }
  }
  return ITTS_OK;
}

itts_status itts_gpt_prefill_after(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens,
                                   int32_t n_text, const float *conds, int32_t n_cond,
                                   int32_t lang_id, const int32_t *prior_codes, int32_t n_prior,
                                   float *logits_out) {
  if (!gpt || !kv || kv->gpt != gpt) return set_error(ITTS_E_VALIDATION, "kv_cache: cache belongs to another decoder");
  int T = 0;
  itts_status st = run_prefill(gpt, kv, text_tokens, n_text, conds, n_cond, lang_id, prior_codes, n_prior, &T);
  if (st) return st;
  if (logits_out)
    HIP_TRY(hipMemcpyAsync(logits_out, gpt->logits.p, sizeof(float) * gpt->cfg.mel_vocab,
                           hipMemcpyDeviceToHost, gpt->stream));
  HIP_TRY(hipStreamSynchronize(gpt->stream));
  return ITTS_OK;
}

itts_status itts_gpt_teacher_forced(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens, int32_t n_text,
                                    const float *conds, int32_t n_cond, int32_t lang_id, const int32_t *codes,
                                    int32_t n_codes, float *log_probs_out, float *attention_out) {
  if (itts_status st = check_replay_args(gpt, kv, codes, n_codes)) return st;
  if (!log_probs_out) return set_error(ITTS_E_VALIDATION, "log_probs: null output");
  if (attention_out)
    for (int i = 0; i < gpt->n_align; i++)
      if (gpt->align_pairs[i][0] >= gpt->cfg.n_layer || gpt->align_pairs[i][1] >= gpt->cfg.n_head)
        return set_error(ITTS_E_VALIDATION, "alignment_heads: (%d, %d) outside the model", gpt->align_pairs[i][0],
                         gpt->align_pairs[i][1]);
  // the last code is only a target: the fed rows are codes[..n-1] (gpt.rs:806-811)
  const std::vector<int32_t> fed(codes, codes + n_codes - 1);
  const int text_hi = n_cond + n_text + 2;
  int T = 0;
  if (itts_status st = replay(gpt, kv, text_tokens, n_text, conds, n_cond, lang_id, fed, text_hi, gpt->cfg.n_layer,
                              n_codes, attention_out, &T))
    return st;
  // rows text_hi .. T-1 (the start-Mel row and the fed codes) predict codes[0..n)
  if (itts_status st = head_rows(gpt, text_hi, n_codes)) return st;
  HIP_TRY(gpt->pcodes.ensure(sizeof(int32_t) * n_codes));
  HIP_TRY(gpt->plp.ensure(sizeof(float) * n_codes));
  HIP_TRY(hipMemcpyAsync(gpt->pcodes.p, codes, sizeof(int32_t) * n_codes, hipMemcpyHostToDevice, gpt->stream));
  HIP_TRY(launch_log_softmax_pick(gpt->plog.as<float>(), n_codes, gpt->cfg.mel_vocab, gpt->pcodes.as<int>(),
                                  gpt->plp.as<float>(), gpt->stream));
  HIP_TRY(hipMemcpyAsync(log_probs_out, gpt->plp.p, sizeof(float) * n_codes, hipMemcpyDeviceToHost, gpt->stream));
  HIP_TRY(hipStreamSynchronize(gpt->stream));
  kv->valid_len = 0;
  return ITTS_OK;
}

itts_status itts_gpt_alignment_attention(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens, int32_t n_text,
                                         const float *conds, int32_t n_cond, int32_t lang_id,
                                         const int32_t *prior_codes, int32_t n_prior, const int32_t *codes,
                                         int32_t n_codes, float *attention_out) {
  if (itts_status st = check_replay_args(gpt, kv, codes, n_codes)) return st;
  if (!attention_out) return set_error(ITTS_E_VALIDATION, "attention: null output");
  if (n_prior < 0 || (n_prior > 0 && !prior_codes)) return set_error(ITTS_E_VALIDATION, "codes: null prior codes");
  int n_layers = 0;
  for (int i = 0; i < gpt->n_align; i++) {
    if (gpt->align_pairs[i][0] >= gpt->cfg.n_layer || gpt->align_pairs[i][1] >= gpt->cfg.n_head)
      return set_error(ITTS_E_VALIDATION, "alignment_heads: (%d, %d) outside the model", gpt->align_pairs[i][0],
                       gpt->align_pairs[i][1]);
    n_layers = std::max(n_layers, gpt->align_pairs[i][0] + 1);
  }
  // fed = prior ++ codes[..n-1]; queries from the row that predicted codes[0] (gpt.rs:885-895)
  std::vector<int32_t> fed(prior_codes, prior_codes + n_prior);
  fed.insert(fed.end(), codes, codes + n_codes - 1);
  const int q0 = n_cond + n_text + 2 + n_prior;
  int T = 0;
  if (itts_status st = replay(gpt, kv, text_tokens, n_text, conds, n_cond, lang_id, fed, q0, n_layers, n_codes,
                              attention_out, &T))
    return st;
  kv->valid_len = 0;
  return ITTS_OK;
}

itts_status itts_gpt_set_alignment_heads(itts_gpt *gpt, const int32_t *pairs, int32_t n_pairs) {
  if (!gpt || !pairs || n_pairs < 1 || n_pairs > 2)
    return set_error(ITTS_E_VALIDATION, "alignment_heads: 1 or 2 (layer, head) pairs expected");
  for (int i = 0; i < n_pairs; i++)
    if (pairs[2 * i] < 0 || pairs[2 * i] >= gpt->cfg.n_layer || pairs[2 * i + 1] < 0 ||
        pairs[2 * i + 1] >= gpt->cfg.n_head)
      return set_error(ITTS_E_VALIDATION, "alignment_heads: (%d, %d) outside the model", pairs[2 * i],
                       pairs[2 * i + 1]);
  for (int i = 0; i < n_pairs; i++) {
    gpt->align_pairs[i][0] = pairs[2 * i];
    gpt->align_pairs[i][1] = pairs[2 * i + 1];
  }
  gpt->n_align = n_pairs;
  return ITTS_OK;
}

itts_status itts_gpt_forward_logits(itts_gpt *gpt, const itts_code_prompt *prompts, int32_t batch,
                                    float *logits_out) {
  if (!gpt || !prompts || batch <= 0)
    return set_error(ITTS_E_VALIDATION, "prompts: a non-empty batch is required");
  std::vector<int> row0, T;
  int M = 0;
  if (itts_status st = embed_prompts(gpt, prompts, batch, row0, T, &M)) return st;
  std::vector<int> kstart(M);
  for (int b = 0; b < batch; b++)
    for (int r = 0; r < T[b]; r++) kstart[row0[b] + r] = row0[b];
  if (itts_status st = forward_rows_stack(gpt, M, kstart, gpt->cfg.n_layer, {})) return st;
  if (itts_status st = head_rows(gpt, 0, M)) return st;
  if (logits_out)
    HIP_TRY(hipMemcpyAsync(logits_out, gpt->plog.p, sizeof(float) * (size_t)M * gpt->cfg.mel_vocab,
                           hipMemcpyDeviceToHost, gpt->stream));
  HIP_TRY(hipStreamSynchronize(gpt->stream));
  return ITTS_OK;
}

itts_status itts_gpt_prefill(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens, int32_t n_text,
                             const float *conds, int32_t n_cond, int32_t lang_id, float *logits_out) {
  return itts_gpt_prefill_after(gpt, kv, text_tokens, n_text, conds, n_cond, lang_id, nullptr, 0,
                                logits_out);
}

itts_status itts_gpt_step(itts_gpt *gpt, itts_kv *kv, int32_t mel_token_id, int32_t pos_idx,
                          float *logits_out) {
  if (!gpt || !kv || kv->gpt != gpt) return set_error(ITTS_E_VALIDATION, "kv_cache: cache belongs to another decoder");
  const itts_config &c = gpt->cfg;
  if (mel_token_id < 0 || mel_token_id >= c.mel_vocab)
    return set_error(ITTS_E_VALIDATION, "mel_token_id: mel_token_id %d out of range 0..%d", mel_token_id,
                     c.mel_vocab);
  if (pos_idx < 0 || pos_idx >= c.mel_pos_len)
    return set_error(ITTS_E_VALIDATION, "pos_idx: pos_idx %d out of range 0..%d", pos_idx, c.mel_pos_len);
  if (kv->valid_len + 1 > kv->max_seq)
    return set_error(ITTS_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d",
                     kv->valid_len + 1, kv->max_seq);
  DecodeCtl h{};
  h.tok = mel_token_id;
  h.pos = pos_idx;
  h.valid_len = kv->valid_len;
  if (itts_status st = write_ctl(kv, h)) return st;
  if (itts_status st = enqueue_decode_step(gpt, kv)) return st;
  if (logits_out)
    HIP_TRY(hipMemcpyAsync(logits_out, gpt->logits.p, sizeof(float) * c.mel_vocab, hipMemcpyDeviceToHost,
                           gpt->stream));
  HIP_TRY(hipStreamSynchronize(gpt->stream));
  if (itts_status st = check_persist(kv)) return st;
  kv->valid_len += 1;
  return ITTS_OK;
}

uint64_t itts_rng_new(uint64_t seed) { return seed ^ 0x9E3779B97F4A7C15ull; }

uint64_t itts_rng_next_u64(uint64_t *state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

float itts_rng_next_f32(uint64_t *state) {
  const uint32_t upper = (uint32_t)(itts_rng_next_u64(state) >> 40);
  return (float)upper * (1.0f / 16777216.0f);
}

void itts_seen_init(uint64_t words[129]) {
  memset(words, 0, 129 * sizeof(uint64_t));
  itts_seen_insert(words, 1);
  itts_seen_insert(words, 8192);
}

void itts_seen_insert(uint64_t words[129], int32_t token_id) {
  if (token_id >= 0 && token_id < 129 * 64) words[token_id / 64] |= 1ull << (token_id % 64);
}

itts_status itts_sample_next_token(itts_gpt *gpt, float *logits, int32_t n, const uint64_t seen[129],
                                   const itts_sampling *p, uint64_t *rng_state, int32_t *token_out) {
  if (!gpt || !logits || !seen || !rng_state || !token_out)
    return set_error(ITTS_E_VALIDATION, "logits: null argument");
  if (n <= 0) return set_error(ITTS_E_VALIDATION, "logits: logits slice must not be empty");
  if (n > 9216) return set_error(ITTS_E_VALIDATION, "logits: at most 9216 logits");
  if (itts_status st = itts_sampling_validate(p)) return st;
  hipStream_t s = gpt->stream;
  HIP_TRY(gpt->s_logits.ensure(sizeof(float) * n));
  HIP_TRY(gpt->s_seen.ensure(sizeof(uint64_t) * 129));
  HIP_TRY(gpt->s_rng.ensure(sizeof(uint64_t)));
  HIP_TRY(gpt->s_tok.ensure(sizeof(int32_t)));
  HIP_TRY(hipMemcpyAsync(gpt->s_logits.p, logits, sizeof(float) * n, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(gpt->s_seen.p, seen, sizeof(uint64_t) * 129, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(gpt->s_rng.p, rng_state, sizeof(uint64_t), hipMemcpyHostToDevice, s));
  HIP_TRY(launch_sampler(gpt->s_logits.as<float>(), n, gpt->s_seen.as<uint64_t>(), to_dev_sampling(*p, n),
                         gpt->s_rng.as<uint64_t>(), gpt->s_tok.as<int32_t>(), nullptr, nullptr, -1, 0, s));
  HIP_TRY(hipMemcpyAsync(logits, gpt->s_logits.p, sizeof(float) * n, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(rng_state, gpt->s_rng.p, sizeof(uint64_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(token_out, gpt->s_tok.p, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return ITTS_OK;
}

// Calls on one device share its staging area: they are serialised here (each call
// returns only after its copies back have completed).
std::mutex g_stage_call_mu[kMaxDevices];

itts_status itts_sample_next_token_noalloc(itts_gpt *gpt, float *logits, int32_t n, const uint64_t seen[129],
                                           const itts_sampling *p, uint64_t *rng_state, int32_t *token_out) {
  if (!gpt || !logits || !seen || !rng_state || !token_out)
    return set_error(ITTS_E_VALIDATION, "logits: null argument");
  if (n <= 0) return set_error(ITTS_E_VALIDATION, "logits: logits slice must not be empty");
  if (n > kStageMaxLogits)
    return set_error(ITTS_E_VALIDATION, "logits: at most %d logits (the size of the staging area)", kStageMaxLogits);
  if (itts_status st = itts_sampling_validate(p)) return st;
  SamplerStage sg{};
  if (!sampler_stage(gpt->device, &sg))
    return set_error(ITTS_E_DEVICE, "sampler staging area of device %d is not set up", gpt->device);
  std::lock_guard<std::mutex> lock(g_stage_call_mu[gpt->device]);
  hipStream_t s = gpt->stream;
  HIP_TRY(hipMemcpyAsync(sg.logits, logits, sizeof(float) * n, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(sg.seen, seen, sizeof(uint64_t) * 129, hipMemcpyHostToDevice, s));
  HIP_TRY(hipMemcpyAsync(sg.rng, rng_state, sizeof(uint64_t), hipMemcpyHostToDevice, s));
  HIP_TRY(launch_sampler(sg.logits, n, sg.seen, to_dev_sampling(*p, n), sg.rng, sg.tok, nullptr, nullptr, -1, 0, s));
  HIP_TRY(hipMemcpyAsync(logits, sg.logits, sizeof(float) * n, hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(rng_state, sg.rng, sizeof(uint64_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipMemcpyAsync(token_out, sg.tok, sizeof(int32_t), hipMemcpyDeviceToHost, s));
  HIP_TRY(hipStreamSynchronize(s));
  return ITTS_OK;
}

static bool same_sampling(const DevSampling &a, const DevSampling &b) {
  return memcmp(&a, &b, sizeof(DevSampling)) == 0;
}

itts_status itts_generate_codes_after(itts_gpt *gpt, itts_kv *kv, const itts_code_prompt *prompt,
                                      const itts_sampling *p, uint64_t *rng_state, int32_t *codes_out,
                                      int32_t codes_cap, int32_t *n_codes) {
  if (!gpt || !kv || !prompt || !rng_state || !codes_out || !n_codes)
    return set_error(ITTS_E_VALIDATION, "generate: null argument");
  if (kv->gpt != gpt) return set_error(ITTS_E_VALIDATION, "kv_cache: cache belongs to another decoder");
  if (itts_status st = itts_sampling_validate(p)) return st;
  const itts_config &c = gpt->cfg;
  const int room = std::max(0, c.mel_pos_len - 3 - prompt->n_prior);
  const int max_steps = std::min<int>((int)p->max_mel_tokens, room);
  if (max_steps == 0)
    return set_error(ITTS_E_VALIDATION,
                     "max_mel_tokens: no Mel positions left to generate (max_mel_tokens is 0 or the prior "
                     "codes fill the capacity)");
  if (codes_cap < max_steps) return set_error(ITTS_E_VALIDATION, "codes_out: capacity %d < %d", codes_cap, max_steps);
  if (prompt->min_codes < 0) return set_error(ITTS_E_VALIDATION, "min_codes: negative");
  kv->timing_valid = false;
  for (hipEvent_t &ev : kv->ev_t)
    if (!ev) HIP_TRY(hipEventCreate(&ev));
  HIP_TRY(hipEventRecord(kv->ev_t[0], gpt->stream));
  int T = 0;
  itts_status st = run_prefill(gpt, kv, prompt->text_tokens, prompt->n_text, prompt->conds, prompt->n_cond,
                               prompt->lang_id, prompt->prior_codes, prompt->n_prior, &T);
  if (st) return st;
  HIP_TRY(hipEventRecord(kv->ev_t[1], gpt->stream));
  // Sample s is followed by a step that writes cache row T + s; the reference fails that
  // step with a KV-capacity error once T + s + 1 > max_seq (gpt.rs:157-165).  The device
  // loop therefore runs at most max_seq - T + 1 samples and reports the overflow if it
  // gets there without STOP.
  const int fit = kv->max_seq - T + 1;
  const int dev_steps = std::min(max_steps, fit);
  DecodeCtl h{};
  h.valid_len = T;
  h.min_codes = prompt->min_codes;
  h.max_steps = dev_steps;
  h.n_prior = prompt->n_prior;
  h.rng = *rng_state;
  h.last_tok = -1;
  // prior codes are not added to the penalty set (sampler.rs:365-368)
  memset(h.seen, 0, sizeof h.seen);
  h.seen[0] |= 1ull << 1;
  const int start_mel = c.mel_vocab - 2;
  h.seen[start_mel / 64] |= 1ull << (start_mel % 64);
  if ((st = write_ctl(kv, h))) return st;

  const DevSampling ds = to_dev_sampling(*p, c.mel_vocab);
  auto enqueue_iteration = [&]() -> itts_status {
    hipError_t le = launch_sampler(gpt->logits.as<float>(), c.mel_vocab, nullptr, ds, nullptr, nullptr,
                                   kv->ctl.as<DecodeCtl>(), kv->codes.as<int32_t>(), c.mel_vocab - 1, 1,
                                   gpt->stream);
    if (le != hipSuccess) return set_error(ITTS_E_DEVICE, "sampler launch failed: %s", hipGetErrorName(le));
    return enqueue_decode_step(gpt, kv);
  };
  // Replay in batches of `batch` iterations (sample, then step).  One graph is captured
  // once per cache and sampling parameters: the whole batch for the persistent step (its
  // launch is ordered against other decoders' persistent launches around the graph), one
  // iteration for the multi-kernel step.
  const int batch = 8;
  const bool use_graph = gpt->use_graph;
  const int per_graph = kv->persist ? batch : 1;
  auto enqueue_captured = [&]() -> itts_status {
    for (int i = 0; i < per_graph; i++) {
      hipError_t le = launch_sampler(gpt->logits.as<float>(), c.mel_vocab, nullptr, ds, nullptr, nullptr,
                                     kv->ctl.as<DecodeCtl>(), kv->codes.as<int32_t>(), c.mel_vocab - 1, 1,
                                     gpt->stream);
      if (le != hipSuccess) return set_error(ITTS_E_DEVICE, "sampler launch failed: %s", hipGetErrorName(le));
      if (kv->persist) {
        le = launch_decode_persist(kv->pa, c.quant_bits, gpt->ptype(), gpt->stream);
        if (le != hipSuccess) return set_error(ITTS_E_DEVICE, "decode step launch failed: %s", hipGetErrorName(le));
      } else if (itts_status st2 = enqueue_decode_step(gpt, kv)) {
        return st2;
      }
    }
    return ITTS_OK;
  };
  if (use_graph && (!kv->have_graph || !same_sampling(kv->gkey, ds))) {
    if (kv->gexec) {
      (void)hipGraphExecDestroy(kv->gexec);
      kv->gexec = nullptr;
    }
    if (kv->graph) {
      (void)hipGraphDestroy(kv->graph);
      kv->graph = nullptr;
    }
    kv->have_graph = false;
    HIP_TRY(hipStreamSynchronize(gpt->stream));
    HIP_TRY(hipStreamBeginCapture(gpt->stream, hipStreamCaptureModeThreadLocal));
    itts_status es = enqueue_captured();
    hipGraph_t graph = nullptr;
    hipError_t ce = hipStreamEndCapture(gpt->stream, &graph);
    if (es) {
      if (graph) (void)hipGraphDestroy(graph);
      return es;
    }
    HIP_TRY(ce);
    kv->graph = graph;
    HIP_TRY(hipGraphInstantiate(&kv->gexec, kv->graph, nullptr, nullptr, 0));
    kv->gkey = ds;
    kv->have_graph = true;
  }
  // Keep one batch in flight while the previous one's control block is inspected;
  // iterations after `done` exit at their first instruction.
  DecodeCtl *slot[2] = {kv->host_ctl, kv->host_ctl + 1};
  hipEvent_t ev[2];
  HIP_TRY(hipEventCreateWithFlags(&ev[0], hipEventDisableTiming));
  if (hipEventCreateWithFlags(&ev[1], hipEventDisableTiming) != hipSuccess) {
    (void)hipEventDestroy(ev[0]);
    return set_error(ITTS_E_DEVICE, "hipEventCreate failed");
  }
  auto cleanup = [&]() {
    (void)hipEventDestroy(ev[0]);
    (void)hipEventDestroy(ev[1]);
  };
  // Batch nb holds min(batch, max_steps - nb * batch) iterations that can sample; a shorter
  // last batch (a short generation, the time to the first token) is launched iteration by
  // iteration rather than as the whole graph, whose surplus iterations would only exit.
  auto launch_batch = [&](int which, int iters) -> hipError_t {
    if (iters < batch) {
      for (int i = 0; i < iters; i++)
        if (enqueue_iteration() != ITTS_OK) return hipErrorLaunchFailure;
    } else if (use_graph && kv->persist) {
      if (persist_chained(gpt, [&] { return hipGraphLaunch(kv->gexec, gpt->stream); }) != ITTS_OK)
        return hipErrorLaunchFailure;
    } else {
      for (int i = 0; i < batch; i++) {
        if (use_graph) {
          hipError_t e = hipGraphLaunch(kv->gexec, gpt->stream);
          if (e != hipSuccess) return e;
        } else if (enqueue_iteration() != ITTS_OK) {
          return hipErrorLaunchFailure;
        }
      }
    }
    hipError_t e = hipMemcpyAsync(slot[which], kv->ctl.p, offsetof(DecodeCtl, seen), hipMemcpyDeviceToHost,
                                  gpt->stream);
    if (e != hipSuccess) return e;
    return hipEventRecord(ev[which], gpt->stream);
  };
  // Each iteration samples once and `done` is set by step max_steps-1 at the latest, so
  // ceil(max_steps / batch) batches always reach the end.
  const int nb_total = (max_steps + batch - 1) / batch;
  auto iters_of = [&](int b) { return std::min(batch, max_steps - b * batch); };
  int nb = 0;
  hipError_t e = launch_batch(0, iters_of(0));
  nb = 1;
  for (int i = 0; e == hipSuccess; i++) {
    if (nb < nb_total) {
      e = launch_batch(nb & 1, iters_of(nb));
      nb++;
      if (e != hipSuccess) break;
    }
    e = hipEventSynchronize(ev[i & 1]);
    if (e != hipSuccess) break;
    if (slot[i & 1]->done || i + 1 >= nb_total) break;
  }
  // the end event, the error word and the final control block, then one synchronisation
  // (every batch's copy into the slots has completed by then)
  if (e == hipSuccess) e = hipEventRecord(kv->ev_t[2], gpt->stream);
  if (e == hipSuccess) e = persist_err_enqueue(kv);
  if (e == hipSuccess)
    e = hipMemcpyAsync(slot[0], kv->ctl.p, offsetof(DecodeCtl, seen), hipMemcpyDeviceToHost, gpt->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(gpt->stream);
  cleanup();
  HIP_TRY(e);
  if (itts_status pst = persist_err_check(kv)) return pst;
  DecodeCtl fin{};
  memcpy(&fin, slot[0], offsetof(DecodeCtl, seen));
  if (!fin.done) return set_error(ITTS_E_INTERNAL, "generation did not reach its end");
  kv->valid_len = fin.valid_len;
  HIP_TRY(hipEventElapsedTime(&kv->timing.prefill_ms, kv->ev_t[0], kv->ev_t[1]));
  HIP_TRY(hipEventElapsedTime(&kv->timing.decode_ms, kv->ev_t[1], kv->ev_t[2]));
  kv->timing.prefill_rows = T;
  kv->timing.decode_steps = fin.valid_len - T;
  kv->timing.samples = fin.step;
  kv->timing_valid = true;
  if (dev_steps < max_steps && fin.n_codes == dev_steps)
    return set_error(ITTS_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d",
                     kv->max_seq + 1, kv->max_seq);
  HIP_TRY(hipMemcpy(codes_out, kv->codes.p, sizeof(int32_t) * fin.n_codes, hipMemcpyDeviceToHost));
  *n_codes = fin.n_codes;
  *rng_state = fin.rng;
  kv->valid_len = fin.valid_len;
  return ITTS_OK;
}

itts_status itts_gpt_step_batch(itts_gpt *gpt, itts_kv *const *caches, int32_t batch, const int32_t *tokens,
                                const int32_t *positions, float *logits_out) {
  if (!gpt || !tokens || !positions) return set_error(ITTS_E_VALIDATION, "step_batch: null argument");
  if (itts_status st = prepare_batch(gpt, caches, batch)) return st;
  const itts_config &c = gpt->cfg;
  for (int b = 0; b < batch; b++) {  // Gpt::step's checks, per sequence (gpt.rs:707-718)
    itts_kv *kv = caches[b];
    if (tokens[b] < 0 || tokens[b] >= c.mel_vocab)
      return set_error(ITTS_E_VALIDATION, "mel_token_id: mel_token_id %d out of range 0..%d", tokens[b], c.mel_vocab);
    if (positions[b] < 0 || positions[b] >= c.mel_pos_len)
      return set_error(ITTS_E_VALIDATION, "pos_idx: pos_idx %d out of range 0..%d", positions[b], c.mel_pos_len);
    if (kv->valid_len + 1 > kv->max_seq)
      return set_error(ITTS_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d",
                       kv->valid_len + 1, kv->max_seq);
  }
  for (int b = 0; b < batch; b++) {
    DecodeCtl h{};
    h.tok = tokens[b];
    h.pos = positions[b];
    h.valid_len = caches[b]->valid_len;
    if (itts_status st = write_ctl(caches[b], h)) return st;
  }
  if (itts_status st = enqueue_step_batch(gpt, batch, caches[0]->max_seq, caches[0]->kvt)) return st;
  if (logits_out)
    HIP_TRY(hipMemcpyAsync(logits_out, gpt->blog.p, sizeof(float) * (size_t)batch * c.mel_vocab,
                           hipMemcpyDeviceToHost, gpt->stream));
  HIP_TRY(hipStreamSynchronize(gpt->stream));
  for (int b = 0; b < batch; b++) caches[b]->valid_len += 1;
  return ITTS_OK;
}

itts_status itts_generate_codes_batch(itts_gpt *gpt, itts_kv *const *caches, const itts_code_prompt *prompts,
                                      const itts_sampling *params, int32_t batch, uint64_t *rng_states,
                                      int32_t *codes_out, int32_t codes_cap, int32_t *n_codes) {
  if (!gpt || !prompts || !params || !rng_states || !codes_out || !n_codes)
    return set_error(ITTS_E_VALIDATION, "generate: null argument");
  if (itts_status st = prepare_batch(gpt, caches, batch)) return st;
  const itts_config &c = gpt->cfg;
  std::vector<int> max_steps(batch), dev_steps(batch), T(batch);
  std::vector<DevSampling> ds(batch);
  int top_k_max = 1, longest = 0;
  bool any_sampled = false;
  for (int b = 0; b < batch; b++) {  // generate_codes_after's checks, per sequence
    const itts_code_prompt &pr = prompts[b];
    if (itts_status st = itts_sampling_validate(&params[b])) return st;
    const int room = std::max(0, c.mel_pos_len - 3 - pr.n_prior);
    max_steps[b] = std::min<int>((int)params[b].max_mel_tokens, room);
    if (max_steps[b] == 0)
      return set_error(ITTS_E_VALIDATION,
                       "max_mel_tokens: no Mel positions left to generate (max_mel_tokens is 0 or the prior "
                       "codes fill the capacity)");
    if (codes_cap < max_steps[b])
      return set_error(ITTS_E_VALIDATION, "codes_out: capacity %d < %d", codes_cap, max_steps[b]);
    if (pr.min_codes < 0) return set_error(ITTS_E_VALIDATION, "min_codes: negative");
    ds[b] = to_dev_sampling(params[b], c.mel_vocab);
    if (!ds[b].greedy) {
      any_sampled = true;
      top_k_max = std::max(top_k_max, ds[b].top_k);
    }
  }
  // prefill each prompt into its cache; its last-row logits seed the batch's first sample
  for (int b = 0; b < batch; b++) {
    itts_kv *kv = caches[b];
    const itts_code_prompt &pr = prompts[b];
    if (itts_status st = run_prefill(gpt, kv, pr.text_tokens, pr.n_text, pr.conds, pr.n_cond, pr.lang_id,
                                     pr.prior_codes, pr.n_prior, &T[b]))
      return st;
    HIP_TRY(hipMemcpyAsync(gpt->blog.as<float>() + (size_t)b * c.mel_vocab, gpt->logits.p,
                           sizeof(float) * c.mel_vocab, hipMemcpyDeviceToDevice, gpt->stream));
    dev_steps[b] = std::min(max_steps[b], kv->max_seq - T[b] + 1);
    longest = std::max(longest, dev_steps[b]);
    DecodeCtl h{};
    h.valid_len = T[b];
    h.min_codes = pr.min_codes;
    h.max_steps = dev_steps[b];
    h.n_prior = pr.n_prior;
    h.rng = rng_states[b];
    h.last_tok = -1;
    memset(h.seen, 0, sizeof h.seen);
    h.seen[0] |= 1ull << 1;
    const int start_mel = c.mel_vocab - 2;
    h.seen[start_mel / 64] |= 1ull << (start_mel % 64);
    *kv->host_ctl = h;
    HIP_TRY(hipMemcpyAsync(kv->ctl.p, kv->host_ctl, offsetof(DecodeCtl, xstep), hipMemcpyHostToDevice,
                           gpt->stream));
    HIP_TRY(hipStreamSynchronize(gpt->stream));  // host_ctl is reused below
  }
  HIP_TRY(gpt->bps.ensure(sizeof(DevSampling) * batch));
  HIP_TRY(hipMemcpyAsync(gpt->bps.p, ds.data(), sizeof(DevSampling) * batch, hipMemcpyHostToDevice, gpt->stream));
  const int max_seq = caches[0]->max_seq, kvt = caches[0]->kvt;
  auto enqueue_iteration = [&]() -> itts_status {
    hipError_t le = launch_sampler_batch(gpt->blog.as<float>(), c.mel_vocab, gpt->bps.as<DevSampling>(),
                                         gpt->bseqs.as<BatchSeq>(), batch, c.mel_vocab - 1, top_k_max, any_sampled,
                                         gpt->stream);
    if (le != hipSuccess) return set_error(ITTS_E_DEVICE, "sampler launch failed: %s", hipGetErrorName(le));
    return enqueue_step_batch(gpt, batch, max_seq, kvt);
  };
  // one iteration (sample every sequence, then step the batch) captured once per call
  hipGraph_t graph = nullptr;
  hipGraphExec_t gexec = nullptr;
  auto release = [&]() {
    if (gexec) (void)hipGraphExecDestroy(gexec);
    if (graph) (void)hipGraphDestroy(graph);
  };
  if (gpt->use_graph) {
    HIP_TRY(hipStreamSynchronize(gpt->stream));
    HIP_TRY(hipStreamBeginCapture(gpt->stream, hipStreamCaptureModeThreadLocal));
    itts_status es = enqueue_iteration();
    hipError_t ce = hipStreamEndCapture(gpt->stream, &graph);
    if (es) {
      release();
      return es;
    }
    if (ce == hipSuccess) ce = hipGraphInstantiate(&gexec, graph, nullptr, nullptr, 0);
    if (ce != hipSuccess) {
      release();
      return set_error(ITTS_E_DEVICE, "graph capture failed: %s", hipGetErrorName(ce));
    }
  }
  // replay in chunks of 8 iterations; finished sequences skip their work, so the batch
  // runs until every sequence is done (at most the longest sequence's steps)
  std::vector<DecodeCtl> fin(batch);
  const int chunk = 8;
  hipError_t e = hipSuccess;
  for (int it = 0; it < longest && e == hipSuccess;) {
    for (int i = 0; i < chunk && it < longest; i++, it++) {
      if (gexec) {
        e = hipGraphLaunch(gexec, gpt->stream);
      } else if (enqueue_iteration() != ITTS_OK) {
        e = hipErrorLaunchFailure;
      }
      if (e != hipSuccess) break;
    }
    for (int b = 0; b < batch && e == hipSuccess; b++)
      e = hipMemcpyAsync(&fin[b], caches[b]->ctl.p, offsetof(DecodeCtl, seen), hipMemcpyDeviceToHost, gpt->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(gpt->stream);
    bool all = true;
    for (int b = 0; b < batch; b++) all = all && fin[b].done;
    if (all) break;
  }
  release();
  HIP_TRY(e);
  for (int b = 0; b < batch; b++)
    if (!fin[b].done) return set_error(ITTS_E_INTERNAL, "generation did not reach its end");
  itts_status result = ITTS_OK;
  for (int b = 0; b < batch; b++) {
    itts_kv *kv = caches[b];
    kv->valid_len = fin[b].valid_len;
    n_codes[b] = fin[b].n_codes;
    rng_states[b] = fin[b].rng;
    HIP_TRY(hipMemcpy(codes_out + (size_t)b * codes_cap, kv->codes.p, sizeof(int32_t) * fin[b].n_codes,
                      hipMemcpyDeviceToHost));
    if (dev_steps[b] < max_steps[b] && fin[b].n_codes == dev_steps[b] && result == ITTS_OK)
      result = set_error(ITTS_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d",
                         kv->max_seq + 1, kv->max_seq);
  }
  return result;
}

itts_status itts_kv_last_timing(const itts_kv *kv, itts_timing *out) {
  if (!kv || !out) return set_error(ITTS_E_VALIDATION, "timing: null argument");
  if (!kv->timing_valid) return set_error(ITTS_E_VALIDATION, "timing: no completed generate call on this cache");
  *out = kv->timing;
  return ITTS_OK;
}

itts_status itts_generate_codes(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens, int32_t n_text,
                                const float *conds, int32_t n_cond, int32_t lang_id, const itts_sampling *p,
                                uint64_t *rng_state, int32_t *codes_out, int32_t codes_cap, int32_t *n_codes) {
  itts_code_prompt pr{};
  pr.text_tokens = text_tokens;
  pr.n_text = n_text;
  pr.conds = conds;
  pr.n_cond = n_cond;
  pr.lang_id = lang_id;
  return itts_generate_codes_after(gpt, kv, &pr, p, rng_state, codes_out, codes_cap, n_codes);
}

itts_status itts_decode_timing(itts_gpt *gpt, itts_kv *kv, int32_t mel_token_id, int32_t pos_idx, int32_t n_steps,
                               float *ms_per_step) {
  if (!gpt || !kv || !ms_per_step || kv->gpt != gpt) return set_error(ITTS_E_VALIDATION, "timing: bad argument");
  const itts_config &c = gpt->cfg;
  if (n_steps < 1) return set_error(ITTS_E_VALIDATION, "n_steps: must be >= 1");
  if (mel_token_id < 0 || mel_token_id >= c.mel_vocab)
    return set_error(ITTS_E_VALIDATION, "mel_token_id: mel_token_id %d out of range 0..%d", mel_token_id,
                     c.mel_vocab);
  if (pos_idx < 0 || pos_idx >= c.mel_pos_len)
    return set_error(ITTS_E_VALIDATION, "pos_idx: pos_idx %d out of range 0..%d", pos_idx, c.mel_pos_len);
  if (kv->valid_len + n_steps > kv->max_seq)
    return set_error(ITTS_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d",
                     kv->valid_len + n_steps, kv->max_seq);
  for (hipEvent_t &ev : kv->ev_t)
    if (!ev) HIP_TRY(hipEventCreate(&ev));
  DecodeCtl h{};
  h.tok = mel_token_id;
  h.pos = pos_idx;
  h.valid_len = kv->valid_len;
  if (itts_status st = write_ctl(kv, h)) return st;
  HIP_TRY(hipEventRecord(kv->ev_t[0], gpt->stream));
  for (int i = 0; i < n_steps; i++)
    if (itts_status st = enqueue_decode_step(gpt, kv)) return st;
  HIP_TRY(hipEventRecord(kv->ev_t[1], gpt->stream));
  HIP_TRY(hipEventSynchronize(kv->ev_t[1]));
  if (itts_status st = check_persist(kv)) return st;
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, kv->ev_t[0], kv->ev_t[1]));
  kv->valid_len += n_steps;
  *ms_per_step = ms / (float)n_steps;
  return ITTS_OK;
}

// ---- quantiser ----

static inline uint16_t f32_to_f16_rne(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    if (ax < 0x33000000u) return (uint16_t)sign;
    const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, sh = 126 - e;
    uint32_t h = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = (ax >> 13) - (112u << 10);
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

static inline float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float out;
  if (e == 0) {
    out = (float)m * 5.9604644775390625e-08f;
    return sign ? -out : out;
  }
  const uint32_t bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  memcpy(&out, &bits, 4);
  return out;
}

itts_status itts_quantize(const float *w, int32_t N, int32_t K, int32_t bits, itts_dtype param_dtype,
                          void *codes, void *scales, void *biases) {
  if (!w || !codes || !scales || !biases) return set_error(ITTS_E_VALIDATION, "quantize: null argument");
  if (N <= 0 || K <= 0 || K % 64 != 0) return set_error(ITTS_E_VALIDATION, "quantize: K must be a multiple of 64");
  if (bits != 8 && bits != 4) return set_error(ITTS_E_VALIDATION, "quantize: bits must be 8 or 4");
  if (param_dtype != ITTS_F16 && param_dtype != ITTS_F32)
    return set_error(ITTS_E_VALIDATION, "quantize: param_dtype must be F16 or F32");
  const int G = K / 64;
  const float levels = bits == 8 ? 255.0f : 15.0f;
  const bool f32 = param_dtype == ITTS_F32;
  uint8_t *cb = static_cast<uint8_t *>(codes);
  auto work = [&](int r0, int r1) {
    for (int o = r0; o < r1; o++) {
      if (bits == 4) memset(cb + (size_t)o * (K / 2), 0, K / 2);
      for (int g = 0; g < G; g++) {
        const float *p = w + (size_t)o * K + (size_t)g * 64;
        float mn = p[0], mx = p[0];
        for (int i = 1; i < 64; i++) {
          mn = p[i] < mn ? p[i] : mn;
          mx = p[i] > mx ? p[i] : mx;
        }
        float s = (mx - mn) / levels, b = mn;
        const size_t gi = (size_t)o * G + g;
        if (f32) {
          static_cast<float *>(scales)[gi] = s;
          static_cast<float *>(biases)[gi] = b;
        } else {
          const uint16_t sh = f32_to_f16_rne(s), bh = f32_to_f16_rne(b);
          static_cast<uint16_t *>(scales)[gi] = sh;
          static_cast<uint16_t *>(biases)[gi] = bh;
          s = f16_to_f32(sh);
          b = f16_to_f32(bh);
        }
        for (int i = 0; i < 64; i++) {
          float q = 0.0f;
          if (s != 0.0f) {
            q = std::rint((p[i] - b) / s);
            q = q < 0.0f ? 0.0f : (q > levels ? levels : q);
          }
          const int k = g * 64 + i;
          if (bits == 8) cb[(size_t)o * K + k] = (uint8_t)q;
          else cb[(size_t)o * (K / 2) + k / 2] |= (uint8_t)((int)q << ((k & 1) * 4));
        }
      }
    }
  };
  const int nt = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> th;
  const int per = (N + nt - 1) / nt;
  for (int t = 0; t < nt; t++) {
    const int r0 = t * per, r1 = std::min(N, r0 + per);
    if (r0 < r1) th.emplace_back(work, r0, r1);
  }
  for (auto &t : th) t.join();
  return ITTS_OK;
}

// ---- kernel-level entry points ----

static itts_status temp_ql(QLHost &q, const itts_qlinear *ql, int N, int K, int bits, itts_dtype pd) {
  if (!ql) return set_error(ITTS_E_VALIDATION, "qlinear: null");
  if (N <= 0 || K <= 0 || K % 64) return set_error(ITTS_E_VALIDATION, "qlinear: K must be a multiple of 64");
  if (bits != 8 && bits != 4) return set_error(ITTS_E_VALIDATION, "qlinear: bits must be 8 or 4");
  if (pd != ITTS_F16 && pd != ITTS_F32) return set_error(ITTS_E_VALIDATION, "qlinear: param dtype");
  std::vector<float> zero;
  itts_qlinear tmp = *ql;
  if (!tmp.bias) {
    zero.assign(N, 0.0f);
    tmp.bias = zero.data();
  }
  return upload_ql(q, tmp, N, K, bits, pd == ITTS_F32, "qlinear");
}

itts_status itts_dequantize(itts_gpt *gpt, const itts_qlinear *ql, int32_t N, int32_t K, int32_t bits,
                            itts_dtype param_dtype, float *out) {
  if (!gpt || !out) return set_error(ITTS_E_VALIDATION, "dequantize: null argument");
  QLHost q;
  if (itts_status st = temp_ql(q, ql, N, K, bits, param_dtype)) return st;
  DevBuf o;
  HIP_TRY(o.ensure(sizeof(float) * (size_t)N * K));
  HIP_TRY(launch_dequant(q.dev(), bits, param_dtype == ITTS_F32 ? kParamF32 : kParamF16, o.as<float>(),
                         gpt->stream));
  HIP_TRY(hipMemcpyAsync(out, o.p, sizeof(float) * (size_t)N * K, hipMemcpyDeviceToHost, gpt->stream));
  HIP_TRY(hipStreamSynchronize(gpt->stream));
  return ITTS_OK;
}

itts_status itts_qlinear_forward(itts_gpt *gpt, const itts_qlinear *ql, int32_t N, int32_t K, int32_t bits,
                                 itts_dtype param_dtype, const float *x, int32_t M, float *y) {
  if (!gpt || !x || !y || M <= 0) return set_error(ITTS_E_VALIDATION, "qlinear: bad argument");
  QLHost q;
  if (itts_status st = temp_ql(q, ql, N, K, bits, param_dtype)) return st;
  const int epc = bits == 8 ? 16 : 32;
  if (M == 1 && K / epc > 512) return set_error(ITTS_E_VALIDATION, "qlinear: K too large for the GEMV");
  DevBuf dx, dy;
  HIP_TRY(dx.ensure(sizeof(float) * (size_t)M * K));
  HIP_TRY(dy.ensure(sizeof(float) * (size_t)M * N));
  HIP_TRY(hipMemcpyAsync(dx.p, x, sizeof(float) * (size_t)M * K, hipMemcpyHostToDevice, gpt->stream));
  const int pt = param_dtype == ITTS_F32 ? kParamF32 : kParamF16;
  if (M == 1) {
    GemvArgs a{};
    a.ql = q.dev();
    a.x = dx.as<float>();
    a.y = dy.as<float>();
    HIP_TRY(launch_gemv(a, bits, pt, kProNone, kEpiStore, kKvBf16, gpt->stream));
  } else {
    SplitBuf xs;
    HIP_TRY(xs.ensure(M, K));
    HIP_TRY(launch_split_rows(dx.as<float>(), M, K, xs.out(), gpt->stream));
    GemmArgs a{};
    a.ql = q.dev();
    a.x = xs.act();
    a.M = M;
    a.y = dy.as<float>();
    a.ws = gpt->gws.as<float>();
    a.ws_floats = gpt->gws.bytes / sizeof(float);
    a.cnt = gpt->gcnt.as<uint32_t>();
    a.cnt_words = kGemmCounters;
    a.n_cu = gpt->n_cu;
    HIP_TRY(launch_gemm(a, bits, pt, kEpiStore, kKvBf16, gpt->stream));
    HIP_TRY(hipStreamSynchronize(gpt->stream));
  }
  HIP_TRY(hipMemcpyAsync(y, dy.p, sizeof(float) * (size_t)M * N, hipMemcpyDeviceToHost, gpt->stream));
  HIP_TRY(hipStreamSynchronize(gpt->stream));
  return ITTS_OK;
}

}  // extern "C"
