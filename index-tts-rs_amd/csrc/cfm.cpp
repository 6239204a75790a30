// libitts_hip: the Stage-2 CFM DiT estimator and its Euler / classifier-free-guidance solver
// (crates/core/src/models/cfm.rs), the itts_cfm_* entry points of include/itts_hip.h.
//
// CfmDit::from_weights -> itts_cfm_create (tensors by checkpoint name, checked by element
// count), forward_merged -> itts_cfm_forward, solve_euler -> itts_cfm_solve_euler.  The
// estimator keeps fp32 activations: its linears (and WaveNet's kernel-5 convolution, as one
// GEMM over a zero-padded buffer whose operand rows overlap) run on the split-fp16 MFMA GEMM
// of kernels_cfm.hip on the estimator's stream, products under 64 rows on its few-row fp32
// product; the other kernels in kernels_cfm.hip do the rest.  Layout: activations [B][T][C] row-major, the CFG
// pair as batch rows 0 (conditioned) and 1 (unconditioned).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/itts_hip.h"
#include "kernels.h"

namespace itts {
itts_status set_error_text(itts_status st, const char *msg);  // runtime.cpp
}

namespace {

using namespace itts;

itts_status cerr(itts_status st, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return set_error_text(st, buf);
}

#define CK(expr)                                                                                       \
  do {                                                                                                 \
    hipError_t e_ = (expr);                                                                            \
    if (e_ != hipSuccess) return cerr(ITTS_E_DEVICE, "HIP error %s at %s:%d", hipGetErrorName(e_), __FILE__, __LINE__); \
  } while (0)

constexpr int kFreqDim = 256;

struct Buf {
  float *p = nullptr;
  size_t n = 0;
  Buf() = default;
  Buf(const Buf &) = delete;
  Buf &operator=(const Buf &) = delete;
  Buf(Buf &&o) noexcept : p(o.p), n(o.n) { o.p = nullptr, o.n = 0; }
  ~Buf() {
    if (p) (void)hipFree(p);
  }
  hipError_t ensure(size_t count) {
    if (count <= n) return hipSuccess;
    if (p) {
      hipError_t e = hipFree(p);
      p = nullptr;
      n = 0;
      if (e != hipSuccess) return e;
    }
    hipError_t e = hipMalloc(&p, count * sizeof(float));
    if (e == hipSuccess) n = count;
    return e;
  }
};

hipError_t gemm(itts_cfm *m, int M, int N, int K, const float *A, int lda, const float *W, int ldw, float *y,
                int ldy, float beta, const float *bias = nullptr, const float *yr = nullptr);

struct Block {
  const float *wqkv, *wo, *w13, *w2, *skip_w, *skip_b, *an_w, *fn_w;
};
struct WnLayer {
  const float *in_w, *in_b, *rs_w, *rs_b;
};

}  // namespace

struct itts_cfm {
  itts_cfm_config c{};
  hipStream_t s = nullptr;
  float *arena = nullptr;
  const float *cond_w, *cond_b, *merge_w, *merge_b;
  const float *te_w0[2], *te_b0[2], *te_w2[2], *te_b2[2];
  const float *ada_w, *ada_b, *tn_w;  // AdaLN projections packed [(2L+1)*2d][d]: layer i attn 2i, ffn 2i+1, final 2L
  const float *skl_w, *skl_b, *c1_w, *c1_b, *rp_w, *rp_b, *wc_w, *wc_b, *fa_w, *fa_b, *fl_w, *fl_b, *c2_w, *c2_b;
  std::vector<Block> L;
  std::vector<WnLayer> wn;
  // per-forward workspace (sized for R = B*T rows)
  Buf emb, th, t1, t2, st, mods, wng, fmod, tdev;
  Buf hA, hB, n, qkv, att, gu, act, xres, hpad, acts, rs, oacc, v, rope, apo, aml, kvs;
  int rope_T = 0;  // sequence length the rope table holds
  int n_cu = 0;    // compute units of the device (the attention's split planner)
  std::vector<Buf> skips;
  // solve / API staging
  Buf x, xt, merged, catc, refm, sty, io_a, io_b;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float last_ms = -1.0f;
  // the weights' fp16 hi/lo quads for the MFMA GEMM, split on first use: (W, ldw, N, K,
  // interleave) -> cfm_split_weights output
  std::map<std::tuple<const float *, int, int, int, int>, uint4 *> wsplit;
  ~itts_cfm() {
    for (auto &kv : wsplit) (void)hipFree(kv.second);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (arena) (void)hipFree(arena);
    if (s) (void)hipStreamDestroy(s);
  }
};

namespace {

// The split quads of the weight view (W, ldw, N, K; rows interleaved when ilv > 0), made on
// the estimator's stream at its first use (the weights are constant while the estimator
// lives); nullptr on failure.
uint4 *split_weights(itts_cfm *m, const float *W, int ldw, int N, int K, int ilv = 0) {
  const auto key = std::make_tuple(W, ldw, N, K, ilv);
  auto it = m->wsplit.find(key);
  if (it != m->wsplit.end()) return it->second;
  uint4 *p = nullptr;
  if (hipMalloc(&p, itts::cfm_split_weights_quads(N, K) * sizeof(uint4)) != hipSuccess) return nullptr;
  if (itts::cfm_split_weights(W, ldw, N, K, p, m->s, ilv) != hipSuccess) {
    (void)hipFree(p);
    return nullptr;
  }
  m->wsplit.emplace(key, p);
  return p;
}

// y[M][N] = A[M][K] W[N][K]^T (+ bias[n]) + beta y (row-major; W rows ldw apart) on the
// estimator's stream: row blocks of 64 and more on the split-fp16 MFMA GEMM over the weight's split
// quads, fewer rows (the per-batch timestep, AdaLN and WaveNet-conditioning projections,
// forwards of under 64 frames) and operands the MFMA GEMM cannot take on the few-row fp32
// product.
hipError_t gemm(itts_cfm *m, int M, int N, int K, const float *A, int lda, const float *W, int ldw, float *y,
                int ldy, float beta, const float *bias, const float *yr) {
  if (M >= 64 && itts::cfm_gemm_fits(A, lda, W, ldw, K)) {
    const uint4 *wp = split_weights(m, W, ldw, N, K);
    if (!wp) return hipErrorOutOfMemory;
    return itts::cfm_gemm_split_w(1, M, N, K, A, lda, 0, wp, y, ldy, 0, beta, m->s, bias, yr);
  }
  return itts::cfm_rows_gemm(1, M, N, K, A, lda, 0, W, ldw, 0, y, ldy, 0, beta, m->s, bias, yr);
}

itts_status check_config(const itts_cfm_config &c) {
  if (c.n_heads < 1 || c.dim != 64 * c.n_heads || c.n_layers < 1 || c.inter < 1 || c.in_ch < 1 || c.style_dim < 0 ||
      c.wn_layers < 1 || c.wn_kernel < 1 || c.wn_kernel % 2 == 0 || c.dim > 8192 || c.inter > 65536)
    return cerr(ITTS_E_VALIDATION, "cfm config: unsupported shape (dim must be 64 * n_heads, wn_kernel odd)");
  return ITTS_OK;
}

itts_status ensure_rows(itts_cfm *m, int B, int T) {
  const itts_cfm_config &c = m->c;
  const size_t R = (size_t)B * T, d = c.dim, F = c.inter, NL = c.wn_layers, pad = c.wn_kernel / 2;
  const size_t na = 2 * (size_t)c.n_layers + 1;
  CK(m->emb.ensure(B * kFreqDim));
  CK(m->th.ensure(B * d));
  CK(m->t1.ensure(B * d));
  CK(m->t2.ensure(B * d));
  CK(m->st.ensure(B * d));
  CK(m->mods.ensure(B * na * 2 * d));
  CK(m->wng.ensure(B * 2 * d * NL));
  CK(m->fmod.ensure(B * 2 * d));
  CK(m->tdev.ensure(B));
  CK(m->hA.ensure(R * d));
  CK(m->hB.ensure(R * d));
  CK(m->n.ensure(R * d));
  CK(m->qkv.ensure(R * 3 * d));
  CK(m->att.ensure(R * d));
  CK(m->gu.ensure(R * 2 * F));
  CK(m->act.ensure(R * (F > d ? F : d)));
  CK(m->xres.ensure(R * d));
  CK(m->hpad.ensure((size_t)B * (T + 2 * pad) * d));
  CK(m->acts.ensure(R * 2 * d));
  CK(m->rs.ensure(R * 2 * d));
  CK(m->oacc.ensure(R * d));
  CK(m->v.ensure(R * c.in_ch));
  for (auto &b : m->skips) CK(b.ensure(R * d));
  CK(m->kvs.ensure(((size_t)cfm_kv_split_halves(B, T, c.n_heads) + 1) / 2));  // 16-bit values, float units
  const size_t S = (size_t)cfm_attn_splits(B, T, c.n_heads, m->n_cu);
  if (S > 1) {
    CK(m->apo.ensure(S * R * d));
    CK(m->aml.ensure(S * R * c.n_heads * 2));
  }
  if (m->rope_T != T) {
    CK(m->rope.ensure((size_t)T * 64));
    CK(cfm_rope_table(T, m->rope.p, m->s));
    m->rope_T = T;
  }
  return ITTS_OK;
}

// TimestepEmbedder::forward (cfm.rs:141-146) for embedder e on the device t [B] -> out [B][d]
itts_status timestep(itts_cfm *m, int e, int B, float *out) {
  const int d = m->c.dim;
  hipStream_t s = m->s;
  CK(cfm_temb(m->tdev.p, B, m->emb.p, s));
  CK(gemm(m, B, d, kFreqDim, m->emb.p, kFreqDim, m->te_w0[e], kFreqDim, m->th.p, d, 0.0f, m->te_b0[e]));
  CK(cfm_silu(m->th.p, m->th.p, B * d, s));
  CK(gemm(m, B, d, d, m->th.p, d, m->te_w2[e], d, out, d, 0.0f, m->te_b2[e]));
  return ITTS_OK;
}

// forward_merged (cfm.rs:545-617) on device inputs x_t [B][T][C], merged [B][T][MD] and the
// timesteps already in m->tdev; the velocity lands in m->v as [B][T][C].
itts_status forward(itts_cfm *m, const float *x_t, const float *merged, int B, int T) {
  const itts_cfm_config &c = m->c;
  const int d = c.dim, F = c.inter, C = c.in_ch, NL = c.wn_layers, K = c.wn_kernel, pad = K / 2;
  const int MD = 2 * C + d + c.style_dim, R = B * T, Lc = c.n_layers, split = Lc / 2;
  const int na2 = (2 * Lc + 1) * 2 * d;  // packed AdaLN modulation width
  hipStream_t s = m->s;
  if (itts_status st = ensure_rows(m, B, T)) return st;
  // conditioning vectors: t1, t2, every AdaLN's (w, b), WaveNet's per-layer g, FinalLayer's (shift, scale)
  if (itts_status st = timestep(m, 0, B, m->t1.p)) return st;
  if (itts_status st = timestep(m, 1, B, m->t2.p)) return st;
  CK(gemm(m, B, na2, d, m->t1.p, d, m->ada_w, d, m->mods.p, na2, 0.0f, m->ada_b));
  CK(gemm(m, B, 2 * d * NL, d, m->t2.p, d, m->wc_w, d, m->wng.p, 2 * d * NL, 0.0f, m->wc_b));
  CK(cfm_silu(m->t1.p, m->st.p, B * d, s));
  CK(gemm(m, B, 2 * d, d, m->st.p, d, m->fa_w, d, m->fmod.p, 2 * d, 0.0f, m->fa_b));
  // h = cond_x_merge_linear(x_merged)
  float *cur = m->hA.p, *oth = m->hB.p;
  CK(gemm(m, R, d, MD, merged, MD, m->merge_w, MD, cur, d, 0.0f, m->merge_b));
  // U-ViT blocks with long skips (cfm.rs:553-563)
  int nsk = 0;
  for (int i = 0; i < Lc; i++) {
    const Block &b = m->L[i];
    float *xin = cur;
    if (i > split && nsk > 0) {  // skip_in_linear([h, skip]) as two accumulating GEMMs
      const float *sk = m->skips[--nsk].p;
      CK(gemm(m, R, d, d, cur, d, b.skip_w, 2 * d, oth, d, 0.0f, b.skip_b));
      CK(gemm(m, R, d, d, sk, d, b.skip_w + d, 2 * d, oth, d, 1.0f));
      xin = oth;
      oth = cur;
      cur = xin;
    }
    const float *mod_a = m->mods.p + (size_t)(2 * i) * 2 * d, *mod_f = m->mods.p + (size_t)(2 * i + 1) * 2 * d;
    CK(cfm_adaln(xin, m->n.p, R, T, d, mod_a, na2, b.an_w, s));
    CK(gemm(m, R, 3 * d, d, m->n.p, d, b.wqkv, d, m->qkv.p, 3 * d, 0.0f));
    CK(cfm_attention(m->qkv.p, m->rope.p, B, T, d, c.n_heads, m->att.p, m->apo.p, m->aml.p,
                     reinterpret_cast<uint16_t *>(m->kvs.p), m->n_cu, s));
    // hidden = x_in + attn: in place, except where x_in must be kept (a block of the first
    // half writes its output straight into its long-skip stash; the middle block's input
    // is the last stash) and the sum goes out of place
    if (i <= split) {
      float *dst = i < split ? m->skips[nsk].p : (cur == m->hA.p ? m->hB.p : m->hA.p);
      CK(gemm(m, R, d, d, m->att.p, d, b.wo, d, dst, d, 1.0f, nullptr, xin));
      xin = dst;
    } else {
      CK(gemm(m, R, d, d, m->att.p, d, b.wo, d, xin, d, 1.0f));
    }
    CK(cfm_adaln(xin, m->n.p, R, T, d, mod_f, na2, b.fn_w, s));
    if (R >= 64 && F % 32 == 0 && cfm_gemm_fits(m->n.p, d, b.w13, d, d)) {
      // the SwiGLU in the [w1; w3] product's epilogue, over rows interleaved per 32
      const uint4 *q13 = split_weights(m, b.w13, d, 2 * F, d, F);
      if (!q13) return cerr(ITTS_E_DEVICE, "out of device memory for the split FFN weights");
      CK(cfm_gemm_swiglu(R, F, d, m->n.p, d, q13, m->act.p, F, s));
    } else {
      CK(gemm(m, R, 2 * F, d, m->n.p, d, b.w13, d, m->gu.p, 2 * F, 0.0f));
      CK(cfm_swiglu(m->gu.p, R, F, m->act.p, s));
    }
    CK(gemm(m, R, d, F, m->act.p, F, b.w2, F, xin, d, 1.0f));  // hidden + ffn
    if (i < split) nsk++;
    if (i <= split) {  // the block's output, in its stash or in the scratch buffer that is not cur
      if (i == split) oth = cur == m->hA.p || cur == m->hB.p ? cur : (xin == m->hA.p ? m->hB.p : m->hA.p);
      cur = xin;
    }
  }
  // transformer.norm, x_res = skip_linear([h, x_t]), h = conv1(x_res)
  CK(cfm_adaln(cur, m->n.p, R, T, d, m->mods.p + (size_t)(2 * Lc) * 2 * d, na2, m->tn_w, s));
  CK(gemm(m, R, d, d, m->n.p, d, m->skl_w, d + C, m->xres.p, d, 0.0f, m->skl_b));
  CK(gemm(m, R, d, C, x_t, C, m->skl_w + d, d + C, m->xres.p, d, 1.0f));
  CK(gemm(m, R, d, d, m->xres.p, d, m->c1_w, d, oth, d, 0.0f, m->c1_b));
  // WaveNet (cfm.rs:373-408): h in a zero-padded [B][T + 2 pad][d] buffer
  CK(cfm_pad_rows(oth, B, T, d, pad, m->hpad.p, s));
  CK(hipMemsetAsync(m->oacc.p, 0, sizeof(float) * R * d, s));
  const long sp = (long)(T + 2 * pad) * d;
  for (int l = 0; l < NL; l++) {
    const WnLayer &w = m->wn[l];
    const bool last = l + 1 == NL;
    const int rso = last ? d : 2 * d;
    // all taps as one product: row t of the padded input read K * d wide (rows t .. t+K-1);
    // d is a multiple of 64, so the operands always suit the MFMA GEMM
    const uint4 *in_q = split_weights(m, w.in_w, K * d, 2 * d, K * d);
    if (!in_q) return cerr(ITTS_E_DEVICE, "out of device memory for the split WaveNet weights");
    CK(cfm_gemm_split_w(B, T, 2 * d, K * d, m->hpad.p, d, sp, in_q, m->acts.p, 2 * d, (long)T * 2 * d, 0.0f, s));
    CK(cfm_gate(m->acts.p, w.in_b, m->wng.p + (size_t)l * 2 * d, 2 * d * NL, R, T, d, m->act.p, s));
    CK(gemm(m, R, rso, d, m->act.p, d, w.rs_w, d, m->rs.p, rso, 0.0f));
    CK(cfm_res_skip(m->rs.p, w.rs_b, last ? 1 : 0, R, T, d, pad, m->hpad.p, m->oacc.p, s));
  }
  // h = wavenet + res_projection(x_res); FinalLayer; conv2
  CK(cfm_add_bias(m->oacc.p, d, m->rp_b, R, d, s));
  CK(gemm(m, R, d, d, m->xres.p, d, m->rp_w, d, m->oacc.p, d, 1.0f));
  CK(cfm_final_norm(m->oacc.p, m->n.p, R, T, d, m->fmod.p, s));
  CK(gemm(m, R, d, d, m->n.p, d, m->fl_w, d, cur, d, 0.0f, m->fl_b));
  CK(gemm(m, R, C, d, cur, d, m->c2_w, d, m->v.p, C, 0.0f, m->c2_b));
  return ITTS_OK;
}

}  // namespace

extern "C" {

itts_status itts_cfm_create(const itts_cfm_config *cfg, const char *const *names, const float *const *data,
                            const int64_t *numel, int32_t n, itts_cfm **out) {
  if (!cfg || !out || (n > 0 && (!names || !data || !numel))) return cerr(ITTS_E_VALIDATION, "cfm: null argument");
  *out = nullptr;
  if (itts_status st = check_config(*cfg)) return st;
  const itts_cfm_config c = *cfg;
  const size_t d = c.dim, F = c.inter, C = c.in_ch, NL = c.wn_layers, K = c.wn_kernel, Lc = c.n_layers;
  const size_t MD = 2 * C + d + c.style_dim;
  // arena slots: name -> (offset, count); AdaLN projections and w1/w3 packed as used
  struct Slot {
    size_t off, count;
  };
  std::map<std::string, Slot> slots;
  size_t top = 0;
  auto put = [&](const std::string &nm, size_t count) {
    slots[nm] = Slot{top, count};
    top += (count + 63) & ~size_t(63);
  };
  auto put_at = [&](const std::string &nm, size_t off, size_t count) { slots[nm] = Slot{off, count}; };
  put("cond_projection.weight", d * d);
  put("cond_projection.bias", d);
  put("cond_x_merge_linear.weight", d * MD);
  put("cond_x_merge_linear.bias", d);
  for (const char *p : {"t_embedder", "t_embedder2"}) {
    put(std::string(p) + ".mlp.layers.0.weight", d * kFreqDim);
    put(std::string(p) + ".mlp.layers.0.bias", d);
    put(std::string(p) + ".mlp.layers.2.weight", d * d);
    put(std::string(p) + ".mlp.layers.2.bias", d);
  }
  const size_t na = 2 * Lc + 1, ada_w = top;
  top += na * 2 * d * d;
  const size_t ada_b = top;
  top += (na * 2 * d + 63) & ~size_t(63);
  auto ada = [&](const std::string &p, size_t slot) {
    put_at(p + ".project_layer.weight", ada_w + slot * 2 * d * d, 2 * d * d);
    put_at(p + ".project_layer.bias", ada_b + slot * 2 * d, 2 * d);
    put(p + ".norm.weight", d);
  };
  for (size_t i = 0; i < Lc; i++) {
    const std::string p = "transformer.layers." + std::to_string(i);
    ada(p + ".attention_norm", 2 * i);
    ada(p + ".ffn_norm", 2 * i + 1);
    put(p + ".attention.wqkv.weight", 3 * d * d);
    put(p + ".attention.wo.weight", d * d);
    put_at(p + ".feed_forward.w1.weight", top, F * d);  // w3 right after w1: the packed [w1; w3]
    put_at(p + ".feed_forward.w3.weight", top + F * d, F * d);
    top += (2 * F * d + 63) & ~size_t(63);
    put(p + ".feed_forward.w2.weight", d * F);
    put(p + ".skip_in_linear.weight", d * 2 * d);
    put(p + ".skip_in_linear.bias", d);
  }
  ada("transformer.norm", 2 * Lc);
  put("skip_linear.weight", d * (d + C));
  put("skip_linear.bias", d);
  put("conv1.weight", d * d);
  put("conv1.bias", d);
  put("res_projection.weight", d * d);
  put("res_projection.bias", d);
  put("wavenet.cond_layer.weight", 2 * d * NL * d);
  put("wavenet.cond_layer.bias", 2 * d * NL);
  for (size_t i = 0; i < NL; i++) {
    const size_t rso = i + 1 == NL ? d : 2 * d;
    put("wavenet.in_layers." + std::to_string(i) + ".weight", 2 * d * K * d);
    put("wavenet.in_layers." + std::to_string(i) + ".bias", 2 * d);
    put("wavenet.res_skip_layers." + std::to_string(i) + ".weight", rso * d);
    put("wavenet.res_skip_layers." + std::to_string(i) + ".bias", rso);
  }
  put("final_layer.adaLN_modulation.layers.1.weight", 2 * d * d);
  put("final_layer.adaLN_modulation.layers.1.bias", 2 * d);
  put("final_layer.linear.weight", d * d);
  put("final_layer.linear.bias", d);
  put("conv2.weight", C * d);
  put("conv2.bias", C);
  // every required tensor exactly once, with the element count its name requires
  std::map<std::string, int> seen;
  for (int32_t i = 0; i < n; i++) {
    if (!names[i] || !data[i]) return cerr(ITTS_E_VALIDATION, "cfm: null tensor name or data at %d", i);
    auto it = slots.find(names[i]);
    if (it == slots.end()) continue;  // tensors the estimator does not use are ignored, as the filtered loader does
    if (numel[i] != (int64_t)it->second.count)
      return cerr(ITTS_E_WEIGHT, "weight load error in `%s`: %lld elements, expected %zu", names[i],
                  (long long)numel[i], it->second.count);
    if (seen.count(names[i])) return cerr(ITTS_E_WEIGHT, "weight load error in `%s`: given twice", names[i]);
    seen[names[i]] = i;
  }
  for (const auto &kv : slots)
    if (!seen.count(kv.first)) return cerr(ITTS_E_WEIGHT, "weight load error in `%s`: missing tensor", kv.first.c_str());
  auto *m = new itts_cfm();
  m->c = c;
  auto fail = [&](itts_status st) {
    delete m;
    return st;
  };
  if (hipStreamCreate(&m->s) != hipSuccess) return fail(cerr(ITTS_E_DEVICE, "hipStreamCreate failed"));
  {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&m->n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return fail(cerr(ITTS_E_DEVICE, "querying the device's compute units failed"));
  }
  if (hipMalloc(&m->arena, top * sizeof(float)) != hipSuccess)
    return fail(cerr(ITTS_E_DEVICE, "out of device memory for the CFM weights (%zu bytes)", top * sizeof(float)));
  for (const auto &kv : seen) {
    const Slot &sl = slots[kv.first];
    if (hipMemcpy(m->arena + sl.off, data[kv.second], sl.count * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
      return fail(cerr(ITTS_E_DEVICE, "copying `%s` to the device failed", kv.first.c_str()));
  }
  auto at = [&](const std::string &nm) -> const float * { return m->arena + slots[nm].off; };
  m->cond_w = at("cond_projection.weight");
  m->cond_b = at("cond_projection.bias");
  m->merge_w = at("cond_x_merge_linear.weight");
  m->merge_b = at("cond_x_merge_linear.bias");
  const char *te[2] = {"t_embedder", "t_embedder2"};
  for (int e = 0; e < 2; e++) {
    m->te_w0[e] = at(std::string(te[e]) + ".mlp.layers.0.weight");
    m->te_b0[e] = at(std::string(te[e]) + ".mlp.layers.0.bias");
    m->te_w2[e] = at(std::string(te[e]) + ".mlp.layers.2.weight");
    m->te_b2[e] = at(std::string(te[e]) + ".mlp.layers.2.bias");
  }
  m->ada_w = m->arena + ada_w;
  m->ada_b = m->arena + ada_b;
  m->tn_w = at("transformer.norm.norm.weight");
  for (size_t i = 0; i < Lc; i++) {
    const std::string p = "transformer.layers." + std::to_string(i);
    m->L.push_back(Block{at(p + ".attention.wqkv.weight"), at(p + ".attention.wo.weight"),
                         at(p + ".feed_forward.w1.weight"), at(p + ".feed_forward.w2.weight"),
                         at(p + ".skip_in_linear.weight"), at(p + ".skip_in_linear.bias"),
                         at(p + ".attention_norm.norm.weight"), at(p + ".ffn_norm.norm.weight")});
  }
  m->skl_w = at("skip_linear.weight");
  m->skl_b = at("skip_linear.bias");
  m->c1_w = at("conv1.weight");
  m->c1_b = at("conv1.bias");
  m->rp_w = at("res_projection.weight");
  m->rp_b = at("res_projection.bias");
  m->wc_w = at("wavenet.cond_layer.weight");
  m->wc_b = at("wavenet.cond_layer.bias");
  for (size_t i = 0; i < NL; i++) {
    const std::string a = "wavenet.in_layers." + std::to_string(i), b = "wavenet.res_skip_layers." + std::to_string(i);
    m->wn.push_back(WnLayer{at(a + ".weight"), at(a + ".bias"), at(b + ".weight"), at(b + ".bias")});
  }
  m->fa_w = at("final_layer.adaLN_modulation.layers.1.weight");
  m->fa_b = at("final_layer.adaLN_modulation.layers.1.bias");
  m->fl_w = at("final_layer.linear.weight");
  m->fl_b = at("final_layer.linear.bias");
  m->c2_w = at("conv2.weight");
  m->c2_b = at("conv2.bias");
  m->skips.resize(Lc / 2);
  if (hipEventCreate(&m->e0) != hipSuccess || hipEventCreate(&m->e1) != hipSuccess)
    return fail(cerr(ITTS_E_DEVICE, "hipEventCreate failed"));
  *out = m;
  return ITTS_OK;
}

void itts_cfm_destroy(itts_cfm *cfm) { delete cfm; }

itts_status itts_cfm_forward(itts_cfm *m, const float *x_t, const float *x_merged, const float *t, int32_t B,
                             int32_t T, float *out) {
  if (!m || !x_t || !x_merged || !t || !out) return cerr(ITTS_E_VALIDATION, "cfm forward: null argument");
  if (B < 1 || T < 1) return cerr(ITTS_E_VALIDATION, "x_t: expected [B, T, %d] with B, T >= 1", m->c.in_ch);
  const itts_cfm_config &c = m->c;
  const size_t R = (size_t)B * T, C = c.in_ch, MD = 2 * C + c.dim + c.style_dim;
  CK(m->io_a.ensure(R * C));
  CK(m->io_b.ensure(R * MD));
  if (itts_status st = ensure_rows(m, B, T)) return st;
  CK(hipMemcpyAsync(m->io_a.p, x_t, sizeof(float) * R * C, hipMemcpyHostToDevice, m->s));
  CK(hipMemcpyAsync(m->io_b.p, x_merged, sizeof(float) * R * MD, hipMemcpyHostToDevice, m->s));
  CK(hipMemcpyAsync(m->tdev.p, t, sizeof(float) * B, hipMemcpyHostToDevice, m->s));
  if (itts_status st = forward(m, m->io_a.p, m->io_b.p, B, T)) return st;
  CK(m->xt.ensure(R * C));
  CK(cfm_transpose_tc(m->v.p, B, T, (int)C, m->xt.p, m->s));
  CK(hipMemcpyAsync(out, m->xt.p, sizeof(float) * R * C, hipMemcpyDeviceToHost, m->s));
  CK(hipStreamSynchronize(m->s));
  return ITTS_OK;
}

itts_status itts_cfm_solve_euler(itts_cfm *m, const float *cat_condition, int32_t T_total, const float *ref_mel,
                                 int32_t T_ref, const float *style, const float *noise_z, int32_t n_timesteps,
                                 float cfg_rate, float *mel_out) {
  if (!m || !cat_condition || !style || !noise_z || !mel_out || (T_ref > 0 && !ref_mel))
    return cerr(ITTS_E_VALIDATION, "cfm solve: null argument");
  if (n_timesteps < 1) return cerr(ITTS_E_VALIDATION, "n_timesteps: n_timesteps must be >= 1");
  if (T_total < 1) return cerr(ITTS_E_VALIDATION, "cat_condition: expected [1, T_total, %d], got T_total %d", m->c.dim, T_total);
  if (T_ref < 0 || T_ref >= T_total)
    return cerr(ITTS_E_VALIDATION,
                "ref_mel: ref_mel length (%d) must be strictly less than cat_condition length (%d)", T_ref, T_total);
  const itts_cfm_config &c = m->c;
  const int d = c.dim, C = c.in_ch, S = c.style_dim, T = T_total, MD = 2 * C + d + S;
  hipStream_t s = m->s;
  m->last_ms = -1.0f;
  CK(m->x.ensure((size_t)C * T));
  CK(m->xt.ensure((size_t)2 * T * C));
  CK(m->merged.ensure((size_t)2 * T * MD));
  CK(m->catc.ensure((size_t)T * d));
  CK(m->refm.ensure((size_t)C * (T_ref > 0 ? T_ref : 1)));
  CK(m->sty.ensure((size_t)(S > 0 ? S : 1)));
  if (itts_status st = ensure_rows(m, 2, T)) return st;
  CK(hipMemcpyAsync(m->catc.p, cat_condition, sizeof(float) * T * d, hipMemcpyHostToDevice, s));
  if (T_ref > 0) CK(hipMemcpyAsync(m->refm.p, ref_mel, sizeof(float) * C * T_ref, hipMemcpyHostToDevice, s));
  if (S > 0) CK(hipMemcpyAsync(m->sty.p, style, sizeof(float) * S, hipMemcpyHostToDevice, s));
  CK(hipMemcpyAsync(m->x.p, noise_z, sizeof(float) * C * T, hipMemcpyHostToDevice, s));
  // static CFG tail (cfm.rs:682-711): prompt mel and style in row 0, cond_projection of the
  // condition in row 0 and of zeros (= its bias) in row 1
  CK(hipMemsetAsync(m->merged.p, 0, sizeof(float) * 2 * T * MD, s));
  CK(cfm_static_tail(m->merged.p, MD, C, d, S, T, m->refm.p, T_ref, m->sty.p, s));
  CK(cfm_bias_rows(m->merged.p + 2 * C, MD, m->cond_b, 2 * T, d, s));
  CK(gemm(m, T, d, d, m->catc.p, d, m->cond_w, d, m->merged.p + 2 * C, MD, 1.0f));
  CK(hipEventRecord(m->e0, s));
  const float dt = 1.0f / (float)n_timesteps;
  for (int step = 0; step < n_timesteps; step++) {
    CK(cfm_fill(m->tdev.p, 2, (float)step * dt, s));
    CK(cfm_euler_prep(m->x.p, C, T, T_ref, m->xt.p, m->merged.p, MD, s));
    if (itts_status st = forward(m, m->xt.p, m->merged.p, 2, T)) return st;
    CK(cfm_euler_update(m->x.p, m->v.p, C, T, dt, cfg_rate, s));
  }
  CK(hipEventRecord(m->e1, s));
  const int G = T - T_ref;
  CK(hipMemcpy2DAsync(mel_out, sizeof(float) * G, m->x.p + T_ref, sizeof(float) * T, sizeof(float) * G, C,
                      hipMemcpyDeviceToHost, s));
  CK(hipStreamSynchronize(s));
  float ms = 0.0f;
  CK(hipEventElapsedTime(&ms, m->e0, m->e1));
  m->last_ms = ms;
  return ITTS_OK;
}

itts_status itts_cfm_last_solve_ms(itts_cfm *m, float *ms) {
  if (!m || !ms) return cerr(ITTS_E_VALIDATION, "cfm timing: null argument");
  if (m->last_ms < 0.0f) return cerr(ITTS_E_VALIDATION, "cfm timing: no completed solve_euler call");
  *ms = m->last_ms;
  return ITTS_OK;
}

}  // extern "C"
