/*
 * itts_oracle.c — CPU restatement of the index-tts-rs Stage-1 decoder and sampler.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP decoder.  Loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the product.
 * Build with -ffp-contract=off so every fp32 multiply and add rounds on its own.
 */
#include "itts_oracle.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

struct ito_kv {
  int n_layer, n_head, max_seq, valid_len;
  int kv_bf16, mode_f64;
  void *k, *v;
};

static __thread char g_err[512];
static __thread int g_err_code;

static int set_err(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  g_err_code = code;
  return code;
}

const char *ito_last_error(void) { return g_err; }

void ito_set_threads(int32_t n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------ */
/* Number formats                                                      */
/* ------------------------------------------------------------------ */

static inline uint32_t fbits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bitsf(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE binary16 -> binary32, exact. */
float ito_half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  const uint32_t e = (h >> 10) & 0x1F, mant = h & 0x3FF;
  if (e == 0) {
    /* zero or subnormal: mant * 2^-24 is exact in binary32 */
    const float v = (float)mant * bitsf(0x33800000u); /* 2^-24 */
    return sign ? -v : v;
  }
  if (e == 31) return bitsf(sign | 0x7F800000u | (mant << 13));
  return bitsf(sign | ((e + 112) << 23) | (mant << 13));
}

/* binary32 -> binary16 with round-to-nearest-even, overflow to infinity. */
uint16_t ito_float_to_half(float f) {
  const uint32_t x = fbits(f);
  const uint32_t sign = (x >> 16) & 0x8000;
  const uint32_t ax = x & 0x7FFFFFFF;
  if (ax >= 0x7F800000u) {
    if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00);
    return (uint16_t)(sign | 0x7E00 | ((ax >> 13) & 0x3FF));
  }
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00); /* >= 65520 */
  if (ax < 0x38800000u) {                                  /* below 2^-14: subnormal */
    if (ax < 0x33000000u) return (uint16_t)sign;            /* < 2^-25 */
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7FFFFF) | 0x800000;
    const uint32_t shift = 126 - e; /* 14..24 */
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1))) h++;
    return (uint16_t)(sign | h);
  }
  uint32_t h = (ax >> 13) - (112u << 10);
  const uint32_t rem = ax & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
  return (uint16_t)(sign | h);
}

/* binary32 -> bfloat16, round-to-nearest-even; NaN stays a quiet NaN. */
uint16_t ito_float_to_bf16(float f) {
  uint32_t x = fbits(f);
  if ((x & 0x7FFFFFFF) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40);
  x += 0x7FFFu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

float ito_bf16_to_float(uint16_t b) { return bitsf((uint32_t)b << 16); }

static inline float param_at(const void *p, int pf32, size_t i) {
  return pf32 ? ((const float *)p)[i] : ito_half_to_float(((const uint16_t *)p)[i]);
}

/* Code of element (o, k): bits=8 one byte per element; bits=4 two per byte, low
 * nibble first (MLX uint32 packing, gpt.rs:235 / QUANT_BITS, viewed as LE bytes). */
static inline int code_at(const uint8_t *codes, int bits, int K, int o, int k) {
  if (bits == 8) return codes[(size_t)o * K + k];
  const uint8_t b = codes[(size_t)o * (K / 2) + k / 2];
  return (k & 1) ? (b >> 4) : (b & 0xF);
}

/* ------------------------------------------------------------------ */
/* exp: Cody-Waite reduction by ln2 and a degree-7 Taylor polynomial    */
/* ------------------------------------------------------------------ */
/* Results below FLT_MIN are flushed to +0, so no subnormal rounding enters.  This is
 * the exponential the sampler's softmax uses (sampler.rs:233-248); the device sampler
 * evaluates the identical operation sequence. */
float ito_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -87.33654022216797f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187045e-06f, r);
  float p = 1.98412698412698413e-4f;     /* 1/7! */
  p = fmaf(p, r, 1.38888888888888889e-3f); /* 1/6! */
  p = fmaf(p, r, 8.33333333333333333e-3f); /* 1/5! */
  p = fmaf(p, r, 4.16666666666666667e-2f); /* 1/4! */
  p = fmaf(p, r, 1.66666666666666667e-1f); /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const float y = ldexpf(p, (int)n);
  return y < 1.17549435082228751e-38f ? 0.0f : y;
}

/* ------------------------------------------------------------------ */
/* SamplerRng (sampler.rs:23-62): SplitMix64 on state seed ^ golden   */
/* ------------------------------------------------------------------ */
uint64_t ito_rng_init(uint64_t seed) { return seed ^ 0x9E3779B97F4A7C15ull; }

uint64_t ito_rng_next_u64(uint64_t *state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

float ito_rng_next_f32(uint64_t *state) {
  const uint32_t upper24 = (uint32_t)(ito_rng_next_u64(state) >> 40);
  return (float)upper24 * (1.0f / 16777216.0f);
}

/* ------------------------------------------------------------------ */
/* Quantiser and dequantiser                                           */
/* ------------------------------------------------------------------ */
/* Workload spec: per 64-group along K, s = (max - min) / (2^b - 1), beta = min, both
 * stored in the parameter dtype (fp16 rounds to nearest even); then
 * q = clamp(rint((w - beta) / s), 0, 2^b - 1) with the stored s, beta; s == 0 -> q = 0. */
int ito_quantize(const float *w, int32_t N, int32_t K, int32_t bits, int32_t pf32,
                 uint8_t *codes, void *scales, void *biases) {
  if (K % 64 != 0 || K <= 0 || N <= 0) return set_err(ITO_E_VALIDATION, "bad quantize shape");
  if (bits != 8 && bits != 4) return set_err(ITO_E_VALIDATION, "bits must be 8 or 4");
  const int G = K / 64;
  const float nb = bits == 8 ? 255.0f : 15.0f;
  const float qmax = nb;
  if (bits == 4) memset(codes, 0, (size_t)N * (K / 2));
#pragma omp parallel for schedule(static)
  for (int o = 0; o < N; o++) {
    for (int g = 0; g < G; g++) {
      const float *p = w + (size_t)o * K + (size_t)g * 64;
      float mn = p[0], mx = p[0];
      for (int i = 1; i < 64; i++) {
        if (p[i] < mn) mn = p[i];
        if (p[i] > mx) mx = p[i];
      }
      float s = (mx - mn) / nb, b = mn;
      const size_t gi = (size_t)o * G + g;
      if (pf32) {
        ((float *)scales)[gi] = s;
        ((float *)biases)[gi] = b;
      } else {
        const uint16_t sh = ito_float_to_half(s), bh = ito_float_to_half(b);
        ((uint16_t *)scales)[gi] = sh;
        ((uint16_t *)biases)[gi] = bh;
        s = ito_half_to_float(sh);
        b = ito_half_to_float(bh);
      }
      for (int i = 0; i < 64; i++) {
        float q = 0.0f;
        if (s != 0.0f) {
          q = rintf((p[i] - b) / s);
          if (q < 0.0f) q = 0.0f;
          if (q > qmax) q = qmax;
        }
        const int k = g * 64 + i;
        if (bits == 8) {
          codes[(size_t)o * K + k] = (uint8_t)q;
        } else {
          uint8_t *byte = codes + (size_t)o * (K / 2) + k / 2;
          *byte |= (uint8_t)((int)q << ((k & 1) * 4));
        }
      }
    }
  }
  return ITO_OK;
}

int ito_dequant(const ito_ql *ql, int32_t bits, int32_t pf32, float *out) {
  const int N = ql->N, K = ql->K, G = K / 64;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < N; o++) {
    for (int k = 0; k < K; k++) {
      const float s = param_at(ql->scales, pf32, (size_t)o * G + k / 64);
      const float b = param_at(ql->biases, pf32, (size_t)o * G + k / 64);
      const float t = (float)code_at(ql->codes, bits, K, o, k) * s;
      out[(size_t)o * K + k] = t + b;
    }
  }
  return ITO_OK;
}

float ito_gelu(float x) {
  const float x3 = x * x * x;
  const float inner = 0.7978845608028654f * (x + 0.044715f * x3);
  return 0.5f * x * (1.0f + tanhf(inner));
}

void ito_layernorm(const float *x, const float *w, const float *b, int32_t n, float eps,
                   float *y) {
  float s = 0;
  for (int i = 0; i < n; i++) s += x[i];
  const float mean = s / (float)n;
  float v = 0;
  for (int i = 0; i < n; i++) {
    const float d = x[i] - mean;
    v += d * d;
  }
  const float rstd = 1.0f / sqrtf(v / (float)n + eps);
  for (int i = 0; i < n; i++) y[i] = (x[i] - mean) * rstd * w[i] + b[i];
}

/* ------------------------------------------------------------------ */
/* Precision-generic decoder                                           */
/* ------------------------------------------------------------------ */
#define REAL float
#define SFX _f32
#define SQRT sqrtf
#define TANH tanhf
#define EXP expf
#include "oracle_model.inc"
#undef REAL
#undef SFX
#undef SQRT
#undef TANH
#undef EXP

#define REAL double
#define SFX _f64
#define SQRT sqrt
#define TANH tanh
#define EXP exp
#include "oracle_model.inc"
#undef REAL
#undef SFX
#undef SQRT
#undef TANH
#undef EXP

int ito_ql_forward(const ito_ql *ql, int32_t bits, int32_t pf32, int32_t mode, const float *x,
                   int32_t M, float *y) {
  const int N = ql->N, K = ql->K;
  if (mode == ITO_F32) {
    ql_fwd__f32(ql, bits, pf32, x, M, y);
    return ITO_OK;
  }
  double *xd = (double *)malloc(sizeof(double) * (size_t)M * K);
  double *yd = (double *)malloc(sizeof(double) * (size_t)M * N);
  for (size_t i = 0; i < (size_t)M * K; i++) xd[i] = x[i];
  ql_fwd__f64(ql, bits, pf32, xd, M, yd);
  for (size_t i = 0; i < (size_t)M * N; i++) y[i] = (float)yd[i];
  free(xd);
  free(yd);
  return ITO_OK;
}

/* ------------------------------------------------------------------ */
/* KV cache                                                            */
/* ------------------------------------------------------------------ */
int ito_kv_create(const ito_config *cfg, int32_t max_seq, int32_t kv_dtype, int32_t mode,
                  ito_kv **out) {
  if (max_seq <= 0) return set_err(ITO_E_VALIDATION, "max_seq: KV cache max_seq must be >= 1");
  ito_kv *kv = (ito_kv *)calloc(1, sizeof(ito_kv));
  if (!kv) return set_err(ITO_E_ALLOC, "out of host memory");
  kv->n_layer = cfg->n_layer;
  kv->n_head = cfg->n_head;
  kv->max_seq = max_seq;
  kv->kv_bf16 = kv_dtype == ITO_KV_BF16;
  kv->mode_f64 = mode == ITO_F64;
  const size_t n = (size_t)cfg->n_layer * cfg->n_head * max_seq * 64;
  const size_t es = kv->mode_f64 ? 8 : (kv->kv_bf16 ? 2 : 4);
  kv->k = calloc(n, es);
  kv->v = calloc(n, es);
  if (!kv->k || !kv->v) {
    ito_kv_destroy(kv);
    return set_err(ITO_E_ALLOC, "out of host memory");
  }
  *out = kv;
  return ITO_OK;
}

void ito_kv_destroy(ito_kv *kv) {
  if (!kv) return;
  free(kv->k);
  free(kv->v);
  free(kv);
}

void ito_kv_reset(ito_kv *kv) { kv->valid_len = 0; }
int32_t ito_kv_valid_len(const ito_kv *kv) { return kv->valid_len; }

int ito_kv_read(const ito_kv *kv, int32_t layer, int32_t which_v, float *out) {
  if (layer < 0 || layer >= kv->n_layer) return set_err(ITO_E_VALIDATION, "layer out of range");
  for (int h = 0; h < kv->n_head; h++) {
    for (int p = 0; p < kv->valid_len; p++) {
      float *dst = out + ((size_t)h * kv->valid_len + p) * 64;
      if (kv->mode_f64) {
        double tmp[64];
        kv_load__f64((ito_kv *)kv, which_v, layer, h, p, tmp);
        for (int e = 0; e < 64; e++) dst[e] = (float)tmp[e];
      } else {
        kv_load__f32((ito_kv *)kv, which_v, layer, h, p, dst);
      }
    }
  }
  return ITO_OK;
}

/* ------------------------------------------------------------------ */
/* Embedding (gpt.rs:535-627)                                          */
/* ------------------------------------------------------------------ */
static int validate_prefix(const ito_model *m, const int32_t *text, int32_t n_text,
                           int32_t n_cond, int32_t lang_id, const int32_t *prior,
                           int32_t n_prior) {
  const ito_config *c = &m->cfg;
  if (n_prior < 0 || n_prior + 3 > c->mel_pos_len)
    return set_err(ITO_E_VALIDATION, "codes: %d codes exceed the Mel positional capacity", n_prior);
  if (n_text <= 0) return set_err(ITO_E_VALIDATION, "text_tokens: text_tokens must not be empty");
  if (n_text + 2 > c->text_pos_len)
    return set_err(ITO_E_VALIDATION, "text_tokens: text sequence length %d exceeds %d",
                   n_text + 2, c->text_pos_len);
  if (n_cond < 0) return set_err(ITO_E_VALIDATION, "conds: negative row count");
  if (lang_id < 0 || lang_id >= c->lang_vocab)
    return set_err(ITO_E_VALIDATION, "lang_id: lang_id %d out of range 0..%d", lang_id,
                   c->lang_vocab);
  for (int i = 0; i < n_text; i++)
    if (text[i] < 0 || text[i] >= c->text_vocab)
      return set_err(ITO_E_VALIDATION, "text_tokens: id %d out of range", text[i]);
  for (int i = 0; i < n_prior; i++)
    if (prior[i] < 0 || prior[i] >= c->mel_vocab)
      return set_err(ITO_E_VALIDATION, "codes: id %d out of range", prior[i]);
  return ITO_OK;
}

int ito_sequence_embedding(const ito_model *m, const int32_t *text, int32_t n_text,
                           const float *conds, int32_t n_cond, int32_t lang_id,
                           const int32_t *prior, int32_t n_prior, float *out) {
  int rc = validate_prefix(m, text, n_text, n_cond, lang_id, prior, n_prior);
  if (rc) return rc;
  const int d = m->cfg.d_model;
  const int start_mel = m->cfg.mel_vocab - 2;
  float *row = out;
  /* conds rows carry no positional embedding (gpt.rs:592) */
  memcpy(row, conds, sizeof(float) * (size_t)n_cond * d);
  row += (size_t)n_cond * d;
  /* [START_TEXT, text..., STOP_TEXT] + lang + text_pos[j] (gpt.rs:562-583) */
  const float *le = m->lang_emb + (size_t)lang_id * d;
  for (int j = 0; j < n_text + 2; j++) {
    const int u = j == 0 ? 0 : (j == n_text + 1 ? 1 : text[j - 1]);
    const float *te = m->text_emb + (size_t)u * d;
    const float *tp = m->text_pos + (size_t)j * d;
    for (int i = 0; i < d; i++) row[i] = (te[i] + le[i]) + tp[i];
    row += d;
  }
  /* START_MEL at Mel position 0 (gpt.rs:585-590) */
  {
    const float *me = m->mel_emb + (size_t)start_mel * d;
    for (int i = 0; i < d; i++) row[i] = me[i] + m->mel_pos[i];
    row += d;
  }
  /* prior codes at Mel positions 2.. (gpt.rs:618-625) */
  for (int i = 0; i < n_prior; i++) {
    const float *me = m->mel_emb + (size_t)prior[i] * d;
    const float *mp = m->mel_pos + (size_t)(i + 2) * d;
    for (int e = 0; e < d; e++) row[e] = me[e] + mp[e];
    row += d;
  }
  return ITO_OK;
}

static int check_mode(const ito_kv *kv, int mode) {
  if ((mode == ITO_F64) != (kv->mode_f64 != 0))
    return set_err(ITO_E_VALIDATION, "kv cache was created for another precision mode");
  return ITO_OK;
}

int ito_prefill_after(const ito_model *m, ito_kv *kv, int32_t mode, const int32_t *text,
                      int32_t n_text, const float *conds, int32_t n_cond, int32_t lang_id,
                      const int32_t *prior, int32_t n_prior, float *logits) {
  int rc = check_mode(kv, mode);
  if (rc) return rc;
  rc = validate_prefix(m, text, n_text, n_cond, lang_id, prior, n_prior);
  if (rc) return rc;
  const int T = n_cond + n_text + 3 + n_prior;
  kv->valid_len = 0; /* cache.reset() precedes the stack (gpt.rs:664) */
  if (T > kv->max_seq)
    return set_err(ITO_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d",
                   T, kv->max_seq);
  float *emb = (float *)malloc(sizeof(float) * (size_t)T * m->cfg.d_model);
  if (!emb) return set_err(ITO_E_ALLOC, "out of host memory");
  ito_sequence_embedding(m, text, n_text, conds, n_cond, lang_id, prior, n_prior, emb);
  rc = mode == ITO_F64 ? prefill__f64(m, kv, emb, T, logits) : prefill__f32(m, kv, emb, T, logits);
  free(emb);
  return rc;
}

int ito_forward_rows(const ito_model *m, ito_kv *kv, int32_t mode, const float *emb, int32_t T,
                     int32_t row0, float *out) {
  int rc = check_mode(kv, mode);
  if (rc) return rc;
  if (T <= 0 || row0 < 0 || row0 >= T) return set_err(ITO_E_VALIDATION, "bad row range");
  kv->valid_len = 0;
  if (T > kv->max_seq) return set_err(ITO_E_CAPACITY, "kv_cache: sequence too long");
  return mode == ITO_F64 ? forward_rows__f64(m, kv, emb, T, row0, out)
                         : forward_rows__f32(m, kv, emb, T, row0, out);
}

int ito_replay(const ito_model *m, ito_kv *kv, int32_t mode, const float *emb, int32_t T,
               int32_t n_layers, const ito_probe *probes, int32_t n_probes, int32_t row0,
               float *logits) {
  int rc = check_mode(kv, mode);
  if (rc) return rc;
  if (T <= 0 || row0 < 0 || row0 >= T || n_layers < 1 || n_layers > m->cfg.n_layer ||
      (logits && n_layers != m->cfg.n_layer))
    return set_err(ITO_E_VALIDATION, "bad replay range");
  for (int i = 0; i < n_probes; i++) {
    const ito_probe *p = &probes[i];
    if (p->layer < 0 || p->layer >= n_layers || p->head < 0 || p->head >= m->cfg.n_head || p->q0 < 0 ||
        p->q0 >= T || p->k0 < 0 || p->k1 <= p->k0 || p->k1 > T || !p->out)
      return set_err(ITO_E_VALIDATION, "bad probe %d", i);
  }
  kv->valid_len = 0;
  if (T > kv->max_seq) return set_err(ITO_E_CAPACITY, "kv_cache: sequence too long");
  return mode == ITO_F64 ? replay__f64(m, kv, emb, T, n_layers, probes, n_probes, row0, logits)
                         : replay__f32(m, kv, emb, T, n_layers, probes, n_probes, row0, logits);
}

int ito_step(const ito_model *m, ito_kv *kv, int32_t mode, int32_t tok, int32_t pos,
             float *logits) {
  int rc = check_mode(kv, mode);
  if (rc) return rc;
  if (tok < 0 || tok >= m->cfg.mel_vocab)
    return set_err(ITO_E_VALIDATION, "mel_token_id: mel_token_id %d out of range 0..%d", tok,
                   m->cfg.mel_vocab);
  if (pos < 0 || pos >= m->cfg.mel_pos_len)
    return set_err(ITO_E_VALIDATION, "pos_idx: pos_idx %d out of range 0..%d", pos,
                   m->cfg.mel_pos_len);
  if (kv->valid_len + 1 > kv->max_seq)
    return set_err(ITO_E_CAPACITY, "kv_cache: sequence length %d exceeds KV cache capacity %d",
                   kv->valid_len + 1, kv->max_seq);
  return mode == ITO_F64 ? step__f64(m, kv, tok, pos, logits) : step__f32(m, kv, tok, pos, logits);
}

/* ------------------------------------------------------------------ */
/* Sampler (sampler.rs:66-284)                                         */
/* ------------------------------------------------------------------ */
int ito_sampling_validate(const ito_sampling *p) {
  /* config.rs: Temperature 0.05..=2, TopP 0.01..=1, TopK <= 8194,
   * RepetitionPenalty 1..=50, max_mel_tokens 1..=1815 */
  if (!isfinite(p->temperature) || !(p->temperature >= 0.05f && p->temperature <= 2.0f))
    return set_err(ITO_E_VALIDATION, "temperature: must be finite and in 0.05..=2.0");
  if (!isfinite(p->top_p) || !(p->top_p >= 0.01f && p->top_p <= 1.0f))
    return set_err(ITO_E_VALIDATION, "top_p: must be finite and in 0.01..=1.0");
  if (p->top_k > 8194) return set_err(ITO_E_VALIDATION, "top_k: must be <= 8194");
  if (!isfinite(p->repetition_penalty) ||
      !(p->repetition_penalty >= 1.0f && p->repetition_penalty <= 50.0f))
    return set_err(ITO_E_VALIDATION, "repetition_penalty: must be finite and in 1.0..=50.0");
  if (p->max_mel_tokens < 1 || p->max_mel_tokens > 1815)
    return set_err(ITO_E_VALIDATION, "max_mel_tokens: must be in 1..=1815");
  return ITO_OK;
}

/* SeenTokenBitSet::new_with_initial_tokens: {STOP_TEXT_TOKEN 1, START_MEL_TOKEN}
 * (sampler.rs:110-115); START_MEL is 8192 for the 8194-entry Mel vocabulary. */
void ito_seen_init(uint64_t *w, int32_t start_mel) {
  memset(w, 0, 129 * sizeof(uint64_t));
  ito_seen_insert(w, 1);
  ito_seen_insert(w, start_mel);
}

void ito_seen_insert(uint64_t *w, int32_t tok) {
  if (tok >= 0 && tok < 129 * 64) w[tok / 64] |= 1ull << (tok % 64);
}

void ito_apply_repetition_penalty(const uint64_t *w, float *logits, int32_t n, float p) {
  if (fabsf(p - 1.0f) <= 1.1920928955078125e-7f) return;
  for (int wi = 0; wi < 129; wi++) {
    uint64_t bits = w[wi];
    while (bits) {
      const int b = __builtin_ctzll(bits);
      const int tid = wi * 64 + b;
      if (tid < n) {
        if (logits[tid] < 0.0f) logits[tid] = logits[tid] * p;
        else logits[tid] = logits[tid] / p;
      }
      bits &= bits - 1;
    }
  }
}

int32_t ito_argmax_finite(const float *logits, int32_t n) {
  int32_t best = 0;
  float bv = -INFINITY;
  for (int i = 0; i < n; i++)
    if (isfinite(logits[i]) && logits[i] > bv) {
      bv = logits[i];
      best = i;
    }
  return best;
}

typedef struct {
  int32_t id;
  float v;
} cand_t;

/* Descending by value (-0 == +0, as partial_cmp), ties by ascending id: a total order
 * that fixes the order the reference leaves to its unstable sort. */
static int cand_cmp(const void *pa, const void *pb) {
  const cand_t *a = (const cand_t *)pa, *b = (const cand_t *)pb;
  if (a->v > b->v) return -1;
  if (a->v < b->v) return 1;
  return (a->id > b->id) - (a->id < b->id);
}

int ito_sample_next_token(float *logits, int32_t n, const uint64_t *seen, const ito_sampling *p,
                          uint64_t *rng, int32_t *tok_out) {
  if (n <= 0) return set_err(ITO_E_VALIDATION, "logits: logits slice must not be empty");
  ito_apply_repetition_penalty(seen, logits, n, p->repetition_penalty);
  if (p->greedy) {
    *tok_out = ito_argmax_finite(logits, n);
    return ITO_OK;
  }
  const float inv_temp = 1.0f / p->temperature;
  cand_t *c = (cand_t *)malloc(sizeof(cand_t) * (size_t)n);
  float *pr = (float *)malloc(sizeof(float) * (size_t)n);
  if (!c || !pr) {
    free(c);
    free(pr);
    return set_err(ITO_E_ALLOC, "out of host memory");
  }
  for (int i = 0; i < n; i++) {
    c[i].id = i;
    c[i].v = isfinite(logits[i]) ? logits[i] * inv_temp : -INFINITY;
  }
  const int k = (p->top_k == 0) ? n : ((int)p->top_k < n ? (int)p->top_k : n);
  qsort(c, (size_t)n, sizeof(cand_t), cand_cmp);
  const float mx = isfinite(c[0].v) ? c[0].v : 0.0f;
  float prob_sum = 0.0f;
  for (int i = 0; i < k; i++) {
    pr[i] = isfinite(c[i].v) ? ito_expf(c[i].v - mx) : 0.0f;
    prob_sum += pr[i];
  }
  int32_t result;
  if (prob_sum <= 0.0f || !isfinite(prob_sum)) {
    result = c[0].id;
  } else {
    float cum = 0.0f;
    int active = k;
    for (int i = 0; i < k; i++) {
      const float norm = pr[i] / prob_sum;
      if (i > 0 && cum > p->top_p) {
        active = i;
        break;
      }
      cum += norm;
    }
    float active_sum = 0.0f;
    for (int i = 0; i < active; i++) active_sum += pr[i];
    if (active_sum <= 0.0f || !isfinite(active_sum)) {
      result = c[0].id;
    } else {
      const float draw = ito_rng_next_f32(rng) * active_sum;
      float acc = 0.0f;
      result = c[active - 1].id;
      for (int i = 0; i < active; i++) {
        acc += pr[i];
        if (draw <= acc) {
          result = c[i].id;
          break;
        }
      }
    }
  }
  free(c);
  free(pr);
  *tok_out = result;
  return ITO_OK;
}

/* generate_codes_after (sampler.rs:340-392). */
int ito_generate_codes_after(const ito_model *m, ito_kv *kv, int32_t mode, const int32_t *text,
                             int32_t n_text, const float *conds, int32_t n_cond,
                             int32_t lang_id, const int32_t *prior, int32_t n_prior,
                             int32_t min_codes, const ito_sampling *p, uint64_t *rng,
                             int32_t *codes_out, int32_t codes_cap, int32_t *n_codes,
                             float *first_logits) {
  int rc = ito_sampling_validate(p);
  if (rc) return rc;
  const int V = m->cfg.mel_vocab, stop = V - 1;
  int room = m->cfg.mel_pos_len - 3 - n_prior;
  if (room < 0) room = 0;
  const int max_steps = (int)p->max_mel_tokens < room ? (int)p->max_mel_tokens : room;
  if (max_steps == 0)
    return set_err(ITO_E_VALIDATION,
                   "max_mel_tokens: no Mel positions left to generate (max_mel_tokens is 0 or "
                   "the prior codes fill the capacity)");
  if (codes_cap < max_steps) return set_err(ITO_E_VALIDATION, "codes_out: capacity too small");
  float *logits = (float *)malloc(sizeof(float) * (size_t)V);
  if (!logits) return set_err(ITO_E_ALLOC, "out of host memory");
  rc = ito_prefill_after(m, kv, mode, text, n_text, conds, n_cond, lang_id, prior, n_prior,
                         logits);
  if (rc) {
    free(logits);
    return rc;
  }
  if (first_logits) memcpy(first_logits, logits, sizeof(float) * (size_t)V);
  uint64_t seen[129];
  ito_seen_init(seen, V - 2);
  int n = 0;
  for (int s = 0; s < max_steps; s++) {
    if (n < min_codes) logits[stop] = -INFINITY;
    int32_t tok;
    rc = ito_sample_next_token(logits, V, seen, p, rng, &tok);
    if (rc) break;
    if (tok == stop) break;
    codes_out[n++] = tok;
    ito_seen_insert(seen, tok);
    if (s + 1 < max_steps) {
      rc = ito_step(m, kv, mode, tok, n_prior + s + 2, logits);
      if (rc) break;
    }
  }
  free(logits);
  *n_codes = n;
  return rc;
}

/* ------------------------------------------------------------------ */
/* Stage-2 CFM DiT estimator and Euler solver                          */
/* ------------------------------------------------------------------ */
#include "cfm_oracle.inc"
