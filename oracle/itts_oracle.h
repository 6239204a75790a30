/*
 * itts_oracle — CPU restatement of the index-tts-rs Stage-1 GPT decoder and of the
 * Stage-2 CFM DiT estimator with its Euler solver.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP decoder is
 * compared against.  Only tests/, __graft_entry__.smoke() and the cpu_baseline leg
 * of bench.py may load it; the product library never links or calls it.
 *
 * It restates, in plain C, the semantics of (paths relative to the reference repo):
 *   crates/core/src/models/gpt.rs      QuantizedLinear 221-264, Gpt2Block::forward 325-384,
 *                                      prefix/sequence embedding 535-627, prefill_after 655-696,
 *                                      step 706-754, KvCache 76-217
 *   crates/core/src/models/sampler.rs  SamplerRng 23-62, SeenTokenBitSet 66-158,
 *                                      sample_next_token 191-284, generate_codes_after 340-392,
 *                                      argmax_finite 395-405
 *   crates/core/src/config.rs          sampling parameter ranges 454-683, 1283-1321
 * The arithmetic those call sites delegate to MLX (quantized_matmul, fast::layer_norm,
 * scaled_dot_product_attention, gelu_approximate) is restated from its published
 * definition; MLX itself (mlx-rs 0.33.0 / mlx-sys 0.7.0) is not vendored in the reference.
 *
 * Two arithmetic modes of the decoder:
 *   ITO_F32  fp32 activations and accumulation, dequantised weight w = s*q + b rounded
 *            twice (no FMA contraction), like MLX's fp32 quantized_matmul.
 *   ITO_F64  the same algorithm in double precision ("truth"), used to flag
 *            ill-conditioned steps (tiny top-1/top-2 margins).
 * The sampler is defined on fp32 logits only and is bit-exact by construction.
 */
#ifndef ITTS_ORACLE_H
#define ITTS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ITO_OK = 0, ITO_E_VALIDATION = 1, ITO_E_CAPACITY = 4, ITO_E_ALLOC = 5 };
enum { ITO_F32 = 0, ITO_F64 = 1 };
enum { ITO_KV_F32 = 0, ITO_KV_BF16 = 1 };

typedef struct {
  int32_t n_layer, d_model, n_head, d_ffn;
  int32_t mel_vocab, text_vocab, lang_vocab, mel_pos_len, text_pos_len;
  int32_t bits;      /* 8 or 4 */
  int32_t param_f32; /* 0: fp16 scales/biases, 1: fp32 */
} ito_config;

/* One group-quantized linear: out[N] = x[K] . dequant(W)[N,K]^T + bias[N].
 * codes: bits=8 -> uint8 [N][K]; bits=4 -> uint8 [N][K/2], element k of a row in
 * byte k/2, low nibble first (the MLX uint32 packing viewed as little-endian bytes).
 * scales/biases: [N][K/64] as fp16 bits (uint16) or fp32. */
typedef struct {
  const uint8_t *codes;
  const void *scales;
  const void *biases;
  const float *bias;
  int32_t N, K;
} ito_ql;

typedef struct {
  const float *ln1_w, *ln1_b;
  ito_ql c_attn, c_proj;
  const float *ln2_w, *ln2_b;
  ito_ql c_fc, mlp_proj;
} ito_layer;

typedef struct {
  ito_config cfg;
  const float *text_emb, *lang_emb, *mel_emb, *mel_pos, *text_pos;
  const ito_layer *layers;
  const float *ln_f_w, *ln_f_b, *fn_w, *fn_b;
  ito_ql head;
} ito_model;

typedef struct ito_kv ito_kv;

typedef struct {
  int32_t greedy;
  float temperature;
  float top_p;
  uint32_t top_k;
  float repetition_penalty;
  uint32_t max_mel_tokens;
} ito_sampling;

/* ---- primitives (exposed for unit tests) ---- */
float ito_half_to_float(uint16_t h);
uint16_t ito_float_to_half(float f);
uint16_t ito_float_to_bf16(float f);
float ito_bf16_to_float(uint16_t b);
float ito_expf(float x);
uint64_t ito_rng_init(uint64_t seed);
uint64_t ito_rng_next_u64(uint64_t *state);
float ito_rng_next_f32(uint64_t *state);

/* MLX-affine group-64 quantiser of the workload spec. w: fp32 [N][K]. */
int ito_quantize(const float *w, int32_t N, int32_t K, int32_t bits, int32_t param_f32,
                 uint8_t *codes, void *scales, void *biases);
/* Dequantise to fp32 [N][K]: float(q)*s then +b, two roundings. */
int ito_dequant(const ito_ql *ql, int32_t bits, int32_t param_f32, float *out);
/* y[M][N] = x[M][K] . Wdeq^T + bias (+ optional fused ops are NOT applied). */
int ito_ql_forward(const ito_ql *ql, int32_t bits, int32_t param_f32, int32_t mode,
                   const float *x, int32_t M, float *y);
void ito_layernorm(const float *x, const float *w, const float *b, int32_t n, float eps,
                   float *y);
float ito_gelu(float x);

/* ---- KV cache (gpt.rs KvCache) ---- */
int ito_kv_create(const ito_config *cfg, int32_t max_seq, int32_t kv_dtype, int32_t mode,
                  ito_kv **out);
void ito_kv_destroy(ito_kv *kv);
void ito_kv_reset(ito_kv *kv);
int32_t ito_kv_valid_len(const ito_kv *kv);
/* Copies layer `layer` of K or V ([n_head][valid_len][64] as fp32) into out. */
int ito_kv_read(const ito_kv *kv, int32_t layer, int32_t which_v, float *out);

/* ---- decoder (gpt.rs prefill_after / step) ---- */
/* logits: [mel_vocab] fp32.  hidden_out (optional): final-row LN(LN(x)) [d_model]. */
int ito_prefill_after(const ito_model *m, ito_kv *kv, int32_t mode, const int32_t *text,
                      int32_t n_text, const float *conds, int32_t n_cond, int32_t lang_id,
                      const int32_t *prior, int32_t n_prior, float *logits);
int ito_step(const ito_model *m, ito_kv *kv, int32_t mode, int32_t tok, int32_t pos,
             float *logits);
/* Teacher-forced all-row logits: embed rows [T][d] given explicitly, run the causal
 * stack and return logits for rows [row0, T): out [(T-row0)][mel_vocab]. */
int ito_forward_rows(const ito_model *m, ito_kv *kv, int32_t mode, const float *emb,
                     int32_t T, int32_t row0, float *out);
/* Attention probe (gpt.rs:391-422 Gpt2Block::head_attention): softmax probabilities of
 * head `head` in layer `layer` for the queries q0..T-1 over keys 0..query (causal), sliced
 * to the key columns [k0, k1): out [(T - q0)][k1 - k0]. */
typedef struct {
  int32_t layer, head, q0, k0, k1;
  float *out;
} ito_probe;
/* Replay (gpt.rs:797-858): the causal stack over emb [T][d] through the first n_layers
 * blocks, filling the probes on the way; when logits != NULL (and n_layers is the whole
 * stack) also the head's logits of rows [row0, T): [(T-row0)][mel_vocab].  The cache is
 * scratch and left empty. */
int ito_replay(const ito_model *m, ito_kv *kv, int32_t mode, const float *emb, int32_t T,
               int32_t n_layers, const ito_probe *probes, int32_t n_probes, int32_t row0,
               float *logits);
/* Embedding rows of gpt.rs sequence_embedding: [n_cond + n_text + 3 + n_prior][d]. */
int ito_sequence_embedding(const ito_model *m, const int32_t *text, int32_t n_text,
                           const float *conds, int32_t n_cond, int32_t lang_id,
                           const int32_t *prior, int32_t n_prior, float *out);

/* ---- sampler (sampler.rs) ---- */
int ito_sampling_validate(const ito_sampling *p);
void ito_seen_init(uint64_t *words /*[129]*/, int32_t start_mel);
void ito_seen_insert(uint64_t *words, int32_t tok);
void ito_apply_repetition_penalty(const uint64_t *words, float *logits, int32_t n, float p);
int32_t ito_argmax_finite(const float *logits, int32_t n);
int ito_sample_next_token(float *logits, int32_t n, const uint64_t *seen, const ito_sampling *p,
                          uint64_t *rng_state, int32_t *tok_out);
int ito_generate_codes_after(const ito_model *m, ito_kv *kv, int32_t mode, const int32_t *text,
                             int32_t n_text, const float *conds, int32_t n_cond,
                             int32_t lang_id, const int32_t *prior, int32_t n_prior,
                             int32_t min_codes, const ito_sampling *p, uint64_t *rng_state,
                             int32_t *codes_out, int32_t codes_cap, int32_t *n_codes,
                             float *first_logits /* optional [mel_vocab] */);

/* ---- CFM DiT estimator and Euler / classifier-free-guidance solver (cfm.rs) ----
 * Restates crates/core/src/models/cfm.rs: compute_rope_freqs 73-101, TimestepEmbedder
 * 104-147, AdaLn 150-183, TransformerBlock::forward 253-313, WaveNet::forward 373-408,
 * CfmDit::forward_merged 545-617, CfmDit::solve_euler 619-760.  The MLX primitives those
 * call (rms_norm, rope with traditional=true, scaled_dot_product_attention without a mask,
 * conv1d, layer_norm without affine parameters, silu / tanh / sigmoid) are restated from
 * their published definitions.  Activations are [B][T][C] row-major; dot products
 * accumulate in double, elementwise functions are fp32 libm calls.  The head dimension is
 * 64 and the timestep frequency embedding 256 wide, as in the reference; everything else
 * comes from the configuration (the reference's values: dim 512, 13 layers, 8 heads,
 * inter 1536, in_ch 80, style 192, 8 WaveNet layers of kernel 5). */
typedef struct {
  int32_t dim, n_layers, n_heads, inter, in_ch, style_dim, wn_layers, wn_kernel;
} ito_cfm_config;
typedef struct {
  const float *proj_w, *proj_b, *norm_w; /* [2*dim][dim], [2*dim], [dim] */
} ito_cfm_adaln;
typedef struct {
  const float *w0, *b0, *w2, *b2; /* [dim][256], [dim], [dim][dim], [dim] */
} ito_cfm_temb;
typedef struct {
  ito_cfm_adaln attn_norm, ffn_norm;
  const float *wqkv;           /* [3*dim][dim] (no bias) */
  const float *wo;             /* [dim][dim] */
  const float *w1, *w3;        /* [inter][dim] */
  const float *w2;             /* [dim][inter] */
  const float *skip_w, *skip_b; /* [dim][2*dim], [dim]: used by layers > n_layers/2 */
} ito_cfm_block;
typedef struct {
  const float *in_w, *in_b; /* [2*dim][wn_kernel][dim], [2*dim] */
  const float *rs_w, *rs_b; /* [rs][dim], [rs]; rs = dim for the last layer, else 2*dim */
} ito_cfm_wn_layer;
typedef struct {
  ito_cfm_config cfg;
  const float *cond_proj_w, *cond_proj_b; /* [dim][dim], [dim] */
  const float *merge_w, *merge_b;         /* [dim][2*in_ch + dim + style], [dim] */
  ito_cfm_temb t1, t2;
  const ito_cfm_block *blocks;            /* [n_layers] */
  ito_cfm_adaln tnorm;
  const float *skip_w, *skip_b;           /* [dim][dim + in_ch], [dim] */
  const float *conv1_w, *conv1_b;         /* [dim][dim], [dim] */
  const float *res_w, *res_b;             /* [dim][dim], [dim] */
  const float *wn_cond_w, *wn_cond_b;     /* [2*dim*wn_layers][dim], [2*dim*wn_layers] */
  const ito_cfm_wn_layer *wn;             /* [wn_layers] */
  const float *fada_w, *fada_b;           /* [2*dim][dim], [2*dim] */
  const float *flin_w, *flin_b;           /* [dim][dim], [dim] */
  const float *conv2_w, *conv2_b;         /* [in_ch][dim], [in_ch] */
} ito_cfm;
/* rope(traditional=true, base 10000, offset 0) of n_heads 64-wide heads, in place on
 * x [T][n_heads*64]: pair (2i, 2i+1) of a head at position t turns by t * 10000^(-2i/64). */
void ito_cfm_rope(float *x, int32_t T, int32_t n_heads);
/* TimestepEmbedder::forward for one t: out [dim]. */
void ito_cfm_timestep(const ito_cfm_temb *e, int32_t dim, float t, float *out);
/* forward_merged: x_t [B][T][in_ch], x_merged [B][T][2*in_ch + dim + style], t [B] ->
 * out [B][in_ch][T]. */
int ito_cfm_forward(const ito_cfm *m, const float *x_t, const float *x_merged, const float *t, int32_t B,
                    int32_t T, float *out);
/* solve_euler: cat_condition [T_total][dim], ref_mel [in_ch][T_ref], style [style],
 * noise [in_ch][T_total] -> out [in_ch][T_total - T_ref]. */
int ito_cfm_solve_euler(const ito_cfm *m, const float *cat_condition, int32_t T_total, const float *ref_mel,
                        int32_t T_ref, const float *style, const float *noise, int32_t n_timesteps,
                        float cfg_rate, float *out);

const char *ito_last_error(void);
void ito_set_threads(int32_t n);

#ifdef __cplusplus
}
#endif
#endif
