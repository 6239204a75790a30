/*
 * itts_hip.h — C ABI of libitts_hip, the MI355X (gfx950) implementation of the
 * index-tts-rs Stage-1 semantic-token decoder (int8/int4 weight-only GPT-2).
 *
 * Each entry point replaces one item of the reference's decoder interface (paths are
 * relative to the reference repository):
 *   crates/core/src/models/gpt.rs       Gpt, KvCache
 *   crates/core/src/models/sampler.rs   SamplerRng, SeenTokenBitSet, sample_next_token,
 *                                       generate_codes, generate_codes_after
 *   crates/core/src/config.rs           SamplingParams and its validated newtypes
 * The reference is a Rust API (no FFI; its core crate forbids `unsafe`,
 * crates/core/src/lib.rs:19), so a thin Rust crate of `extern "C"` declarations and safe
 * wrappers (HipGpt, HipCfm) binds these symbols.
 *
 * Conventions
 *  - Every fallible call returns itts_status; itts_last_error() gives the message of the
 *    calling thread's last failure.  Validation messages start with the reference's field
 *    name ("text_tokens: ...", "mel_token_id: ...") as IndexTtsError::Validation does.
 *  - The caller owns every pointer argument (host memory); the library owns device memory.
 *  - Handles are not thread-safe; drive one itts_gpt from one host thread, as the
 *    reference's single worker thread does.  Each itts_gpt owns one HIP stream.
 */
#ifndef ITTS_HIP_H
#define ITTS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ITTS_ABI_VERSION 1

typedef enum itts_status {
  ITTS_OK = 0,
  ITTS_E_VALIDATION = 1, /* IndexTtsError::Validation (gpt.rs:536-560, 707-718) */
  ITTS_E_WEIGHT = 2,     /* IndexTtsError::WeightLoad (loader.rs:321-329) */
  ITTS_E_DEVICE = 3,     /* IndexTtsError::Mlx: the device failed (HIP error) */
  ITTS_E_CAPACITY = 4,   /* Validation{field:"kv_cache"}: KV overflow (gpt.rs:157-165) */
  ITTS_E_INTERNAL = 5
} itts_status;

typedef enum itts_dtype { ITTS_F16 = 1, ITTS_F32 = 2, ITTS_BF16 = 3 } itts_dtype;

/* Decoder shape.  The reference fixes it (gpt.rs:31-54): 24 layers, d_model 1280,
 * 20 heads of 64, d_ffn 5120, Mel vocab 8194, text vocab 60510, lang vocab 107,
 * Mel positions 1818, text positions 602, 8-bit codes in groups of 64.
 * itts_config_default() returns that shape; smaller shapes serve tests. */
typedef struct itts_config {
  int32_t n_layer;
  int32_t d_model;      /* multiple of 64; n_head * 64 */
  int32_t n_head;
  int32_t d_ffn;        /* multiple of 64 */
  int32_t mel_vocab;    /* START_MEL = mel_vocab-2, STOP_MEL = mel_vocab-1 */
  int32_t text_vocab;
  int32_t lang_vocab;
  int32_t mel_pos_len;
  int32_t text_pos_len;
  int32_t quant_bits;   /* 8, or 4 for the nibble-packed variant */
  int32_t param_dtype;  /* ITTS_F16 or ITTS_F32: dtype of scales and biases */
} itts_config;

/* One QuantizedLinear (gpt.rs:221-264) with N outputs and K inputs, host memory:
 *   codes  : the MLX uint32 weight [N][K*bits/32] viewed as bytes — bits=8: uint8 [N][K];
 *            bits=4: uint8 [N][K/2], element k in byte k/2, low nibble first.
 *   scales : [N][K/64] in param_dtype;  biases: same;  bias: fp32 [N].
 * Wdeq[o][k] = scales[o][k/64] * q[o][k] + biases[o][k/64]. */
typedef struct itts_qlinear {
  const void *codes;
  const void *scales;
  const void *biases;
  const float *bias;
} itts_qlinear;

/* gpt.h.{i}.* tensors (gpt.rs Gpt2Block::from_weights 269-323). */
typedef struct itts_layer_weights {
  const float *ln1_w, *ln1_b;   /* [d] */
  itts_qlinear c_attn;          /* N = 3d, K = d */
  itts_qlinear c_proj;          /* N = d,  K = d */
  const float *ln2_w, *ln2_b;   /* [d] */
  itts_qlinear c_fc;            /* N = d_ffn, K = d */
  itts_qlinear mlp_c_proj;      /* N = d, K = d_ffn */
} itts_layer_weights;

/* All decoder tensors (Gpt::from_weights, gpt.rs:477-515). */
typedef struct itts_weights {
  itts_config config;
  const float *text_embedding;     /* [text_vocab][d] */
  const float *lang_embedding;     /* [lang_vocab][d] */
  const float *mel_embedding;      /* [mel_vocab][d] */
  const float *mel_pos_embedding;  /* [mel_pos_len][d] */
  const float *text_pos_embedding; /* [text_pos_len][d] */
  const itts_layer_weights *layers; /* [n_layer] */
  const float *ln_f_w, *ln_f_b;
  const float *final_norm_w, *final_norm_b;
  itts_qlinear mel_head;           /* N = mel_vocab, K = d */
} itts_weights;

/* SamplingParams (config.rs:1283-1321).  Ranges are validated as the newtypes do:
 * temperature 0.05..=2 (default 0.8), top_p 0.01..=1 (0.8), top_k 0..=8194 with 0
 * meaning no cut (3), repetition_penalty 1..=50 (10), max_mel_tokens 1..=1815 (1500). */
typedef struct itts_sampling {
  int32_t greedy;
  float temperature;
  float top_p;
  uint32_t top_k;
  float repetition_penalty;
  uint32_t max_mel_tokens;
} itts_sampling;

/* CodePrompt (sampler.rs:287-301).  conds is [n_cond][d] fp32 (the reference passes
 * [1,3,1280]; any n_cond <= itts_gpt_max_cond() is accepted). */
typedef struct itts_code_prompt {
  const int32_t *text_tokens;
  int32_t n_text;
  const float *conds;
  int32_t n_cond;
  int32_t lang_id;
  const int32_t *prior_codes;
  int32_t n_prior;
  int32_t min_codes;
} itts_code_prompt;

typedef struct itts_gpt itts_gpt;
typedef struct itts_kv itts_kv;

const char *itts_version(void);
const char *itts_last_error(void);
itts_config itts_config_default(void);
itts_sampling itts_sampling_default(void);               /* SamplingParams::default */
itts_status itts_sampling_validate(const itts_sampling *p);

/* ---- Gpt (gpt.rs:438-525) ---- */
/* Gpt::from_weights: validates the shape, uploads and repacks every tensor. */
itts_status itts_gpt_create(const itts_weights *w, itts_gpt **out);
/* Gpt::load_from_path (gpt.rs:522) for gpt_int8.safetensors: the safetensors header is
 * validated as loader.rs:1410-1458 does, every tensor is checked by name, shape and dtype
 * as Gpt::from_weights does (gpt.rs:477-515, 269-323, 229-247), and the decoder shape is
 * read from the file.  U32 codes are consumed as bytes; F32 (the shipped checkpoint) or
 * F16 group parameters.  Errors: ITTS_E_WEIGHT "weight load error in `<tensor>`: ...". */
itts_status itts_gpt_load_safetensors(const char *path, itts_gpt **out);
/* Releases the caller's handle.  Live KV caches keep the decoder's device state until
 * they are destroyed too, so the two may be destroyed in either order. */
void itts_gpt_destroy(itts_gpt *gpt);
int32_t itts_gpt_num_layers(const itts_gpt *gpt);        /* Gpt::num_layers */
/* The decoder's shape (as created or read from the checkpoint). */
itts_config itts_gpt_config(const itts_gpt *gpt);
int32_t itts_gpt_max_cond(const itts_gpt *gpt);
/* The HIP stream every kernel of this decoder runs on (hipStream_t). */
void *itts_gpt_stream(const itts_gpt *gpt);

/* Decode-step implementation (no counterpart in the reference, whose step is one MLX
 * graph per token, gpt.rs:702-754).  AUTO: the persistent single-launch step wherever it
 * supports the shape (8- or 4-bit codes, fp16 or fp32 group params, bf16 or fp32 cache
 * rows, at most 12 x 216 = 2,592 cache rows, one block per compute unit), else the
 * multi-kernel step.  MULTI forces the multi-kernel step; PERSISTENT makes caches that
 * cannot use it fail at creation.  Applies to caches created afterwards. */
typedef enum itts_decode_path {
  ITTS_DECODE_AUTO = 0,
  ITTS_DECODE_MULTI = 1,
  ITTS_DECODE_PERSISTENT = 2
} itts_decode_path;
itts_status itts_gpt_set_decode_path(itts_gpt *gpt, itts_decode_path path);

/* ---- KvCache (gpt.rs:76-217) ---- */
/* KvCache::new(max_seq); kv_dtype ITTS_BF16 (workload default) or ITTS_F32 (the
 * reference's storage type).  Capacity is preallocated; no growth copies. */
itts_status itts_kv_create(itts_gpt *gpt, int32_t max_seq, itts_dtype kv_dtype, itts_kv **out);
void itts_kv_destroy(itts_kv *kv);
void itts_kv_reset(itts_kv *kv);                       /* KvCache::reset */
int32_t itts_kv_valid_len(const itts_kv *kv);          /* KvCache::valid_len */
int32_t itts_kv_max_seq(const itts_kv *kv);            /* KvCache::max_seq */
/* Copies layer `layer`'s K (which_v=0) or V (1) rows [n_head][valid_len][64] as fp32. */
itts_status itts_kv_read(const itts_kv *kv, int32_t layer, int32_t which_v, float *out);
/* The decode path this cache's steps take: ITTS_DECODE_MULTI or ITTS_DECODE_PERSISTENT. */
itts_decode_path itts_kv_decode_path(const itts_kv *kv);

/* ---- decoding (gpt.rs:636-754) ---- */
/* Gpt::prefill: logits_out receives [mel_vocab] fp32 (may be NULL). */
itts_status itts_gpt_prefill(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens,
                             int32_t n_text, const float *conds, int32_t n_cond,
                             int32_t lang_id, float *logits_out);
/* Gpt::prefill_after: continues after prior_codes (next step position n_prior + 2). */
itts_status itts_gpt_prefill_after(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens,
                                   int32_t n_text, const float *conds, int32_t n_cond,
                                   int32_t lang_id, const int32_t *prior_codes,
                                   int32_t n_prior, float *logits_out);
/* Gpt::step: one decode step for mel_token_id at position pos_idx. */
itts_status itts_gpt_step(itts_gpt *gpt, itts_kv *kv, int32_t mel_token_id, int32_t pos_idx,
                          float *logits_out);

/* ---- teacher-forced replay (gpt.rs:391-422, 756-915; align/mod.rs:37-40) ---- */
/* Gpt::teacher_forced / Gpt::code_log_probs: replays codes[0..n_codes) after the prompt
 * with teacher forcing and writes log p(codes[i] | conds, text, codes[..i]) to
 * log_probs_out [n_codes].  With attention_out set (teacher_forced), it also receives the
 * text attention [n_codes][n_text + 2] averaged over the alignment heads (row i is the
 * query that predicted codes[i]; columns <BOS>, text..., <EOS>); NULL gives
 * code_log_probs.  The cache is scratch and left empty, as in the reference. */
itts_status itts_gpt_teacher_forced(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens,
                                    int32_t n_text, const float *conds, int32_t n_cond,
                                    int32_t lang_id, const int32_t *codes, int32_t n_codes,
                                    float *log_probs_out, float *attention_out);
/* Gpt::alignment_attention: replays codes after prior_codes through the first alignment
 * layers only and writes the text attention [n_codes][n_text + 2] averaged over the
 * alignment heads.  The cache is scratch and left empty. */
itts_status itts_gpt_alignment_attention(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens,
                                         int32_t n_text, const float *conds, int32_t n_cond,
                                         int32_t lang_id, const int32_t *prior_codes,
                                         int32_t n_prior, const int32_t *codes, int32_t n_codes,
                                         float *attention_out);
/* The (layer, head) pairs averaged by the two calls above: n_pairs (1 or 2) pairs as
 * layer0, head0, layer1, head1.  Default (4, 10), (5, 10) as align/mod.rs:37; the replay
 * of alignment_attention runs layers 0..max layer. */
itts_status itts_gpt_set_alignment_heads(itts_gpt *gpt, const int32_t *layer_head_pairs, int32_t n_pairs);
/* One causal forward of a batch of prompts (each: conds, text, lang, prior codes as in
 * prefill_after) producing the logits of every row of every prompt: logits_out
 * [sum_b T_b][mel_vocab], prompts in order, T_b = n_cond + n_text + 3 + n_prior.  Rows of
 * different prompts do not attend to each other; no cache is read or written.  With
 * logits_out NULL the logits stay on the device (for timing the forward alone).  This is
 * the multi-row contraction that replay scores with, batched (no reference counterpart
 * beyond teacher_forced's all-row logits, gpt.rs:838-846). */
itts_status itts_gpt_forward_logits(itts_gpt *gpt, const itts_code_prompt *prompts, int32_t batch,
                                    float *logits_out);

/* ---- sampler (sampler.rs:19-284) ---- */
uint64_t itts_rng_new(uint64_t seed);                  /* SamplerRng::new -> state */
uint64_t itts_rng_next_u64(uint64_t *state);           /* SamplerRng::next_u64 */
float itts_rng_next_f32(uint64_t *state);              /* SamplerRng::next_f32 */
void itts_seen_init(uint64_t words[129]);              /* new_with_initial_tokens */
void itts_seen_insert(uint64_t words[129], int32_t token_id);
/* sample_next_token on the device sampler: penalises logits in place (host array,
 * written back), returns the token id and advances *rng_state as the reference does
 * (one draw per non-greedy call that reaches the draw). */
itts_status itts_sample_next_token(itts_gpt *gpt, float *logits, int32_t n,
                                   const uint64_t seen[129], const itts_sampling *p,
                                   uint64_t *rng_state, int32_t *token_out);
/* itts_sample_next_token without any device allocation: no counterpart in the reference;
 * for callers that cannot allocate device memory (tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, results and errors, but the logits, seen words and
 * RNG state are staged in a static device array of the library (one per device, about
 * 37 KB, held until the process ends) instead of buffers it allocates; n is limited to
 * 9216.  Calls on one device share that array: the library serialises its own calls,
 * and two processes have separate arrays. */
itts_status itts_sample_next_token_noalloc(itts_gpt *gpt, float *logits, int32_t n,
                                           const uint64_t seen[129], const itts_sampling *p,
                                           uint64_t *rng_state, int32_t *token_out);

/* generate_codes_after (sampler.rs:340-392) with the whole loop on the device: prefill,
 * then per step STOP masking (min_codes), repetition penalty, sampling and the next
 * decode step, replayed from a HIP graph; only the codes come back.  codes_cap must be
 * >= min(max_mel_tokens, mel_pos_len - 3 - n_prior). */
itts_status itts_generate_codes_after(itts_gpt *gpt, itts_kv *kv, const itts_code_prompt *prompt,
                                      const itts_sampling *p, uint64_t *rng_state,
                                      int32_t *codes_out, int32_t codes_cap, int32_t *n_codes);
/* ---- batched decode (independent sequences stepped together) ---- */
/* One Gpt::step for each of `batch` sequences (tokens[b] at positions[b] on caches[b]),
 * computed together: every weight byte is read once for the whole batch.  Caches must be
 * distinct, of this decoder, and of one capacity and dtype.  logits_out receives
 * [batch][mel_vocab] (may be NULL).  Per sequence the result is Gpt::step's. */
itts_status itts_gpt_step_batch(itts_gpt *gpt, itts_kv *const *caches, int32_t batch,
                                const int32_t *tokens, const int32_t *positions, float *logits_out);
/* generate_codes_after for `batch` sequences at once: each prompt is prefilled into its
 * cache, then the sequences are sampled and stepped together (one batched step per token)
 * until every one has stopped (STOP after its min_codes, or its max steps); a finished
 * sequence's row is carried but does nothing.  params and rng_states are per sequence;
 * codes_out is [batch][codes_cap] and n_codes [batch].  Per sequence, the codes and the
 * final RNG state equal generate_codes_after on that sequence alone. */
itts_status itts_generate_codes_batch(itts_gpt *gpt, itts_kv *const *caches, const itts_code_prompt *prompts,
                                      const itts_sampling *params, int32_t batch, uint64_t *rng_states,
                                      int32_t *codes_out, int32_t codes_cap, int32_t *n_codes);

/* Device-side timing of the last generate call on this cache, from HIP events recorded
 * on the decoder's stream (the counterpart of the reference's StageTimings.gpt_ms,
 * crates/core/src/engine/stream.rs:19-44, split into its two phases). */
typedef struct itts_timing {
  float prefill_ms;      /* embedding + stack + head of the prompt rows */
  float decode_ms;       /* sampling + decode steps until the end of the loop */
  int32_t prefill_rows;  /* rows of the prompt */
  int32_t decode_steps;  /* decode steps executed (KV rows appended) */
  int32_t samples;       /* tokens sampled (STOP included) */
} itts_timing;
itts_status itts_kv_last_timing(const itts_kv *kv, itts_timing *out);

/* generate_codes (sampler.rs:309-326): no prior codes, min_codes 0. */
itts_status itts_generate_codes(itts_gpt *gpt, itts_kv *kv, const int32_t *text_tokens,
                                int32_t n_text, const float *conds, int32_t n_cond,
                                int32_t lang_id, const itts_sampling *p, uint64_t *rng_state,
                                int32_t *codes_out, int32_t codes_cap, int32_t *n_codes);

/* ---- weight format (the workload's MLX-affine quantiser) ---- */
/* Quantises fp32 w [N][K] per 64-group: s=(max-min)/(2^bits-1), beta=min, both stored in
 * param_dtype, q=clamp(rint((w-beta)/s),0,2^bits-1) (s==0 -> 0).  Host, multi-threaded. */
itts_status itts_quantize(const float *w, int32_t N, int32_t K, int32_t bits,
                          itts_dtype param_dtype, void *codes, void *scales, void *biases);

/* ---- kernel-level entry points (unit parity of the device kernels) ---- */
/* Device dequantisation of one QuantizedLinear into fp32 [N][K] (host out). */
itts_status itts_dequantize(itts_gpt *gpt, const itts_qlinear *ql, int32_t N, int32_t K,
                            int32_t bits, itts_dtype param_dtype, float *out);
/* y[M][N] = x[M][K] . Wdeq^T + bias on the device; M == 1 runs the decode GEMV, M > 1
 * the prefill MFMA GEMM. */
itts_status itts_qlinear_forward(itts_gpt *gpt, const itts_qlinear *ql, int32_t N, int32_t K,
                                 int32_t bits, itts_dtype param_dtype, const float *x,
                                 int32_t M, float *y);
/* Times the decode step alone: n_steps steps, each of mel_token_id at position pos_idx,
 * enqueued back to back on the decoder's stream after the cache's valid_len rows and
 * bracketed by HIP events; *ms_per_step = elapsed / n_steps.  The cache grows by n_steps
 * rows (the last step's logits stay on the device).  No counterpart in the reference: a
 * measurement helper for the step kernel(s). */
itts_status itts_decode_timing(itts_gpt *gpt, itts_kv *kv, int32_t mel_token_id, int32_t pos_idx,
                               int32_t n_steps, float *ms_per_step);

/* ---- Stage-2 CFM DiT estimator and Euler / CFG solver (crates/core/src/models/cfm.rs) ----
 * Replaces CfmDit (cfm.rs:411-761): the 13-layer U-ViT transformer (AdaLN over RMSNorm,
 * rope, SwiGLU, long skips), skip_linear / conv1, the 8-layer WaveNet, the final layer
 * and conv2, evaluated in fp32 on the device, and the 25-step Euler integration with
 * classifier-free guidance.  Weights are fp32, by checkpoint tensor name. */
typedef struct itts_cfm itts_cfm;
typedef struct itts_cfm_config {
  /* reference values (cfm.rs:36-61): 512, 13, 8, 1536, 80, 192, 8, 5; dim == 64 * n_heads */
  int32_t dim, n_layers, n_heads, inter, in_ch, style_dim, wn_layers, wn_kernel;
} itts_cfm_config;
/* CfmDit::from_weights (cfm.rs:460-531): n tensors, names[i] the checkpoint name (e.g.
 * "transformer.layers.3.attention.wqkv.weight"), data[i] its fp32 values (host) and
 * numel[i] its element count, checked against the shape the name requires.  Errors:
 * ITTS_E_WEIGHT naming a missing tensor or one of the wrong size; ITTS_E_VALIDATION for an
 * unsupported configuration. */
itts_status itts_cfm_create(const itts_cfm_config *cfg, const char *const *names, const float *const *data,
                            const int64_t *numel, int32_t n, itts_cfm **out);
void itts_cfm_destroy(itts_cfm *cfm);
/* forward_merged (cfm.rs:545-617): x_t [B][T][in_ch], x_merged [B][T][2*in_ch+dim+style],
 * t [B] (host) -> out [B][in_ch][T] (host). */
itts_status itts_cfm_forward(itts_cfm *cfm, const float *x_t, const float *x_merged, const float *t, int32_t B,
                             int32_t T, float *out);
/* solve_euler (cfm.rs:619-760): cat_condition [T_total][dim], ref_mel [in_ch][T_ref],
 * style [style_dim], noise_z [in_ch][T_total] (host) -> mel_out [in_ch][T_total - T_ref]
 * (host).  Errors as the reference: n_timesteps >= 1, T_ref < T_total. */
itts_status itts_cfm_solve_euler(itts_cfm *cfm, const float *cat_condition, int32_t T_total, const float *ref_mel,
                                 int32_t T_ref, const float *style, const float *noise_z, int32_t n_timesteps,
                                 float cfg_rate, float *mel_out);
/* Device time of the last itts_cfm_solve_euler's integration loop (HIP events), in ms.
 * No counterpart in the reference: a measurement helper. */
itts_status itts_cfm_last_solve_ms(itts_cfm *cfm, float *ms);

#ifdef __cplusplus
}
#endif
#endif
