//! Raw `extern "C"` bindings to `libitts_hip` (declared in `include/itts_hip.h`).
//!
//! The reference's core crate forbids `unsafe` (`crates/core/src/lib.rs:19`), so the FFI
//! lives in this separate crate and the safe wrappers in `core-hip`.  Every item mirrors
//! the C header one to one: `#[repr(C)]` structs with the same fields in the same order,
//! enums passed as `i32`, handles as opaque types.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_void};

/// `itts_status`: 0 on success, else an `ITTS_E_*` code (message in `itts_last_error`).
pub type itts_status = i32;
pub const ITTS_OK: itts_status = 0;
/// `IndexTtsError::Validation` (gpt.rs:536-560, 707-718).
pub const ITTS_E_VALIDATION: itts_status = 1;
/// `IndexTtsError::WeightLoad` (loader.rs:321-329).
pub const ITTS_E_WEIGHT: itts_status = 2;
/// `IndexTtsError::Mlx`: the device failed.
pub const ITTS_E_DEVICE: itts_status = 3;
/// `Validation { field: "kv_cache" }`: KV overflow (gpt.rs:157-165).
pub const ITTS_E_CAPACITY: itts_status = 4;
pub const ITTS_E_INTERNAL: itts_status = 5;

/// `itts_dtype`.
pub type itts_dtype = i32;
pub const ITTS_F16: itts_dtype = 1;
pub const ITTS_F32: itts_dtype = 2;
pub const ITTS_BF16: itts_dtype = 3;

/// `itts_decode_path`.
pub type itts_decode_path = i32;
pub const ITTS_DECODE_AUTO: itts_decode_path = 0;
pub const ITTS_DECODE_MULTI: itts_decode_path = 1;
pub const ITTS_DECODE_PERSISTENT: itts_decode_path = 2;

pub const ITTS_ABI_VERSION: i32 = 1;

/// Decoder shape (gpt.rs:31-54).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct itts_config {
    pub n_layer: i32,
    pub d_model: i32,
    pub n_head: i32,
    pub d_ffn: i32,
    pub mel_vocab: i32,
    pub text_vocab: i32,
    pub lang_vocab: i32,
    pub mel_pos_len: i32,
    pub text_pos_len: i32,
    pub quant_bits: i32,
    pub param_dtype: i32,
}

/// One `QuantizedLinear` (gpt.rs:221-264): the U32 codes viewed as bytes, scales and
/// biases `[N][K/64]` in the config's param dtype, bias f32 `[N]` (host memory).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct itts_qlinear {
    pub codes: *const c_void,
    pub scales: *const c_void,
    pub biases: *const c_void,
    pub bias: *const f32,
}

/// `gpt.h.{i}.*` (Gpt2Block::from_weights, gpt.rs:269-323).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct itts_layer_weights {
    pub ln1_w: *const f32,
    pub ln1_b: *const f32,
    pub c_attn: itts_qlinear,
    pub c_proj: itts_qlinear,
    pub ln2_w: *const f32,
    pub ln2_b: *const f32,
    pub c_fc: itts_qlinear,
    pub mlp_c_proj: itts_qlinear,
}

/// All decoder tensors (Gpt::from_weights, gpt.rs:477-515).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct itts_weights {
    pub config: itts_config,
    pub text_embedding: *const f32,
    pub lang_embedding: *const f32,
    pub mel_embedding: *const f32,
    pub mel_pos_embedding: *const f32,
    pub text_pos_embedding: *const f32,
    pub layers: *const itts_layer_weights,
    pub ln_f_w: *const f32,
    pub ln_f_b: *const f32,
    pub final_norm_w: *const f32,
    pub final_norm_b: *const f32,
    pub mel_head: itts_qlinear,
}

/// `SamplingParams` (config.rs:1283-1321) with its newtypes unwrapped.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct itts_sampling {
    pub greedy: i32,
    pub temperature: f32,
    pub top_p: f32,
    pub top_k: u32,
    pub repetition_penalty: f32,
    pub max_mel_tokens: u32,
}

/// `CodePrompt` (sampler.rs:287-301); conds `[n_cond][d_model]` f32.
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct itts_code_prompt {
    pub text_tokens: *const i32,
    pub n_text: i32,
    pub conds: *const f32,
    pub n_cond: i32,
    pub lang_id: i32,
    pub prior_codes: *const i32,
    pub n_prior: i32,
    pub min_codes: i32,
}

/// Device-side timing of the last generate call.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct itts_timing {
    pub prefill_ms: f32,
    pub decode_ms: f32,
    pub prefill_rows: i32,
    pub decode_steps: i32,
    pub samples: i32,
}

/// CFM estimator shape (cfm.rs:36-61).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct itts_cfm_config {
    pub dim: i32,
    pub n_layers: i32,
    pub n_heads: i32,
    pub inter: i32,
    pub in_ch: i32,
    pub style_dim: i32,
    pub wn_layers: i32,
    pub wn_kernel: i32,
}

/// Opaque decoder handle.
#[repr(C)]
pub struct itts_gpt {
    _private: [u8; 0],
}
/// Opaque KV cache handle.
#[repr(C)]
pub struct itts_kv {
    _private: [u8; 0],
}
/// Opaque CFM estimator handle.
#[repr(C)]
pub struct itts_cfm {
    _private: [u8; 0],
}

#[link(name = "itts_hip")]
extern "C" {
    pub fn itts_version() -> *const c_char;
    pub fn itts_last_error() -> *const c_char;
    pub fn itts_config_default() -> itts_config;
    pub fn itts_sampling_default() -> itts_sampling;
    pub fn itts_sampling_validate(p: *const itts_sampling) -> itts_status;

    pub fn itts_gpt_create(w: *const itts_weights, out: *mut *mut itts_gpt) -> itts_status;
    pub fn itts_gpt_load_safetensors(path: *const c_char, out: *mut *mut itts_gpt) -> itts_status;
    pub fn itts_gpt_destroy(gpt: *mut itts_gpt);
    pub fn itts_gpt_num_layers(gpt: *const itts_gpt) -> i32;
    pub fn itts_gpt_config(gpt: *const itts_gpt) -> itts_config;
    pub fn itts_gpt_max_cond(gpt: *const itts_gpt) -> i32;
    pub fn itts_gpt_stream(gpt: *const itts_gpt) -> *mut c_void;
    pub fn itts_gpt_set_decode_path(gpt: *mut itts_gpt, path: itts_decode_path) -> itts_status;

    pub fn itts_kv_create(gpt: *mut itts_gpt, max_seq: i32, kv_dtype: itts_dtype, out: *mut *mut itts_kv)
        -> itts_status;
    pub fn itts_kv_destroy(kv: *mut itts_kv);
    pub fn itts_kv_reset(kv: *mut itts_kv);
    pub fn itts_kv_valid_len(kv: *const itts_kv) -> i32;
    pub fn itts_kv_max_seq(kv: *const itts_kv) -> i32;
    pub fn itts_kv_read(kv: *const itts_kv, layer: i32, which_v: i32, out: *mut f32) -> itts_status;
    pub fn itts_kv_decode_path(kv: *const itts_kv) -> itts_decode_path;

    pub fn itts_gpt_prefill(gpt: *mut itts_gpt, kv: *mut itts_kv, text_tokens: *const i32, n_text: i32,
                            conds: *const f32, n_cond: i32, lang_id: i32, logits_out: *mut f32) -> itts_status;
    pub fn itts_gpt_prefill_after(gpt: *mut itts_gpt, kv: *mut itts_kv, text_tokens: *const i32, n_text: i32,
                                  conds: *const f32, n_cond: i32, lang_id: i32, prior_codes: *const i32,
                                  n_prior: i32, logits_out: *mut f32) -> itts_status;
    pub fn itts_gpt_step(gpt: *mut itts_gpt, kv: *mut itts_kv, mel_token_id: i32, pos_idx: i32,
                         logits_out: *mut f32) -> itts_status;

    pub fn itts_gpt_teacher_forced(gpt: *mut itts_gpt, kv: *mut itts_kv, text_tokens: *const i32, n_text: i32,
                                   conds: *const f32, n_cond: i32, lang_id: i32, codes: *const i32,
                                   n_codes: i32, log_probs_out: *mut f32, attention_out: *mut f32)
        -> itts_status;
    pub fn itts_gpt_alignment_attention(gpt: *mut itts_gpt, kv: *mut itts_kv, text_tokens: *const i32,
                                        n_text: i32, conds: *const f32, n_cond: i32, lang_id: i32,
                                        prior_codes: *const i32, n_prior: i32, codes: *const i32,
                                        n_codes: i32, attention_out: *mut f32) -> itts_status;
    pub fn itts_gpt_set_alignment_heads(gpt: *mut itts_gpt, layer_head_pairs: *const i32, n_pairs: i32)
        -> itts_status;
    pub fn itts_gpt_forward_logits(gpt: *mut itts_gpt, prompts: *const itts_code_prompt, batch: i32,
                                   logits_out: *mut f32) -> itts_status;

    pub fn itts_rng_new(seed: u64) -> u64;
    pub fn itts_rng_next_u64(state: *mut u64) -> u64;
    pub fn itts_rng_next_f32(state: *mut u64) -> f32;
    pub fn itts_seen_init(words: *mut u64);
    pub fn itts_seen_insert(words: *mut u64, token_id: i32);
    pub fn itts_sample_next_token(gpt: *mut itts_gpt, logits: *mut f32, n: i32, seen: *const u64,
                                  p: *const itts_sampling, rng_state: *mut u64, token_out: *mut i32)
        -> itts_status;
    pub fn itts_sample_next_token_noalloc(gpt: *mut itts_gpt, logits: *mut f32, n: i32, seen: *const u64,
                                          p: *const itts_sampling, rng_state: *mut u64, token_out: *mut i32)
        -> itts_status;
    pub fn itts_generate_codes_after(gpt: *mut itts_gpt, kv: *mut itts_kv, prompt: *const itts_code_prompt,
                                     p: *const itts_sampling, rng_state: *mut u64, codes_out: *mut i32,
                                     codes_cap: i32, n_codes: *mut i32) -> itts_status;
    pub fn itts_gpt_step_batch(gpt: *mut itts_gpt, caches: *const *mut itts_kv, batch: i32, tokens: *const i32,
                               positions: *const i32, logits_out: *mut f32) -> itts_status;
    pub fn itts_generate_codes_batch(gpt: *mut itts_gpt, caches: *const *mut itts_kv,
                                     prompts: *const itts_code_prompt, params: *const itts_sampling, batch: i32,
                                     rng_states: *mut u64, codes_out: *mut i32, codes_cap: i32,
                                     n_codes: *mut i32) -> itts_status;
    pub fn itts_kv_last_timing(kv: *const itts_kv, out: *mut itts_timing) -> itts_status;
    pub fn itts_generate_codes(gpt: *mut itts_gpt, kv: *mut itts_kv, text_tokens: *const i32, n_text: i32,
                               conds: *const f32, n_cond: i32, lang_id: i32, p: *const itts_sampling,
                               rng_state: *mut u64, codes_out: *mut i32, codes_cap: i32, n_codes: *mut i32)
        -> itts_status;

    pub fn itts_quantize(w: *const f32, n: i32, k: i32, bits: i32, param_dtype: itts_dtype, codes: *mut c_void,
                         scales: *mut c_void, biases: *mut c_void) -> itts_status;
    pub fn itts_dequantize(gpt: *mut itts_gpt, ql: *const itts_qlinear, n: i32, k: i32, bits: i32,
                           param_dtype: itts_dtype, out: *mut f32) -> itts_status;
    pub fn itts_qlinear_forward(gpt: *mut itts_gpt, ql: *const itts_qlinear, n: i32, k: i32, bits: i32,
                                param_dtype: itts_dtype, x: *const f32, m: i32, y: *mut f32) -> itts_status;
    pub fn itts_decode_timing(gpt: *mut itts_gpt, kv: *mut itts_kv, mel_token_id: i32, pos_idx: i32,
                              n_steps: i32, ms_per_step: *mut f32) -> itts_status;

    pub fn itts_cfm_create(cfg: *const itts_cfm_config, names: *const *const c_char, data: *const *const f32,
                           numel: *const i64, n: i32, out: *mut *mut itts_cfm) -> itts_status;
    pub fn itts_cfm_destroy(cfm: *mut itts_cfm);
    pub fn itts_cfm_forward(cfm: *mut itts_cfm, x_t: *const f32, x_merged: *const f32, t: *const f32, b: i32,
                            t_len: i32, out: *mut f32) -> itts_status;
    pub fn itts_cfm_solve_euler(cfm: *mut itts_cfm, cat_condition: *const f32, t_total: i32, ref_mel: *const f32,
                                t_ref: i32, style: *const f32, noise_z: *const f32, n_timesteps: i32,
                                cfg_rate: f32, mel_out: *mut f32) -> itts_status;
    pub fn itts_cfm_last_solve_ms(cfm: *mut itts_cfm, ms: *mut f32) -> itts_status;
}
