//! `HipGpt`, `HipKvCache`, `HipCfm`: the MI355X decoder and CFM estimator behind the
//! reference's `Gpt` / `KvCache` / `CfmDit` method signatures.
//!
//! Swap sites in the engine (reference paths):
//! - `crates/core/src/engine/actor.rs:154-157`: `Gpt::load_from_path` + `KvCache::new(2048)`
//!   become `HipGpt::load_from_path` + `HipKvCache::new`;
//! - `actor.rs:468-476, 521-522`: `generate_codes_after` (this crate's, the loop runs on
//!   the device);
//! - `actor.rs:660-677`, `actor/align.rs:131-144`: `teacher_forced`, `code_log_probs`,
//!   `alignment_attention`;
//! - `render_mel` (`actor.rs:528-532`): `CfmDit` becomes `HipCfm`.
//!
//! Errors map onto `IndexTtsError` as the reference raises them: `Validation` (the
//! library's message starts with the reference's field name), `WeightLoad`, and `Mlx` for
//! device failures.  Each handle is driven from one thread, as the reference's actor does.

use std::ffi::{CStr, CString};
use std::os::raw::c_char;
use std::os::unix::ffi::OsStrExt;
use std::path::Path;

use index_tts_rs_core::{IndexTtsError, Result, SamplingParams};
use itts_hip_sys as sys;

/// Decoder constants of the reference (gpt.rs:31-63).
pub const D_MODEL: usize = 1280;
/// `MEL_VOCAB` (8194 Mel ids, STOP = 8193).
pub const MEL_VOCAB: usize = 8194;

fn last_error() -> String {
    // SAFETY: itts_last_error returns a NUL-terminated thread-local string that stays valid
    // until the next failing call on this thread.
    unsafe { CStr::from_ptr(sys::itts_last_error()) }.to_string_lossy().into_owned()
}

/// The reference's error kinds for a library status (error.rs:30-93).
fn check(st: sys::itts_status) -> Result<()> {
    if st == sys::ITTS_OK {
        return Ok(());
    }
    let msg = last_error();
    Err(match st {
        sys::ITTS_E_VALIDATION | sys::ITTS_E_CAPACITY => {
            let field: &'static str = match msg.split(':').next().unwrap_or("decoder") {
                "text_tokens" => "text_tokens",
                "mel_token_id" => "mel_token_id",
                "pos_idx" => "pos_idx",
                "kv_cache" => "kv_cache",
                "conds" => "conds",
                "lang_id" => "lang_id",
                "codes" => "codes",
                "max_mel_tokens" => "max_mel_tokens",
                _ => "decoder",
            };
            IndexTtsError::validation(field, msg)
        }
        sys::ITTS_E_WEIGHT => IndexTtsError::weight_load("gpt_int8.safetensors", msg),
        _ => IndexTtsError::mlx(msg),
    })
}

fn i32_len(n: usize, field: &'static str) -> Result<i32> {
    i32::try_from(n).map_err(|_| IndexTtsError::validation(field, "length does not fit the device interface"))
}

/// `SamplingParams` as the library's plain struct (config.rs:1283-1321).
fn sampling(p: &SamplingParams) -> sys::itts_sampling {
    sys::itts_sampling {
        greedy: i32::from(p.greedy),
        temperature: p.temperature.get(),
        top_p: p.top_p.get(),
        top_k: p.top_k.get(),
        repetition_penalty: p.repetition_penalty.get(),
        max_mel_tokens: p.max_mel_tokens,
    }
}

/// Replaces `Gpt` (gpt.rs:438-915).
#[derive(Debug)]
pub struct HipGpt {
    raw: *mut sys::itts_gpt,
}

/// Replaces `KvCache` (gpt.rs:76-217); bf16 rows by default, f32 on request.
#[derive(Debug)]
pub struct HipKvCache {
    raw: *mut sys::itts_kv,
}

/// Replaces `SamplerRng` (sampler.rs:23-62): the same SplitMix64 state, kept here because
/// the reference's state field is private.
#[derive(Clone, Copy, Debug)]
pub struct HipSamplerRng {
    /// SplitMix64 state (`seed ^ 0x9E3779B97F4A7C15` for a new generator).
    pub state: u64,
}

impl HipSamplerRng {
    /// `SamplerRng::new(seed)`.
    pub fn new(seed: u64) -> Self {
        Self { state: seed ^ 0x9E37_79B9_7F4A_7C15 }
    }
}

/// `CodePrompt` (sampler.rs:287-301) with the conditioning as host floats
/// (`[n_cond][1280]`, the engine's `[1, 3, 1280]` array).
#[derive(Clone, Copy, Debug)]
pub struct HipCodePrompt<'a> {
    /// Text token ids (language prefix included).
    pub text_tokens: &'a [i32],
    /// Conditioning rows, row-major.
    pub conds: &'a [f32],
    /// Language token id.
    pub lang_id: i32,
    /// Codes already spoken; generation continues after them.
    pub prior_codes: &'a [i32],
    /// Fewest new codes before STOP may be sampled.
    pub min_codes: usize,
}

/// Teacher-forced replay output (`TeacherForced`, gpt.rs:428-434).
#[derive(Clone, Debug, Default)]
pub struct TeacherForced {
    /// Row-major `[codes][text + 2]` attention averaged over the alignment heads.
    pub attention: Vec<f32>,
    /// Log-probability of every code given the text and the codes before it.
    pub log_probs: Vec<f32>,
}

impl HipGpt {
    /// `Gpt::load_from_path` (gpt.rs:522): the library reads and validates
    /// `gpt_int8.safetensors` itself (header, names, shapes, dtypes).
    pub fn load_from_path(path: impl AsRef<Path>) -> Result<Self> {
        let c = CString::new(path.as_ref().as_os_str().as_bytes())
            .map_err(|_| IndexTtsError::validation("weight_path", "path contains a NUL byte"))?;
        let mut raw = std::ptr::null_mut();
        // SAFETY: c is a valid C string; raw receives a handle owned by the returned value.
        check(unsafe { sys::itts_gpt_load_safetensors(c.as_ptr(), &mut raw) })?;
        Ok(Self { raw })
    }

    /// `Gpt::from_weights` (gpt.rs:477) from already-gathered host tensors.
    ///
    /// # Safety
    /// Every pointer in `w` must reference host memory of the size the config implies for
    /// the duration of the call.
    pub unsafe fn from_raw_weights(w: &sys::itts_weights) -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        check(sys::itts_gpt_create(w, &mut raw))?;
        Ok(Self { raw })
    }

    /// `Gpt::num_layers` (gpt.rs:528).
    pub fn num_layers(&self) -> usize {
        // SAFETY: self.raw is a live handle.
        unsafe { sys::itts_gpt_num_layers(self.raw) as usize }
    }

    fn n_cond(&self, conds: &[f32]) -> Result<i32> {
        if conds.len() % D_MODEL != 0 {
            return Err(IndexTtsError::validation("conds", "conditioning must be [n, 1280] floats"));
        }
        i32_len(conds.len() / D_MODEL, "conds")
    }

    /// `Gpt::prefill` (gpt.rs:636).
    pub fn prefill(&self, text_tokens: &[i32], conds: &[f32], lang_id: i32, cache: &mut HipKvCache) -> Result<Vec<f32>> {
        self.prefill_after(text_tokens, conds, lang_id, &[], cache)
    }

    /// `Gpt::prefill_after` (gpt.rs:655).
    pub fn prefill_after(&self, text_tokens: &[i32], conds: &[f32], lang_id: i32, prior_codes: &[i32],
                         cache: &mut HipKvCache) -> Result<Vec<f32>> {
        let mut logits = vec![0f32; MEL_VOCAB];
        let n_cond = self.n_cond(conds)?;
        // SAFETY: slices are valid for their lengths; logits holds MEL_VOCAB floats.
        check(unsafe {
            sys::itts_gpt_prefill_after(self.raw, cache.raw, text_tokens.as_ptr(), i32_len(text_tokens.len(), "text_tokens")?,
                                        conds.as_ptr(), n_cond, lang_id, prior_codes.as_ptr(),
                                        i32_len(prior_codes.len(), "codes")?, logits.as_mut_ptr())
        })?;
        Ok(logits)
    }

    /// `Gpt::step` (gpt.rs:706).
    pub fn step(&self, cache: &mut HipKvCache, mel_token_id: i32, pos_idx: i32) -> Result<Vec<f32>> {
        let mut logits = vec![0f32; MEL_VOCAB];
        // SAFETY: logits holds MEL_VOCAB floats.
        check(unsafe { sys::itts_gpt_step(self.raw, cache.raw, mel_token_id, pos_idx, logits.as_mut_ptr()) })?;
        Ok(logits)
    }

    /// `Gpt::teacher_forced` (gpt.rs:766).
    pub fn teacher_forced(&self, text_tokens: &[i32], conds: &[f32], lang_id: i32, codes: &[i32],
                          cache: &mut HipKvCache) -> Result<TeacherForced> {
        let mut out = TeacherForced {
            attention: vec![0f32; codes.len() * (text_tokens.len() + 2)],
            log_probs: vec![0f32; codes.len()],
        };
        let n_cond = self.n_cond(conds)?;
        // SAFETY: output buffers hold codes * (text + 2) and codes floats.
        check(unsafe {
            sys::itts_gpt_teacher_forced(self.raw, cache.raw, text_tokens.as_ptr(), i32_len(text_tokens.len(), "text_tokens")?,
                                         conds.as_ptr(), n_cond, lang_id, codes.as_ptr(), i32_len(codes.len(), "codes")?,
                                         out.log_probs.as_mut_ptr(), out.attention.as_mut_ptr())
        })?;
        Ok(out)
    }

    /// `Gpt::code_log_probs` (gpt.rs:785): teacher_forced without the attention.
    pub fn code_log_probs(&self, text_tokens: &[i32], conds: &[f32], lang_id: i32, codes: &[i32],
                          cache: &mut HipKvCache) -> Result<Vec<f32>> {
        let mut log_probs = vec![0f32; codes.len()];
        let n_cond = self.n_cond(conds)?;
        // SAFETY: log_probs holds codes floats; a null attention output selects code_log_probs.
        check(unsafe {
            sys::itts_gpt_teacher_forced(self.raw, cache.raw, text_tokens.as_ptr(), i32_len(text_tokens.len(), "text_tokens")?,
                                         conds.as_ptr(), n_cond, lang_id, codes.as_ptr(), i32_len(codes.len(), "codes")?,
                                         log_probs.as_mut_ptr(), std::ptr::null_mut())
        })?;
        Ok(log_probs)
    }

    /// `Gpt::alignment_attention` (gpt.rs:875).
    pub fn alignment_attention(&self, text_tokens: &[i32], conds: &[f32], lang_id: i32, prior_codes: &[i32],
                               codes: &[i32], cache: &mut HipKvCache) -> Result<Vec<f32>> {
        let mut attention = vec![0f32; codes.len() * (text_tokens.len() + 2)];
        let n_cond = self.n_cond(conds)?;
        // SAFETY: attention holds codes * (text + 2) floats.
        check(unsafe {
            sys::itts_gpt_alignment_attention(self.raw, cache.raw, text_tokens.as_ptr(),
                                              i32_len(text_tokens.len(), "text_tokens")?, conds.as_ptr(), n_cond, lang_id,
                                              prior_codes.as_ptr(), i32_len(prior_codes.len(), "codes")?, codes.as_ptr(),
                                              i32_len(codes.len(), "codes")?, attention.as_mut_ptr())
        })?;
        Ok(attention)
    }
}

impl HipKvCache {
    /// `KvCache::new(max_seq)` (gpt.rs:102) with bf16 rows (the workload's cache).
    pub fn new(gpt: &HipGpt, max_seq: usize) -> Result<Self> {
        Self::with_dtype(gpt, max_seq, sys::ITTS_BF16)
    }

    /// A cache of f32 rows (the reference's storage type) or bf16 rows.
    pub fn with_dtype(gpt: &HipGpt, max_seq: usize, dtype: sys::itts_dtype) -> Result<Self> {
        let mut raw = std::ptr::null_mut();
        // SAFETY: gpt.raw is a live handle; raw receives a handle owned by the returned value.
        check(unsafe { sys::itts_kv_create(gpt.raw, i32_len(max_seq, "kv_cache")?, dtype, &mut raw) })?;
        Ok(Self { raw })
    }

    /// `KvCache::reset` (gpt.rs:131).
    pub fn reset(&mut self) {
        // SAFETY: self.raw is a live handle.
        unsafe { sys::itts_kv_reset(self.raw) }
    }

    /// `KvCache::valid_len` (gpt.rs:137).
    pub fn valid_len(&self) -> usize {
        // SAFETY: self.raw is a live handle.
        unsafe { sys::itts_kv_valid_len(self.raw) as usize }
    }

    /// `KvCache::max_seq` (gpt.rs:143).
    pub fn max_seq(&self) -> usize {
        // SAFETY: self.raw is a live handle.
        unsafe { sys::itts_kv_max_seq(self.raw) as usize }
    }
}

/// `generate_codes_after` (sampler.rs:340-392) with the whole loop on the device; `rng`
/// advances as `SamplerRng` does.
pub fn generate_codes_after(gpt: &HipGpt, prompt: &HipCodePrompt<'_>, cache: &mut HipKvCache,
                            params: &SamplingParams, rng: &mut HipSamplerRng) -> Result<Vec<i32>> {
    let cap = params.max_mel_tokens as usize;
    let mut codes = vec![0i32; cap.max(1)];
    let mut n = 0i32;
    let p = sys::itts_code_prompt {
        text_tokens: prompt.text_tokens.as_ptr(),
        n_text: i32_len(prompt.text_tokens.len(), "text_tokens")?,
        conds: prompt.conds.as_ptr(),
        n_cond: gpt.n_cond(prompt.conds)?,
        lang_id: prompt.lang_id,
        prior_codes: prompt.prior_codes.as_ptr(),
        n_prior: i32_len(prompt.prior_codes.len(), "codes")?,
        min_codes: i32_len(prompt.min_codes, "min_codes")?,
    };
    let s = sampling(params);
    // SAFETY: the prompt's slices outlive the call; codes holds cap ints.
    check(unsafe {
        sys::itts_generate_codes_after(gpt.raw, cache.raw, &p, &s, &mut rng.state, codes.as_mut_ptr(),
                                       i32_len(codes.len(), "max_mel_tokens")?, &mut n)
    })?;
    codes.truncate(n as usize);
    Ok(codes)
}

/// `sample_next_token` (sampler.rs:191) on the device sampler; `logits` are penalised in
/// place and `seen` is the `SeenTokenBitSet` words (129 x u64).
pub fn sample_next_token(gpt: &HipGpt, logits: &mut [f32], seen: &[u64; 129], params: &SamplingParams,
                         rng: &mut HipSamplerRng) -> Result<i32> {
    let s = sampling(params);
    let mut tok = 0i32;
    // SAFETY: logits and seen are valid for their lengths.
    check(unsafe {
        sys::itts_sample_next_token(gpt.raw, logits.as_mut_ptr(), i32_len(logits.len(), "logits")?, seen.as_ptr(), &s,
                                    &mut rng.state, &mut tok)
    })?;
    Ok(tok)
}

impl Drop for HipKvCache {
    fn drop(&mut self) {
        // SAFETY: the handle is released once; the decoder stays alive while caches exist.
        unsafe { sys::itts_kv_destroy(self.raw) }
    }
}

impl Drop for HipGpt {
    fn drop(&mut self) {
        // SAFETY: the handle is released once.
        unsafe { sys::itts_gpt_destroy(self.raw) }
    }
}

/// Replaces `CfmDit` (cfm.rs:411-761).
#[derive(Debug)]
pub struct HipCfm {
    raw: *mut sys::itts_cfm,
}

impl HipCfm {
    /// The reference estimator's shape (cfm.rs:36-61).
    pub const CONFIG: sys::itts_cfm_config = sys::itts_cfm_config {
        dim: 512, n_layers: 13, n_heads: 8, inter: 1536, in_ch: 80, style_dim: 192, wn_layers: 8, wn_kernel: 5,
    };

    /// `CfmDit::from_weights` (cfm.rs:460-531): every f32 tensor of `cfm_estimator` by name.
    pub fn from_tensors<'a>(tensors: impl IntoIterator<Item = (&'a str, &'a [f32])>) -> Result<Self> {
        let (names, slices): (Vec<CString>, Vec<&[f32]>) = tensors
            .into_iter()
            .map(|(n, s)| (CString::new(n).expect("tensor names contain no NUL"), s))
            .unzip();
        let name_ptrs: Vec<*const c_char> = names.iter().map(|n| n.as_ptr()).collect();
        let data: Vec<*const f32> = slices.iter().map(|s| s.as_ptr()).collect();
        let numel: Vec<i64> = slices.iter().map(|s| s.len() as i64).collect();
        let mut raw = std::ptr::null_mut();
        // SAFETY: the name and data arrays hold n valid entries for the duration of the call.
        check(unsafe {
            sys::itts_cfm_create(&Self::CONFIG, name_ptrs.as_ptr(), data.as_ptr(), numel.as_ptr(),
                                 i32_len(name_ptrs.len(), "cfm")?, &mut raw)
        })?;
        Ok(Self { raw })
    }

    /// `CfmDit::solve_euler` (cfm.rs:619-760): cat_condition `[T, 512]`, ref_mel `[80, T_ref]`,
    /// style `[192]`, noise_z `[80, T]` -> mel `[80, T - T_ref]`.
    pub fn solve_euler(&self, cat_condition: &[f32], t_total: usize, ref_mel: &[f32], t_ref: usize, style: &[f32],
                       noise_z: &[f32], n_timesteps: usize, cfg_rate: f32) -> Result<Vec<f32>> {
        if t_ref >= t_total {
            return Err(IndexTtsError::validation("ref_mel", "reference frames must be fewer than the total"));
        }
        let mut mel = vec![0f32; 80 * (t_total - t_ref)];
        // SAFETY: the inputs hold the documented sizes; mel holds 80 * (T - T_ref) floats.
        check(unsafe {
            sys::itts_cfm_solve_euler(self.raw, cat_condition.as_ptr(), i32_len(t_total, "cat_condition")?,
                                      ref_mel.as_ptr(), i32_len(t_ref, "ref_mel")?, style.as_ptr(), noise_z.as_ptr(),
                                      i32_len(n_timesteps, "n_timesteps")?, cfg_rate, mel.as_mut_ptr())
        })?;
        Ok(mel)
    }
}

impl Drop for HipCfm {
    fn drop(&mut self) {
        // SAFETY: the handle is released once.
        unsafe { sys::itts_cfm_destroy(self.raw) }
    }
}
