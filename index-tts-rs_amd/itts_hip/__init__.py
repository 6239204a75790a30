"""Python binding of libitts_hip (ctypes over the C ABI in include/itts_hip.h).

The classes mirror the reference's decoder interface so that tests read like the
reference's own (paths relative to the reference repository):

    Gpt            crates/core/src/models/gpt.rs   Gpt::{from_weights, prefill,
                                                   prefill_after, step, num_layers}
    KvCache        crates/core/src/models/gpt.rs   KvCache::{new, reset, valid_len, max_seq}
    SamplingParams crates/core/src/config.rs       SamplingParams (validated ranges)
    SamplerRng     crates/core/src/models/sampler.rs SamplerRng::{new, next_u64, next_f32}
    SeenTokenBitSet, sample_next_token, generate_codes, generate_codes_after

Errors raise ``IttsError`` carrying the status code and the library's message
(``ValidationError`` for ITTS_E_VALIDATION, ``CapacityError`` for ITTS_E_CAPACITY ...),
as the reference returns ``IndexTtsError`` variants.

The library is the product: there is no fallback.  If ``lib/libitts_hip.so`` is missing
the import fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# the in-tree build, unless ITTS_HIP_LIB names another build of the same library
LIB_PATH = os.environ.get("ITTS_HIP_LIB") or os.path.join(os.path.dirname(_HERE), "lib", "libitts_hip.so")

ITTS_OK, ITTS_E_VALIDATION, ITTS_E_WEIGHT, ITTS_E_DEVICE, ITTS_E_CAPACITY, ITTS_E_INTERNAL = range(6)
ITTS_F16, ITTS_F32, ITTS_BF16 = 1, 2, 3
ITTS_DECODE_AUTO, ITTS_DECODE_MULTI, ITTS_DECODE_PERSISTENT = 0, 1, 2

GPT_MEL_VOCAB = 8194
START_TEXT_TOKEN, STOP_TEXT_TOKEN = 0, 1
START_MEL_TOKEN, STOP_MEL_TOKEN = 8192, 8193


class IttsError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


class ValidationError(IttsError):
    pass


class WeightLoadError(IttsError):
    pass


class DeviceError(IttsError):
    pass


class CapacityError(IttsError):
    pass


_ERRORS = {ITTS_E_VALIDATION: ValidationError, ITTS_E_WEIGHT: WeightLoadError,
           ITTS_E_DEVICE: DeviceError, ITTS_E_CAPACITY: CapacityError}


class itts_config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layer", "d_model", "n_head", "d_ffn", "mel_vocab", "text_vocab", "lang_vocab",
        "mel_pos_len", "text_pos_len", "quant_bits", "param_dtype")]


class itts_qlinear(C.Structure):
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("bias", C.c_void_p)]


class itts_layer_weights(C.Structure):
    _fields_ = [("ln1_w", C.c_void_p), ("ln1_b", C.c_void_p), ("c_attn", itts_qlinear),
                ("c_proj", itts_qlinear), ("ln2_w", C.c_void_p), ("ln2_b", C.c_void_p),
                ("c_fc", itts_qlinear), ("mlp_c_proj", itts_qlinear)]


class itts_weights(C.Structure):
    _fields_ = [("config", itts_config), ("text_embedding", C.c_void_p),
                ("lang_embedding", C.c_void_p), ("mel_embedding", C.c_void_p),
                ("mel_pos_embedding", C.c_void_p), ("text_pos_embedding", C.c_void_p),
                ("layers", C.POINTER(itts_layer_weights)), ("ln_f_w", C.c_void_p),
                ("ln_f_b", C.c_void_p), ("final_norm_w", C.c_void_p),
                ("final_norm_b", C.c_void_p), ("mel_head", itts_qlinear)]


class itts_sampling(C.Structure):
    _fields_ = [("greedy", C.c_int32), ("temperature", C.c_float), ("top_p", C.c_float),
                ("top_k", C.c_uint32), ("repetition_penalty", C.c_float),
                ("max_mel_tokens", C.c_uint32)]


class itts_code_prompt(C.Structure):
    _fields_ = [("text_tokens", C.c_void_p), ("n_text", C.c_int32), ("conds", C.c_void_p),
                ("n_cond", C.c_int32), ("lang_id", C.c_int32), ("prior_codes", C.c_void_p),
                ("n_prior", C.c_int32), ("min_codes", C.c_int32)]


class itts_timing(C.Structure):
    _fields_ = [("prefill_ms", C.c_float), ("decode_ms", C.c_float), ("prefill_rows", C.c_int32),
                ("decode_steps", C.c_int32), ("samples", C.c_int32)]


class itts_cfm_config(C.Structure):
    """CFM DiT estimator shape (cfm.rs:36-61); the head dimension is 64."""
    _fields_ = [(n, C.c_int32) for n in ("dim", "n_layers", "n_heads", "inter", "in_ch", "style_dim",
                                         "wn_layers", "wn_kernel")]


_SIGS = {
    "itts_kv_last_timing": (C.c_int, [C.c_void_p, C.POINTER(itts_timing)]),
    "itts_version": (C.c_char_p, []),
    "itts_last_error": (C.c_char_p, []),
    "itts_config_default": (itts_config, []),
    "itts_sampling_default": (itts_sampling, []),
    "itts_sampling_validate": (C.c_int, [C.POINTER(itts_sampling)]),
    "itts_gpt_create": (C.c_int, [C.POINTER(itts_weights), C.POINTER(C.c_void_p)]),
    "itts_gpt_destroy": (None, [C.c_void_p]),
    "itts_gpt_load_safetensors": (C.c_int, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "itts_gpt_num_layers": (C.c_int32, [C.c_void_p]),
    "itts_gpt_config": (itts_config, [C.c_void_p]),
    "itts_gpt_max_cond": (C.c_int32, [C.c_void_p]),
    "itts_gpt_stream": (C.c_void_p, [C.c_void_p]),
    "itts_gpt_set_decode_path": (C.c_int, [C.c_void_p, C.c_int]),
    "itts_kv_create": (C.c_int, [C.c_void_p, C.c_int32, C.c_int, C.POINTER(C.c_void_p)]),
    "itts_kv_destroy": (None, [C.c_void_p]),
    "itts_kv_reset": (None, [C.c_void_p]),
    "itts_kv_valid_len": (C.c_int32, [C.c_void_p]),
    "itts_kv_max_seq": (C.c_int32, [C.c_void_p]),
    "itts_kv_read": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p]),
    "itts_kv_decode_path": (C.c_int, [C.c_void_p]),
    "itts_gpt_prefill": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                   C.c_int32, C.c_int32, C.c_void_p]),
    "itts_gpt_teacher_forced": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                          C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p,
                                          C.c_void_p]),
    "itts_gpt_alignment_attention": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                               C.c_int32, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p,
                                               C.c_int32, C.c_void_p]),
    "itts_gpt_set_alignment_heads": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32]),
    "itts_gpt_forward_logits": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p]),
    "itts_gpt_step_batch": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p]),
    "itts_generate_codes_batch": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                                            C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p]),
    "itts_gpt_prefill_after": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                                         C.c_void_p, C.c_int32, C.c_int32, C.c_void_p,
                                         C.c_int32, C.c_void_p]),
    "itts_gpt_step": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_void_p]),
    "itts_rng_new": (C.c_uint64, [C.c_uint64]),
    "itts_rng_next_u64": (C.c_uint64, [C.POINTER(C.c_uint64)]),
    "itts_rng_next_f32": (C.c_float, [C.POINTER(C.c_uint64)]),
    "itts_seen_init": (None, [C.c_void_p]),
    "itts_seen_insert": (None, [C.c_void_p, C.c_int32]),
    "itts_sample_next_token": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                         C.POINTER(itts_sampling), C.POINTER(C.c_uint64),
                                         C.POINTER(C.c_int32)]),
    "itts_sample_next_token_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                                 C.POINTER(itts_sampling), C.POINTER(C.c_uint64),
                                                 C.POINTER(C.c_int32)]),
    "itts_generate_codes_after": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(itts_code_prompt),
                                            C.POINTER(itts_sampling), C.POINTER(C.c_uint64),
                                            C.c_void_p, C.c_int32, C.POINTER(C.c_int32)]),
    "itts_generate_codes": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p,
                                      C.c_int32, C.c_int32, C.POINTER(itts_sampling),
                                      C.POINTER(C.c_uint64), C.c_void_p, C.c_int32,
                                      C.POINTER(C.c_int32)]),
    "itts_quantize": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int, C.c_void_p,
                                C.c_void_p, C.c_void_p]),
    "itts_dequantize": (C.c_int, [C.c_void_p, C.POINTER(itts_qlinear), C.c_int32, C.c_int32,
                                  C.c_int32, C.c_int, C.c_void_p]),
    "itts_qlinear_forward": (C.c_int, [C.c_void_p, C.POINTER(itts_qlinear), C.c_int32, C.c_int32,
                                       C.c_int32, C.c_int, C.c_void_p, C.c_int32, C.c_void_p]),
    "itts_decode_timing": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_int32, C.c_int32,
                                     C.POINTER(C.c_float)]),
    "itts_cfm_create": (C.c_int, [C.POINTER(itts_cfm_config), C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32,
                                  C.POINTER(C.c_void_p)]),
    "itts_cfm_destroy": (None, [C.c_void_p]),
    "itts_cfm_forward": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                   C.c_void_p]),
    "itts_cfm_solve_euler": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_void_p,
                                       C.c_void_p, C.c_int32, C.c_float, C.c_void_p]),
    "itts_cfm_last_solve_ms": (C.c_int, [C.c_void_p, C.POINTER(C.c_float)]),
}

EXPORTED_SYMBOLS = tuple(_SIGS)


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libitts_hip is not built: {LIB_PATH} is missing "
                          "(run __graft_entry__.build() or make -C index-tts-rs_amd)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _check(status: int):
    if status != ITTS_OK:
        msg = lib.itts_last_error().decode(errors="replace")
        raise _ERRORS.get(status, IttsError)(status, msg)


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def version() -> str:
    return lib.itts_version().decode()


def last_error() -> str:
    return lib.itts_last_error().decode()


# ----------------------------------------------------------------------------------
# Sampling (config.rs SamplingParams; sampler.rs SamplerRng / SeenTokenBitSet)
# ----------------------------------------------------------------------------------

@dataclass
class SamplingParams:
    greedy: bool = False
    top_k: int = 3
    top_p: float = 0.8
    temperature: float = 0.8
    repetition_penalty: float = 10.0
    max_mel_tokens: int = 1500

    def to_c(self) -> itts_sampling:
        return itts_sampling(int(bool(self.greedy)), float(self.temperature), float(self.top_p),
                             int(self.top_k), float(self.repetition_penalty),
                             int(self.max_mel_tokens))

    def validate(self):
        c = self.to_c()
        _check(lib.itts_sampling_validate(C.byref(c)))
        return self


class SamplerRng:
    """SamplerRng::new(seed): SplitMix64 on state seed ^ 0x9E3779B97F4A7C15."""

    def __init__(self, seed: int = 0, state: int | None = None):
        self.state = C.c_uint64(lib.itts_rng_new(seed & (2**64 - 1)) if state is None else state)

    def next_u64(self) -> int:
        return lib.itts_rng_next_u64(C.byref(self.state))

    def next_f32(self) -> float:
        return lib.itts_rng_next_f32(C.byref(self.state))


class SeenTokenBitSet:
    def __init__(self, words: np.ndarray | None = None):
        if words is None:
            self.words = np.zeros(129, dtype=np.uint64)
            lib.itts_seen_init(_ptr(self.words))
        else:
            self.words = np.ascontiguousarray(words, dtype=np.uint64).copy()

    @classmethod
    def empty(cls):
        return cls(np.zeros(129, dtype=np.uint64))

    def insert(self, token_id: int):
        lib.itts_seen_insert(_ptr(self.words), int(token_id))

    def contains(self, token_id: int) -> bool:
        if not 0 <= token_id < 129 * 64:
            return False
        return bool((int(self.words[token_id // 64]) >> (token_id % 64)) & 1)


# ----------------------------------------------------------------------------------
# Decoder
# ----------------------------------------------------------------------------------

class Gpt:
    """Gpt::from_weights over a weights description (see itts_hip.synth.ModelWeights)."""

    def __init__(self, weights):
        self._weights = weights  # keeps host arrays referenced by the C struct alive
        cw, keep = weights.to_itts()
        h = C.c_void_p()
        _check(lib.itts_gpt_create(C.byref(cw), C.byref(h)))
        del keep  # the library has copied every tensor to the device
        self._h = h
        self.cfg = weights.cfg

    @classmethod
    def load_from_path(cls, path: str) -> "Gpt":
        """Gpt::load_from_path: a gpt_int8 safetensors checkpoint."""
        self = cls.__new__(cls)
        self._weights = None
        h = C.c_void_p()
        _check(lib.itts_gpt_load_safetensors(os.fsencode(path), C.byref(h)))
        self._h = h
        c = lib.itts_gpt_config(h)
        self.cfg = {n: getattr(c, n) for n, _ in itts_config._fields_}
        return self

    def close(self):
        if getattr(self, "_h", None):
            lib.itts_gpt_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def num_layers(self) -> int:
        return lib.itts_gpt_num_layers(self._h)

    @property
    def stream(self) -> int:
        return lib.itts_gpt_stream(self._h)

    def set_decode_path(self, path: int):
        """ITTS_DECODE_AUTO / _MULTI / _PERSISTENT for caches created afterwards."""
        _check(lib.itts_gpt_set_decode_path(self._h, int(path)))

    def kv_cache(self, max_seq: int = 2048, dtype: int = ITTS_BF16) -> "KvCache":
        return KvCache(self, max_seq, dtype)

    def prefill(self, text_tokens, conds, lang_id, cache, logits=True):
        return self.prefill_after(text_tokens, conds, lang_id, [], cache, logits)

    def prefill_after(self, text_tokens, conds, lang_id, prior_codes, cache, logits=True):
        t = np.ascontiguousarray(text_tokens, dtype=np.int32)
        c = np.ascontiguousarray(conds, dtype=np.float32).reshape(-1, self.cfg["d_model"]) \
            if conds is not None else np.zeros((0, self.cfg["d_model"]), np.float32)
        p = np.ascontiguousarray(prior_codes, dtype=np.int32)
        out = np.empty(self.cfg["mel_vocab"], np.float32) if logits else None
        _check(lib.itts_gpt_prefill_after(self._h, cache._h, _ptr(t), len(t), _ptr(c), c.shape[0],
                                          int(lang_id), _ptr(p), len(p), _ptr(out)))
        return out

    def step(self, cache, mel_token_id, pos_idx, logits=True):
        out = np.empty(self.cfg["mel_vocab"], np.float32) if logits else None
        _check(lib.itts_gpt_step(self._h, cache._h, int(mel_token_id), int(pos_idx), _ptr(out)))
        return out

    # teacher-forced replay (gpt.rs:756-915)
    def _tc(self, text_tokens, conds):
        t = np.ascontiguousarray(text_tokens, dtype=np.int32)
        c = np.ascontiguousarray(conds, dtype=np.float32).reshape(-1, self.cfg["d_model"]) \
            if conds is not None else np.zeros((0, self.cfg["d_model"]), np.float32)
        return t, c

    def teacher_forced(self, text_tokens, conds, lang_id, codes, cache, attention=True):
        """Gpt::teacher_forced (attention=True) / code_log_probs (False): returns
        (log_probs [n], attention [n][n_text + 2] or None)."""
        t, c = self._tc(text_tokens, conds)
        cd = np.ascontiguousarray(codes, dtype=np.int32)
        lp = np.empty(len(cd), np.float32)
        att = np.empty((len(cd), len(t) + 2), np.float32) if attention else None
        _check(lib.itts_gpt_teacher_forced(self._h, cache._h, _ptr(t), len(t), _ptr(c), c.shape[0], int(lang_id),
                                           _ptr(cd), len(cd), _ptr(lp), _ptr(att)))
        return lp, att

    def code_log_probs(self, text_tokens, conds, lang_id, codes, cache):
        return self.teacher_forced(text_tokens, conds, lang_id, codes, cache, attention=False)[0]

    def alignment_attention(self, text_tokens, conds, lang_id, prior_codes, codes, cache):
        t, c = self._tc(text_tokens, conds)
        pr = np.ascontiguousarray(prior_codes if prior_codes is not None else [], dtype=np.int32)
        cd = np.ascontiguousarray(codes, dtype=np.int32)
        att = np.empty((len(cd), len(t) + 2), np.float32)
        _check(lib.itts_gpt_alignment_attention(self._h, cache._h, _ptr(t), len(t), _ptr(c), c.shape[0],
                                                int(lang_id), _ptr(pr), len(pr), _ptr(cd), len(cd), _ptr(att)))
        return att

    def set_alignment_heads(self, pairs):
        a = np.ascontiguousarray(np.asarray(pairs, dtype=np.int32).reshape(-1))
        _check(lib.itts_gpt_set_alignment_heads(self._h, _ptr(a), len(a) // 2))

    def forward_logits(self, prompts, copy_out=True):
        """All-row logits of a batch of CodePrompts in one forward: [sum T_b][mel_vocab]
        (copy_out=False leaves them on the device and returns None)."""
        keep, arr = [], (itts_code_prompt * len(prompts))()
        rows = 0
        for i, p in enumerate(prompts):
            t, c = self._tc(p.text_tokens, p.conds)
            pr = np.ascontiguousarray(p.prior_codes if p.prior_codes is not None else [], dtype=np.int32)
            keep += [t, c, pr]
            arr[i] = itts_code_prompt(_ptr(t), len(t), _ptr(c), c.shape[0], int(p.lang_id), _ptr(pr), len(pr), 0)
            rows += c.shape[0] + len(t) + 3 + len(pr)
        out = np.empty((rows, self.cfg["mel_vocab"]), np.float32) if copy_out else None
        _check(lib.itts_gpt_forward_logits(self._h, C.cast(arr, C.c_void_p), len(prompts), _ptr(out)))
        return out

    # kernel-level helpers
    def dequantize(self, codes, scales, biases, N, K, bits, param_dtype):
        q = itts_qlinear(_ptr(codes), _ptr(scales), _ptr(biases), None)
        out = np.empty((N, K), np.float32)
        _check(lib.itts_dequantize(self._h, C.byref(q), N, K, bits, param_dtype, _ptr(out)))
        return out

    def qlinear_forward(self, codes, scales, biases, bias, x, N, K, bits, param_dtype):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
        q = itts_qlinear(_ptr(codes), _ptr(scales), _ptr(biases), _ptr(bias))
        out = np.empty((x.shape[0], N), np.float32)
        _check(lib.itts_qlinear_forward(self._h, C.byref(q), N, K, bits, param_dtype, _ptr(x),
                                        x.shape[0], _ptr(out)))
        return out


class KvCache:
    """KvCache::new(max_seq) on the device (bf16 rows by default, or fp32)."""

    def __init__(self, gpt: Gpt, max_seq: int = 2048, dtype: int = ITTS_BF16):
        self.gpt = gpt
        h = C.c_void_p()
        _check(lib.itts_kv_create(gpt._h, int(max_seq), int(dtype), C.byref(h)))
        self._h = h

    def close(self):
        if getattr(self, "_h", None):
            lib.itts_kv_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        lib.itts_kv_reset(self._h)

    def valid_len(self) -> int:
        return lib.itts_kv_valid_len(self._h)

    def max_seq(self) -> int:
        return lib.itts_kv_max_seq(self._h)

    def decode_path(self) -> int:
        return lib.itts_kv_decode_path(self._h)

    def last_timing(self) -> dict:
        t = itts_timing()
        _check(lib.itts_kv_last_timing(self._h, C.byref(t)))
        return {f: getattr(t, f) for f, _ in itts_timing._fields_}

    def decode_timing(self, mel_token_id: int, pos_idx: int, n_steps: int) -> float:
        """Milliseconds per decode step over n_steps back-to-back steps (the cache grows)."""
        ms = C.c_float()
        _check(lib.itts_decode_timing(self.gpt._h, self._h, int(mel_token_id), int(pos_idx), int(n_steps),
                                      C.byref(ms)))
        return ms.value

    def read(self, layer: int, which_v: bool) -> np.ndarray:
        cfg = self.gpt.cfg
        out = np.empty((cfg["n_head"], self.valid_len(), 64), np.float32)
        _check(lib.itts_kv_read(self._h, layer, int(which_v), _ptr(out)))
        return out


def sample_next_token(gpt: Gpt, logits: np.ndarray, seen: SeenTokenBitSet,
                      params: SamplingParams, rng: SamplerRng) -> int:
    """sample_next_token on the device sampler; `logits` is penalised in place."""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
    tok = C.c_int32()
    p = params.to_c()
    _check(lib.itts_sample_next_token(gpt._h, _ptr(logits), len(logits), _ptr(seen.words),
                                      C.byref(p), C.byref(rng.state), C.byref(tok)))
    return tok.value


def sample_next_token_noalloc(gpt: Gpt, logits: np.ndarray, seen: SeenTokenBitSet,
                              params: SamplingParams, rng: SamplerRng) -> int:
    """sample_next_token through the entry point that allocates no device memory (the
    library's static staging array); `logits` is penalised in place."""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
    tok = C.c_int32()
    p = params.to_c()
    _check(lib.itts_sample_next_token_noalloc(gpt._h, _ptr(logits), len(logits), _ptr(seen.words),
                                              C.byref(p), C.byref(rng.state), C.byref(tok)))
    return tok.value


@dataclass
class CodePrompt:
    text_tokens: np.ndarray
    conds: np.ndarray
    lang_id: int
    prior_codes: np.ndarray | None = None
    min_codes: int = 0


def generate_codes_after(gpt: Gpt, prompt: CodePrompt, cache: KvCache, params: SamplingParams,
                         rng: SamplerRng) -> np.ndarray:
    t = np.ascontiguousarray(prompt.text_tokens, dtype=np.int32)
    c = np.ascontiguousarray(prompt.conds, dtype=np.float32).reshape(-1, gpt.cfg["d_model"])
    pr = np.ascontiguousarray(prompt.prior_codes if prompt.prior_codes is not None else [],
                              dtype=np.int32)
    cp = itts_code_prompt(_ptr(t), len(t), _ptr(c), c.shape[0], int(prompt.lang_id), _ptr(pr),
                          len(pr), int(prompt.min_codes))
    sp = params.to_c()
    cap = max(1, int(params.max_mel_tokens))
    out = np.empty(cap, np.int32)
    n = C.c_int32()
    _check(lib.itts_generate_codes_after(gpt._h, cache._h, C.byref(cp), C.byref(sp),
                                         C.byref(rng.state), _ptr(out), cap, C.byref(n)))
    return out[: n.value].copy()


def step_batch(gpt: Gpt, caches, tokens, positions, logits=True):
    """One batched decode step: Gpt::step for every (cache, token, position); returns
    logits [batch][mel_vocab]."""
    arr = (C.c_void_p * len(caches))(*[c._h for c in caches])
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    p = np.ascontiguousarray(positions, dtype=np.int32)
    out = np.empty((len(caches), gpt.cfg["mel_vocab"]), np.float32) if logits else None
    _check(lib.itts_gpt_step_batch(gpt._h, C.cast(arr, C.c_void_p), len(caches), _ptr(t), _ptr(p), _ptr(out)))
    return out


def generate_codes_batch(gpt: Gpt, prompts, caches, params, rngs):
    """generate_codes_after for several sequences stepped together; params and rngs are
    per sequence (the rngs advance as SamplerRng does).  Returns a list of code arrays."""
    B = len(prompts)
    keep, arr = [], (itts_code_prompt * B)()
    for i, pr in enumerate(prompts):
        t = np.ascontiguousarray(pr.text_tokens, dtype=np.int32)
        c = np.ascontiguousarray(pr.conds, dtype=np.float32).reshape(-1, gpt.cfg["d_model"])
        pp = np.ascontiguousarray(pr.prior_codes if pr.prior_codes is not None else [], dtype=np.int32)
        keep += [t, c, pp]
        arr[i] = itts_code_prompt(_ptr(t), len(t), _ptr(c), c.shape[0], int(pr.lang_id), _ptr(pp), len(pp),
                                  int(pr.min_codes))
    sp = (itts_sampling * B)(*[p.to_c() for p in params])
    cs = (C.c_void_p * B)(*[c._h for c in caches])
    states = np.array([r.state.value for r in rngs], dtype=np.uint64)
    cap = max(1, max(int(p.max_mel_tokens) for p in params))
    out = np.empty((B, cap), np.int32)
    n = np.empty(B, np.int32)
    _check(lib.itts_generate_codes_batch(gpt._h, C.cast(cs, C.c_void_p), C.cast(arr, C.c_void_p),
                                         C.cast(sp, C.c_void_p), B, _ptr(states), _ptr(out), cap, _ptr(n)))
    for r, st in zip(rngs, states):
        r.state.value = int(st)
    return [out[i, : n[i]].copy() for i in range(B)]


def generate_codes(gpt: Gpt, text_tokens, conds, lang_id, cache, params, rng) -> np.ndarray:
    return generate_codes_after(gpt, CodePrompt(text_tokens, conds, lang_id), cache, params, rng)


def quantize(w: np.ndarray, bits: int = 8, param_dtype: int = ITTS_F16):
    """The workload's MLX-affine group-64 quantiser (host, multi-threaded)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    codes = np.empty((N, K * bits // 8), np.uint8)
    pdt = np.uint16 if param_dtype == ITTS_F16 else np.float32
    scales = np.empty((N, K // 64), pdt)
    biases = np.empty((N, K // 64), pdt)
    _check(lib.itts_quantize(_ptr(w), N, K, bits, param_dtype, _ptr(codes), _ptr(scales),
                             _ptr(biases)))
    return codes, scales, biases
