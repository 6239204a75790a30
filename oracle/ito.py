"""ctypes binding of the CPU oracle (oracle/_build/libitts_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product package.  See itts_oracle.h for what each
function restates and the reference lines it follows.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("ITO_LIB") or os.path.join(HERE, "_build", "libitts_oracle.so")

ITO_OK, ITO_E_VALIDATION, ITO_E_CAPACITY, ITO_E_ALLOC = 0, 1, 4, 5
ITO_F32, ITO_F64 = 0, 1
ITO_KV_F32, ITO_KV_BF16 = 0, 1


class OracleError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"[{status}] {message}")
        self.status = status
        self.message = message


class ito_config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layer", "d_model", "n_head", "d_ffn", "mel_vocab", "text_vocab", "lang_vocab",
        "mel_pos_len", "text_pos_len", "bits", "param_f32")]


class ito_ql(C.Structure):
    _fields_ = [("codes", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p),
                ("bias", C.c_void_p), ("N", C.c_int32), ("K", C.c_int32)]


class ito_layer(C.Structure):
    _fields_ = [("ln1_w", C.c_void_p), ("ln1_b", C.c_void_p), ("c_attn", ito_ql),
                ("c_proj", ito_ql), ("ln2_w", C.c_void_p), ("ln2_b", C.c_void_p),
                ("c_fc", ito_ql), ("mlp_proj", ito_ql)]


class ito_model(C.Structure):
    _fields_ = [("cfg", ito_config), ("text_emb", C.c_void_p), ("lang_emb", C.c_void_p),
                ("mel_emb", C.c_void_p), ("mel_pos", C.c_void_p), ("text_pos", C.c_void_p),
                ("layers", C.POINTER(ito_layer)), ("ln_f_w", C.c_void_p), ("ln_f_b", C.c_void_p),
                ("fn_w", C.c_void_p), ("fn_b", C.c_void_p), ("head", ito_ql)]


class ito_probe(C.Structure):
    _fields_ = [("layer", C.c_int32), ("head", C.c_int32), ("q0", C.c_int32), ("k0", C.c_int32),
                ("k1", C.c_int32), ("out", C.c_void_p)]


class ito_sampling(C.Structure):
    _fields_ = [("greedy", C.c_int32), ("temperature", C.c_float), ("top_p", C.c_float),
                ("top_k", C.c_uint32), ("repetition_penalty", C.c_float),
                ("max_mel_tokens", C.c_uint32)]


P = C.c_void_p
_SIGS = {
    "ito_half_to_float": (C.c_float, [C.c_uint16]),
    "ito_float_to_half": (C.c_uint16, [C.c_float]),
    "ito_float_to_bf16": (C.c_uint16, [C.c_float]),
    "ito_bf16_to_float": (C.c_float, [C.c_uint16]),
    "ito_expf": (C.c_float, [C.c_float]),
    "ito_rng_init": (C.c_uint64, [C.c_uint64]),
    "ito_rng_next_u64": (C.c_uint64, [C.POINTER(C.c_uint64)]),
    "ito_rng_next_f32": (C.c_float, [C.POINTER(C.c_uint64)]),
    "ito_quantize": (C.c_int, [P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, P, P, P]),
    "ito_dequant": (C.c_int, [C.POINTER(ito_ql), C.c_int32, C.c_int32, P]),
    "ito_ql_forward": (C.c_int, [C.POINTER(ito_ql), C.c_int32, C.c_int32, C.c_int32, P, C.c_int32, P]),
    "ito_layernorm": (None, [P, P, P, C.c_int32, C.c_float, P]),
    "ito_gelu": (C.c_float, [C.c_float]),
    "ito_kv_create": (C.c_int, [C.POINTER(ito_config), C.c_int32, C.c_int32, C.c_int32,
                                C.POINTER(C.c_void_p)]),
    "ito_kv_destroy": (None, [P]),
    "ito_kv_reset": (None, [P]),
    "ito_kv_valid_len": (C.c_int32, [P]),
    "ito_kv_read": (C.c_int, [P, C.c_int32, C.c_int32, P]),
    "ito_prefill_after": (C.c_int, [C.POINTER(ito_model), P, C.c_int32, P, C.c_int32, P,
                                    C.c_int32, C.c_int32, P, C.c_int32, P]),
    "ito_step": (C.c_int, [C.POINTER(ito_model), P, C.c_int32, C.c_int32, C.c_int32, P]),
    "ito_forward_rows": (C.c_int, [C.POINTER(ito_model), P, C.c_int32, P, C.c_int32, C.c_int32, P]),
    "ito_replay": (C.c_int, [C.POINTER(ito_model), P, C.c_int32, P, C.c_int32, C.c_int32, P, C.c_int32,
                             C.c_int32, P]),
    "ito_sequence_embedding": (C.c_int, [C.POINTER(ito_model), P, C.c_int32, P, C.c_int32,
                                         C.c_int32, P, C.c_int32, P]),
    "ito_sampling_validate": (C.c_int, [C.POINTER(ito_sampling)]),
    "ito_seen_init": (None, [P, C.c_int32]),
    "ito_seen_insert": (None, [P, C.c_int32]),
    "ito_apply_repetition_penalty": (None, [P, P, C.c_int32, C.c_float]),
    "ito_argmax_finite": (C.c_int32, [P, C.c_int32]),
    "ito_sample_next_token": (C.c_int, [P, C.c_int32, P, C.POINTER(ito_sampling),
                                        C.POINTER(C.c_uint64), C.POINTER(C.c_int32)]),
    "ito_generate_codes_after": (C.c_int, [C.POINTER(ito_model), P, C.c_int32, P, C.c_int32, P,
                                           C.c_int32, C.c_int32, P, C.c_int32, C.c_int32,
                                           C.POINTER(ito_sampling), C.POINTER(C.c_uint64), P,
                                           C.c_int32, C.POINTER(C.c_int32), P]),
    "ito_last_error": (C.c_char_p, []),
    "ito_set_threads": (None, [C.c_int32]),
}


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


lib = _load()


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def check(st):
    if st != ITO_OK:
        raise OracleError(st, lib.ito_last_error().decode(errors="replace"))


def _ql(q) -> ito_ql:
    return ito_ql(q.codes.ctypes.data, q.scales.ctypes.data, q.biases.ctypes.data,
                  q.bias.ctypes.data, q.N, q.K)


class Model:
    """An ito_model view over itts_hip.synth.ModelWeights (same host arrays)."""

    def __init__(self, w):
        self.w = w
        c = w.cfg
        self.cfg = ito_config(c["n_layer"], c["d_model"], c["n_head"], c["d_ffn"], c["mel_vocab"],
                              c["text_vocab"], c["lang_vocab"], c["mel_pos_len"], c["text_pos_len"],
                              c["quant_bits"], 1 if c["param_dtype"] == 2 else 0)
        self.layers = (ito_layer * len(w.layers))()
        for i, L in enumerate(w.layers):
            self.layers[i] = ito_layer(L.ln1_w.ctypes.data, L.ln1_b.ctypes.data, _ql(L.c_attn),
                                       _ql(L.c_proj), L.ln2_w.ctypes.data, L.ln2_b.ctypes.data,
                                       _ql(L.c_fc), _ql(L.mlp_c_proj))
        self.m = ito_model(self.cfg, w.text_emb.ctypes.data, w.lang_emb.ctypes.data,
                           w.mel_emb.ctypes.data, w.mel_pos.ctypes.data, w.text_pos.ctypes.data,
                           C.cast(self.layers, C.POINTER(ito_layer)), w.ln_f_w.ctypes.data,
                           w.ln_f_b.ctypes.data, w.fn_w.ctypes.data, w.fn_b.ctypes.data,
                           _ql(w.head))

    @property
    def ref(self):
        return C.byref(self.m)

    def kv(self, max_seq=2048, kv_bf16=True, mode=ITO_F32) -> "KV":
        return KV(self, max_seq, kv_bf16, mode)

    def prefill_after(self, kv, text, conds, lang_id, prior=()):
        t = np.ascontiguousarray(text, np.int32)
        c = np.ascontiguousarray(conds, np.float32).reshape(-1, self.w.cfg["d_model"])
        pr = np.ascontiguousarray(prior, np.int32)
        out = np.empty(self.w.cfg["mel_vocab"], np.float32)
        check(lib.ito_prefill_after(self.ref, kv.h, kv.mode, _p(t), len(t), _p(c), c.shape[0],
                                    int(lang_id), _p(pr), len(pr), _p(out)))
        return out

    def step(self, kv, tok, pos):
        out = np.empty(self.w.cfg["mel_vocab"], np.float32)
        check(lib.ito_step(self.ref, kv.h, kv.mode, int(tok), int(pos), _p(out)))
        return out

    def sequence_embedding(self, text, conds, lang_id, prior=()):
        t = np.ascontiguousarray(text, np.int32)
        c = np.ascontiguousarray(conds, np.float32).reshape(-1, self.w.cfg["d_model"])
        pr = np.ascontiguousarray(prior, np.int32)
        T = c.shape[0] + len(t) + 3 + len(pr)
        out = np.empty((T, self.w.cfg["d_model"]), np.float32)
        check(lib.ito_sequence_embedding(self.ref, _p(t), len(t), _p(c), c.shape[0], int(lang_id),
                                         _p(pr), len(pr), _p(out)))
        return out

    def forward_rows(self, kv, emb, row0=0):
        emb = np.ascontiguousarray(emb, np.float32)
        T = emb.shape[0]
        out = np.empty((T - row0, self.w.cfg["mel_vocab"]), np.float32)
        check(lib.ito_forward_rows(self.ref, kv.h, kv.mode, _p(emb), T, row0, _p(out)))
        return out

    def replay(self, kv, emb, n_layers=None, probes=(), row0=None):
        """Stack over emb [T][d] through n_layers blocks; probes are (layer, head, q0, k0, k1)
        tuples whose attention slices [(T-q0)][k1-k0] are returned; with row0 set (whole
        stack) also the logits of rows row0.. .  Returns (logits or None, [probe arrays])."""
        emb = np.ascontiguousarray(emb, np.float32)
        T = emb.shape[0]
        n_layers = self.w.cfg["n_layer"] if n_layers is None else n_layers
        outs = [np.zeros((T - q0, k1 - k0), np.float32) for (_, _, q0, k0, k1) in probes]
        arr = (ito_probe * max(1, len(probes)))()
        for i, ((l, h, q0, k0, k1), o) in enumerate(zip(probes, outs)):
            arr[i] = ito_probe(l, h, q0, k0, k1, o.ctypes.data)
        logits = None if row0 is None else np.empty((T - row0, self.w.cfg["mel_vocab"]), np.float32)
        check(lib.ito_replay(self.ref, kv.h, kv.mode, _p(emb), T, n_layers, C.cast(arr, C.c_void_p),
                             len(probes), 0 if row0 is None else row0, _p(logits)))
        return logits, outs

    def generate_codes_after(self, kv, text, conds, lang_id, params, rng_state, prior=(),
                             min_codes=0):
        t = np.ascontiguousarray(text, np.int32)
        c = np.ascontiguousarray(conds, np.float32).reshape(-1, self.w.cfg["d_model"])
        pr = np.ascontiguousarray(prior, np.int32)
        sp = sampling(params)
        cap = max(1, int(params.max_mel_tokens))
        out = np.empty(cap, np.int32)
        first = np.empty(self.w.cfg["mel_vocab"], np.float32)
        n = C.c_int32()
        st = C.c_uint64(rng_state)
        check(lib.ito_generate_codes_after(self.ref, kv.h, kv.mode, _p(t), len(t), _p(c), c.shape[0],
                                           int(lang_id), _p(pr), len(pr), int(min_codes),
                                           C.byref(sp), C.byref(st), _p(out), cap, C.byref(n),
                                           _p(first)))
        return out[: n.value].copy(), st.value, first


class KV:
    def __init__(self, model, max_seq, kv_bf16, mode):
        self.model = model
        self.mode = mode
        h = C.c_void_p()
        check(lib.ito_kv_create(C.byref(model.cfg), int(max_seq), ITO_KV_BF16 if kv_bf16 else ITO_KV_F32,
                                mode, C.byref(h)))
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib.ito_kv_destroy(self.h)
            self.h = None

    def valid_len(self):
        return lib.ito_kv_valid_len(self.h)

    def reset(self):
        lib.ito_kv_reset(self.h)

    def read(self, layer, which_v):
        c = self.model.w.cfg
        out = np.empty((c["n_head"], self.valid_len(), 64), np.float32)
        check(lib.ito_kv_read(self.h, layer, int(which_v), _p(out)))
        return out


def sampling(params) -> ito_sampling:
    return ito_sampling(int(bool(params.greedy)), float(params.temperature), float(params.top_p),
                        int(params.top_k), float(params.repetition_penalty), int(params.max_mel_tokens))


def quantize(w, bits=8, param_dtype=1):
    """Oracle quantiser with the itts_hip.quantize calling convention (1 = fp16, 2 = fp32)."""
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    codes = np.empty((N, K * bits // 8), np.uint8)
    f32 = param_dtype == 2
    pdt = np.float32 if f32 else np.uint16
    scales = np.empty((N, K // 64), pdt)
    biases = np.empty((N, K // 64), pdt)
    check(lib.ito_quantize(_p(w), N, K, bits, int(f32), _p(codes), _p(scales), _p(biases)))
    return codes, scales, biases


def dequant(q, bits, param_dtype):
    out = np.empty((q.N, q.K), np.float32)
    ql = _ql(q)
    check(lib.ito_dequant(C.byref(ql), bits, 1 if param_dtype == 2 else 0, _p(out)))
    return out


def ql_forward(q, bits, param_dtype, x, mode=ITO_F32):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, q.K)
    out = np.empty((x.shape[0], q.N), np.float32)
    ql = _ql(q)
    check(lib.ito_ql_forward(C.byref(ql), bits, 1 if param_dtype == 2 else 0, mode, _p(x), x.shape[0],
                             _p(out)))
    return out


def sample_next_token(logits, seen_words, params, rng_state):
    """Returns (token, new rng state); logits are penalised in place."""
    assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
    sp = sampling(params)
    st = C.c_uint64(rng_state)
    tok = C.c_int32()
    check(lib.ito_sample_next_token(_p(logits), len(logits), _p(seen_words), C.byref(sp), C.byref(st),
                                    C.byref(tok)))
    return tok.value, st.value


def seen_init(start_mel=8192):
    w = np.zeros(129, np.uint64)
    lib.ito_seen_init(_p(w), start_mel)
    return w


# ---- Stage-2 CFM DiT estimator (cfm.rs) ---------------------------------------------------
class ito_cfm_config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("dim", "n_layers", "n_heads", "inter", "in_ch", "style_dim",
                                         "wn_layers", "wn_kernel")]


class ito_cfm_adaln(C.Structure):
    _fields_ = [("proj_w", C.c_void_p), ("proj_b", C.c_void_p), ("norm_w", C.c_void_p)]


class ito_cfm_temb(C.Structure):
    _fields_ = [("w0", C.c_void_p), ("b0", C.c_void_p), ("w2", C.c_void_p), ("b2", C.c_void_p)]


class ito_cfm_block(C.Structure):
    _fields_ = [("attn_norm", ito_cfm_adaln), ("ffn_norm", ito_cfm_adaln), ("wqkv", C.c_void_p),
                ("wo", C.c_void_p), ("w1", C.c_void_p), ("w3", C.c_void_p), ("w2", C.c_void_p),
                ("skip_w", C.c_void_p), ("skip_b", C.c_void_p)]


class ito_cfm_wn_layer(C.Structure):
    _fields_ = [("in_w", C.c_void_p), ("in_b", C.c_void_p), ("rs_w", C.c_void_p), ("rs_b", C.c_void_p)]


class ito_cfm(C.Structure):
    _fields_ = [("cfg", ito_cfm_config), ("cond_proj_w", C.c_void_p), ("cond_proj_b", C.c_void_p),
                ("merge_w", C.c_void_p), ("merge_b", C.c_void_p), ("t1", ito_cfm_temb), ("t2", ito_cfm_temb),
                ("blocks", C.POINTER(ito_cfm_block)), ("tnorm", ito_cfm_adaln),
                ("skip_w", C.c_void_p), ("skip_b", C.c_void_p), ("conv1_w", C.c_void_p), ("conv1_b", C.c_void_p),
                ("res_w", C.c_void_p), ("res_b", C.c_void_p), ("wn_cond_w", C.c_void_p), ("wn_cond_b", C.c_void_p),
                ("wn", C.POINTER(ito_cfm_wn_layer)), ("fada_w", C.c_void_p), ("fada_b", C.c_void_p),
                ("flin_w", C.c_void_p), ("flin_b", C.c_void_p), ("conv2_w", C.c_void_p), ("conv2_b", C.c_void_p)]


_CFM_SIGS = {
    "ito_cfm_rope": (None, [C.c_void_p, C.c_int32, C.c_int32]),
    "ito_cfm_timestep": (None, [C.POINTER(ito_cfm_temb), C.c_int32, C.c_float, C.c_void_p]),
    "ito_cfm_forward": (C.c_int, [C.POINTER(ito_cfm), C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_int32,
                                  C.c_void_p]),
    "ito_cfm_solve_euler": (C.c_int, [C.POINTER(ito_cfm), C.c_void_p, C.c_int32, C.c_void_p, C.c_int32,
                                      C.c_void_p, C.c_void_p, C.c_int32, C.c_float, C.c_void_p]),
}
for _n, (_r, _a) in _CFM_SIGS.items():
    getattr(lib, _n).restype = _r
    getattr(lib, _n).argtypes = _a


class CfmModel:
    """The oracle's CFM estimator over a dict of float32 tensors keyed by checkpoint name."""

    def __init__(self, weights: dict, cfg: dict):
        self.cfg = dict(cfg)
        self._keep = {k: np.ascontiguousarray(v, np.float32) for k, v in weights.items()}
        w = lambda n: self._keep[n].ctypes.data
        adaln = lambda p: ito_cfm_adaln(w(f"{p}.project_layer.weight"), w(f"{p}.project_layer.bias"),
                                        w(f"{p}.norm.weight"))
        temb = lambda p: ito_cfm_temb(w(f"{p}.mlp.layers.0.weight"), w(f"{p}.mlp.layers.0.bias"),
                                      w(f"{p}.mlp.layers.2.weight"), w(f"{p}.mlp.layers.2.bias"))
        L = cfg["n_layers"]
        self._blocks = (ito_cfm_block * L)()
        for i in range(L):
            p = f"transformer.layers.{i}"
            self._blocks[i] = ito_cfm_block(adaln(f"{p}.attention_norm"), adaln(f"{p}.ffn_norm"),
                                            w(f"{p}.attention.wqkv.weight"), w(f"{p}.attention.wo.weight"),
                                            w(f"{p}.feed_forward.w1.weight"), w(f"{p}.feed_forward.w3.weight"),
                                            w(f"{p}.feed_forward.w2.weight"), w(f"{p}.skip_in_linear.weight"),
                                            w(f"{p}.skip_in_linear.bias"))
        NL = cfg["wn_layers"]
        self._wn = (ito_cfm_wn_layer * NL)()
        for i in range(NL):
            self._wn[i] = ito_cfm_wn_layer(w(f"wavenet.in_layers.{i}.weight"), w(f"wavenet.in_layers.{i}.bias"),
                                           w(f"wavenet.res_skip_layers.{i}.weight"),
                                           w(f"wavenet.res_skip_layers.{i}.bias"))
        self.m = ito_cfm(ito_cfm_config(**cfg), w("cond_projection.weight"), w("cond_projection.bias"),
                         w("cond_x_merge_linear.weight"), w("cond_x_merge_linear.bias"), temb("t_embedder"),
                         temb("t_embedder2"), self._blocks, adaln("transformer.norm"), w("skip_linear.weight"),
                         w("skip_linear.bias"), w("conv1.weight"), w("conv1.bias"), w("res_projection.weight"),
                         w("res_projection.bias"), w("wavenet.cond_layer.weight"), w("wavenet.cond_layer.bias"),
                         self._wn, w("final_layer.adaLN_modulation.layers.1.weight"),
                         w("final_layer.adaLN_modulation.layers.1.bias"), w("final_layer.linear.weight"),
                         w("final_layer.linear.bias"), w("conv2.weight"), w("conv2.bias"))

    def timestep(self, which: int, t: float) -> np.ndarray:
        out = np.empty(self.cfg["dim"], np.float32)
        lib.ito_cfm_timestep(C.byref(self.m.t1 if which == 1 else self.m.t2), self.cfg["dim"], t, _p(out))
        return out

    def forward_merged(self, x_t, x_merged, t) -> np.ndarray:
        x_t = np.ascontiguousarray(x_t, np.float32)
        x_merged = np.ascontiguousarray(x_merged, np.float32)
        t = np.ascontiguousarray(t, np.float32)
        B, T = x_t.shape[:2]
        out = np.empty((B, self.cfg["in_ch"], T), np.float32)
        check(lib.ito_cfm_forward(C.byref(self.m), _p(x_t), _p(x_merged), _p(t), B, T, _p(out)))
        return out

    def solve_euler(self, cat_condition, ref_mel, style, noise_z, n_timesteps=25, cfg_rate=0.7) -> np.ndarray:
        cc = np.ascontiguousarray(cat_condition, np.float32)
        rm = np.ascontiguousarray(ref_mel, np.float32)
        st = np.ascontiguousarray(style, np.float32)
        nz = np.ascontiguousarray(noise_z, np.float32)
        T, Tr = cc.shape[1], rm.shape[2]
        out = np.empty((1, self.cfg["in_ch"], max(T - Tr, 0)), np.float32)
        check(lib.ito_cfm_solve_euler(C.byref(self.m), _p(cc), T, _p(rm), Tr, _p(st), _p(nz), n_timesteps,
                                      cfg_rate, _p(out)))
        return out


def cfm_rope(x: np.ndarray, n_heads: int) -> np.ndarray:
    """The oracle's rope (traditional pairs) on a copy of x [T, n_heads*64]."""
    y = np.ascontiguousarray(x, np.float32).copy()
    lib.ito_cfm_rope(_p(y), y.shape[0], n_heads)
    return y
