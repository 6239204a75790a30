"""Synthetic decoder workloads: seeded random-init weights of the reference shape
(gpt.rs:31-54, Gpt::from_weights 477-515) quantized with the workload's MLX-affine
group-64 quantiser, plus seeded prompts.

Spec init ("spec"): every linear weight N(0, 0.02) fp32, linear biases 0, LayerNorm
gamma 1 / beta 0, embedding tables N(0, 0.02) fp32.  The "rich" init adds non-trivial
LayerNorm parameters and linear biases so that tests exercise every tensor.

Each tensor draws from its own numpy PCG64 stream keyed by (seed, tensor index), so
the weights are identical on every host with the same numpy.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import ITTS_F16, ITTS_F32, itts_config, itts_layer_weights, itts_qlinear, itts_weights, quantize

FULL_CONFIG = dict(n_layer=24, d_model=1280, n_head=20, d_ffn=5120, mel_vocab=8194,
                   text_vocab=60510, lang_vocab=107, mel_pos_len=1818, text_pos_len=602,
                   quant_bits=8, param_dtype=ITTS_F16)

TINY_CONFIG = dict(n_layer=2, d_model=128, n_head=2, d_ffn=512, mel_vocab=258, text_vocab=300,
                   lang_vocab=8, mel_pos_len=256, text_pos_len=64, quant_bits=8,
                   param_dtype=ITTS_F16)

SMALL_CONFIG = dict(n_layer=4, d_model=256, n_head=4, d_ffn=1024, mel_vocab=1026,
                    text_vocab=2000, lang_vocab=16, mel_pos_len=600, text_pos_len=128,
                    quant_bits=8, param_dtype=ITTS_F16)


@dataclass
class QLinear:
    codes: np.ndarray   # uint8 [N][K*bits/8]
    scales: np.ndarray  # uint16 (fp16 bits) or float32 [N][K/64]
    biases: np.ndarray
    bias: np.ndarray    # float32 [N]
    N: int
    K: int

    def to_c(self) -> itts_qlinear:
        return itts_qlinear(self.codes.ctypes.data, self.scales.ctypes.data,
                            self.biases.ctypes.data, self.bias.ctypes.data)


@dataclass
class Layer:
    ln1_w: np.ndarray
    ln1_b: np.ndarray
    c_attn: QLinear
    c_proj: QLinear
    ln2_w: np.ndarray
    ln2_b: np.ndarray
    c_fc: QLinear
    mlp_c_proj: QLinear


@dataclass
class ModelWeights:
    cfg: dict
    text_emb: np.ndarray
    lang_emb: np.ndarray
    mel_emb: np.ndarray
    mel_pos: np.ndarray
    text_pos: np.ndarray
    layers: list
    ln_f_w: np.ndarray
    ln_f_b: np.ndarray
    fn_w: np.ndarray
    fn_b: np.ndarray
    head: QLinear

    def weight_bytes_per_step(self) -> int:
        """Bytes of quantized weights + group params + biases + LN read by one decode step."""
        total = 0
        qls = [q for L in self.layers for q in (L.c_attn, L.c_proj, L.c_fc, L.mlp_c_proj)] + [self.head]
        for q in qls:
            total += q.codes.nbytes + q.scales.nbytes + q.biases.nbytes + q.bias.nbytes
        d = self.cfg["d_model"]
        total += (len(self.layers) * 4 + 4) * d * 4  # LayerNorm gamma/beta
        total += 2 * d * 4                           # the two embedding rows
        return total

    def to_itts(self):
        """(itts_weights, keep-alive): the struct points into this object's arrays and into
        the returned layer array, which the caller must keep referenced."""
        c = itts_config(**{k: int(self.cfg[k]) for k in (
            "n_layer", "d_model", "n_head", "d_ffn", "mel_vocab", "text_vocab", "lang_vocab",
            "mel_pos_len", "text_pos_len", "quant_bits", "param_dtype")})
        arr = (itts_layer_weights * len(self.layers))()
        for i, L in enumerate(self.layers):
            arr[i] = itts_layer_weights(L.ln1_w.ctypes.data, L.ln1_b.ctypes.data, L.c_attn.to_c(),
                                        L.c_proj.to_c(), L.ln2_w.ctypes.data, L.ln2_b.ctypes.data,
                                        L.c_fc.to_c(), L.mlp_c_proj.to_c())
        w = itts_weights(c, self.text_emb.ctypes.data, self.lang_emb.ctypes.data,
                         self.mel_emb.ctypes.data, self.mel_pos.ctypes.data,
                         self.text_pos.ctypes.data, C.cast(arr, C.POINTER(itts_layer_weights)),
                         self.ln_f_w.ctypes.data, self.ln_f_b.ctypes.data, self.fn_w.ctypes.data,
                         self.fn_b.ctypes.data, self.head.to_c())
        return w, arr


class _Streams:
    def __init__(self, seed: int):
        self.seed = seed
        self.idx = 0

    def next(self) -> np.random.Generator:
        g = np.random.default_rng([self.seed, self.idx])
        self.idx += 1
        return g


def _normal(g: np.random.Generator, shape, std: float) -> np.ndarray:
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def make_weights(cfg: dict | None = None, seed: int = 0, init: str = "spec",
                 quantizer=None) -> ModelWeights:
    """Seeded decoder weights.  `quantizer(w, bits, param_dtype) -> (codes, scales, biases)`
    defaults to the library's itts_quantize."""
    cfg = dict(FULL_CONFIG if cfg is None else cfg)
    qz = quantizer or quantize
    rich = init == "rich"
    S = _Streams(seed)
    d, F, V = cfg["d_model"], cfg["d_ffn"], cfg["mel_vocab"]
    bits, pd = cfg["quant_bits"], cfg["param_dtype"]

    def ql(N, K):
        w = _normal(S.next(), (N, K), 0.02)
        codes, scales, biases = qz(w, bits, pd)
        del w
        bias = _normal(S.next(), (N,), 0.02) if rich else np.zeros(N, np.float32)
        return QLinear(codes, scales, biases, bias, N, K)

    def ln():
        if rich:
            return (1.0 + _normal(S.next(), (d,), 0.1)).astype(np.float32), _normal(S.next(), (d,), 0.1)
        return np.ones(d, np.float32), np.zeros(d, np.float32)

    text_emb = _normal(S.next(), (cfg["text_vocab"], d), 0.02)
    lang_emb = _normal(S.next(), (cfg["lang_vocab"], d), 0.02)
    mel_emb = _normal(S.next(), (V, d), 0.02)
    mel_pos = _normal(S.next(), (cfg["mel_pos_len"], d), 0.02)
    text_pos = _normal(S.next(), (cfg["text_pos_len"], d), 0.02)
    layers = []
    for _ in range(cfg["n_layer"]):
        l1w, l1b = ln()
        attn = ql(3 * d, d)
        proj = ql(d, d)
        l2w, l2b = ln()
        fc = ql(F, d)
        mproj = ql(d, F)
        layers.append(Layer(l1w, l1b, attn, proj, l2w, l2b, fc, mproj))
    lfw, lfb = ln()
    fnw, fnb = ln()
    head = ql(V, d)
    return ModelWeights(cfg, text_emb, lang_emb, mel_emb, mel_pos, text_pos, layers, lfw, lfb,
                        fnw, fnb, head)


@dataclass
class Prompt:
    text_tokens: np.ndarray  # int32 [n]
    conds: np.ndarray        # float32 [n_cond][d]
    lang_id: int


def make_prompt(cfg: dict, n_cond: int, n_text: int, seed: int = 0, lang_id: int = 1) -> Prompt:
    """conds N(0,1); text ids uniform in [2, text_vocab) (the frontend never emits <= 1)."""
    g = np.random.default_rng([seed, 1_000_003])
    conds = g.standard_normal((n_cond, cfg["d_model"]), dtype=np.float32)
    text = g.integers(2, cfg["text_vocab"], size=n_text, dtype=np.int64).astype(np.int32)
    return Prompt(text, conds, min(lang_id, cfg["lang_vocab"] - 1))


def save_safetensors(W: ModelWeights, path: str, drop: tuple = (), override: dict | None = None) -> dict:
    """Writes W as a gpt_int8 checkpoint in the reference's tensor layout
    (crates/core/src/models/gpt.rs:477-515, 269-323, 229-247): F32 tables and LayerNorm
    vectors, each QuantizedLinear as `weight` U32 [N][K*bits/32] (the code bytes in
    little-endian words), `scales`/`biases` [N][K/64] (F32, or F16 for fp16 params) and
    `bias` F32 [N].  `drop` omits tensors and `override` replaces them (error tests).
    Returns the tensor dict written."""
    from safetensors.numpy import save_file

    t = {}

    def params(a):
        return a.view(np.float16) if a.dtype == np.uint16 else a.astype(np.float32)

    def ql(prefix, q):
        t[prefix + ".weight"] = np.ascontiguousarray(q.codes).view(np.uint32)
        t[prefix + ".scales"] = params(q.scales)
        t[prefix + ".biases"] = params(q.biases)
        t[prefix + ".bias"] = q.bias.astype(np.float32)

    t["text_embedding.weight"] = W.text_emb
    t["lang_embedding.weight"] = W.lang_emb
    t["mel_embedding.weight"] = W.mel_emb
    t["mel_pos_embedding.emb.weight"] = W.mel_pos
    t["text_pos_embedding.emb.weight"] = W.text_pos
    for i, L in enumerate(W.layers):
        p = f"gpt.h.{i}"
        t[p + ".ln_1.weight"], t[p + ".ln_1.bias"] = L.ln1_w, L.ln1_b
        t[p + ".ln_2.weight"], t[p + ".ln_2.bias"] = L.ln2_w, L.ln2_b
        ql(p + ".attn.c_attn", L.c_attn)
        ql(p + ".attn.c_proj", L.c_proj)
        ql(p + ".mlp.c_fc", L.c_fc)
        ql(p + ".mlp.c_proj", L.mlp_c_proj)
    t["gpt.ln_f.weight"], t["gpt.ln_f.bias"] = W.ln_f_w, W.ln_f_b
    t["final_norm.weight"], t["final_norm.bias"] = W.fn_w, W.fn_b
    ql("mel_head", W.head)
    for k in drop:
        t.pop(k)
    t.update(override or {})
    t = {k: np.ascontiguousarray(v) for k, v in t.items()}
    save_file(t, path, metadata={"format": "mlx"})
    return t


# ---- Stage-2 CFM DiT estimator ----------------------------------------------------------
def make_cfm_weights(cfg: dict, seed: int = 0) -> dict:
    """Seeded random-init CFM estimator tensors by checkpoint name (cfm.rs:460-531), float32.

    Linear and convolution weights are N(0, 1/fan_in) so activations stay O(1) through the
    13-layer stack; biases N(0, 0.02); RMSNorm weights 1 + N(0, 0.1); AdaLN projection biases
    1 + N(0, 0.1) for the scale half and N(0, 0.1) for the shift half, so that every
    modulation path is exercised.  Each tensor draws from its own stream keyed by
    (seed, tensor index)."""
    from .cfm import tensor_shapes
    out = {}
    for i, (name, shape) in enumerate(tensor_shapes(cfg).items()):
        g = np.random.Generator(np.random.PCG64([seed, 7919, i]))
        if name.endswith("norm.weight"):
            a = 1.0 + 0.1 * g.standard_normal(shape)
        elif name.endswith("project_layer.bias") or name.endswith("adaLN_modulation.layers.1.bias"):
            half = shape[0] // 2
            a = 0.1 * g.standard_normal(shape)
            if name.endswith("project_layer.bias"):
                a[:half] += 1.0
        elif name.endswith(".bias"):
            a = 0.02 * g.standard_normal(shape)
        else:
            fan_in = int(np.prod(shape[1:]))
            a = g.standard_normal(shape) / np.sqrt(fan_in)
        out[name] = np.ascontiguousarray(a, dtype=np.float32)
    return out


def make_cfm_inputs(cfg: dict, t_total: int, t_ref: int, seed: int = 0) -> dict:
    """Seeded solve_euler inputs of the reference's shapes (cfm.rs:621-632): cat_condition
    [1, T_total, dim], ref_mel [1, in_ch, T_ref], style [1, style], noise_z [1, in_ch, T_total]."""
    g = np.random.Generator(np.random.PCG64([seed, 104729]))
    f = lambda *s: g.standard_normal(s).astype(np.float32)
    return dict(cat_condition=f(1, t_total, cfg["dim"]), ref_mel=f(1, cfg["in_ch"], t_ref),
                style=f(1, cfg["style_dim"]), noise_z=f(1, cfg["in_ch"], t_total))
