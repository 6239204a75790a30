"""Stage-2 CFM DiT estimator and its Euler / classifier-free-guidance solver on the HIP
path: the mirror of the reference's ``CfmDit`` (crates/core/src/models/cfm.rs) over the
C ABI of libitts_hip (``itts_cfm_*`` in include/itts_hip.h).

``CfmDit(weights, cfg)`` takes the estimator's tensors by their checkpoint names
(``CfmDit::from_weights``, cfm.rs:460-531) as float32 arrays of the shapes
``tensor_shapes(cfg)`` lists; ``forward_merged`` and ``solve_euler`` follow
cfm.rs:545-617 and 619-760, including the reference's validation errors.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import ValidationError, _check, itts_cfm_config, lib

# cfm.rs:36-61
FULL_CONFIG = dict(dim=512, n_layers=13, n_heads=8, inter=1536, in_ch=80, style_dim=192, wn_layers=8, wn_kernel=5)
# a reduced configuration of the same architecture for tests (head dimension stays 64)
SMALL_CONFIG = dict(dim=128, n_layers=5, n_heads=2, inter=192, in_ch=16, style_dim=24, wn_layers=3, wn_kernel=5)
FREQ_DIM = 256  # TimestepEmbedder input: 128 cosines and 128 sines (cfm.rs:114-121)


def merged_dim(cfg: dict) -> int:
    """Width of the merged input (cfm.rs:58): x_t, prompt mel, projected condition, style."""
    return 2 * cfg["in_ch"] + cfg["dim"] + cfg["style_dim"]


def tensor_shapes(cfg: dict) -> dict:
    """Checkpoint tensor names and shapes CfmDit::from_weights requires (cfm.rs:114-135,
    157-171, 198-251, 332-370, 460-531)."""
    d, F, C_, NL, K = cfg["dim"], cfg["inter"], cfg["in_ch"], cfg["wn_layers"], cfg["wn_kernel"]
    s = {
        "cond_projection.weight": (d, d), "cond_projection.bias": (d,),
        "cond_x_merge_linear.weight": (d, merged_dim(cfg)), "cond_x_merge_linear.bias": (d,),
    }
    for p in ("t_embedder", "t_embedder2"):
        s.update({f"{p}.mlp.layers.0.weight": (d, FREQ_DIM), f"{p}.mlp.layers.0.bias": (d,),
                  f"{p}.mlp.layers.2.weight": (d, d), f"{p}.mlp.layers.2.bias": (d,)})

    def adaln(p):
        s.update({f"{p}.project_layer.weight": (2 * d, d), f"{p}.project_layer.bias": (2 * d,),
                  f"{p}.norm.weight": (d,)})

    for i in range(cfg["n_layers"]):
        p = f"transformer.layers.{i}"
        adaln(f"{p}.attention_norm")
        adaln(f"{p}.ffn_norm")
        s.update({f"{p}.attention.wqkv.weight": (3 * d, d), f"{p}.attention.wo.weight": (d, d),
                  f"{p}.feed_forward.w1.weight": (F, d), f"{p}.feed_forward.w3.weight": (F, d),
                  f"{p}.feed_forward.w2.weight": (d, F),
                  f"{p}.skip_in_linear.weight": (d, 2 * d), f"{p}.skip_in_linear.bias": (d,)})
    adaln("transformer.norm")
    s.update({"skip_linear.weight": (d, d + C_), "skip_linear.bias": (d,),
              "conv1.weight": (d, d), "conv1.bias": (d,),
              "res_projection.weight": (d, d), "res_projection.bias": (d,),
              "wavenet.cond_layer.weight": (2 * d * NL, 1, d), "wavenet.cond_layer.bias": (2 * d * NL,)})
    for i in range(NL):
        rs = d if i + 1 == NL else 2 * d
        s.update({f"wavenet.in_layers.{i}.weight": (2 * d, K, d), f"wavenet.in_layers.{i}.bias": (2 * d,),
                  f"wavenet.res_skip_layers.{i}.weight": (rs, 1, d), f"wavenet.res_skip_layers.{i}.bias": (rs,)})
    s.update({"final_layer.adaLN_modulation.layers.1.weight": (2 * d, d),
              "final_layer.adaLN_modulation.layers.1.bias": (2 * d,),
              "final_layer.linear.weight": (d, d), "final_layer.linear.bias": (d,),
              "conv2.weight": (C_, 1, d), "conv2.bias": (C_,)})
    return s


def _f32(a, name):
    return np.ascontiguousarray(a, dtype=np.float32)


class CfmDit:
    """Device copy of the estimator; one HIP stream, one rocBLAS handle."""

    def __init__(self, weights: dict, cfg: dict | None = None):
        self.cfg = dict(cfg or FULL_CONFIG)
        c = itts_cfm_config(**self.cfg)
        names = list(weights)
        arrs = [_f32(weights[n], n) for n in names]
        n = len(names)
        cn = (C.c_char_p * n)(*[x.encode() for x in names])
        cp = (C.c_void_p * n)(*[a.ctypes.data for a in arrs])
        ce = (C.c_int64 * n)(*[a.size for a in arrs])
        h = C.c_void_p()
        _check(lib.itts_cfm_create(C.byref(c), C.cast(cn, C.c_void_p), C.cast(cp, C.c_void_p),
                                   C.cast(ce, C.c_void_p), n, C.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib.itts_cfm_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def forward_merged(self, x_t, x_merged, t):
        """x_t [B, T, in_ch], x_merged [B, T, merged], t [B] -> [B, in_ch, T]."""
        x_t = _f32(x_t, "x_t")
        x_merged = _f32(x_merged, "x_merged")
        t = _f32(t, "t")
        if x_t.ndim != 3 or x_merged.ndim != 3:
            raise ValidationError(1, "x_t: expected [B, T, in_ch] and [B, T, merged] arrays")
        B, T = x_t.shape[0], x_t.shape[1]
        if (x_t.shape[2] != self.cfg["in_ch"] or x_merged.shape != (B, T, merged_dim(self.cfg))
                or t.shape != (B,)):
            raise ValidationError(1, "x_merged: shapes do not match the estimator")
        out = np.empty((B, self.cfg["in_ch"], T), np.float32)
        _check(lib.itts_cfm_forward(self.h, x_t.ctypes.data, x_merged.ctypes.data, t.ctypes.data, B, T,
                                    out.ctypes.data))
        return out

    def solve_euler(self, cat_condition, ref_mel, style, noise_z, n_timesteps=25, cfg_rate=0.7):
        """cat_condition [1, T_total, dim], ref_mel [1, in_ch, T_ref], style [1, style],
        noise_z [1, in_ch, T_total] -> generated mel [1, in_ch, T_total - T_ref]."""
        cc = _f32(cat_condition, "cat_condition")
        rm = _f32(ref_mel, "ref_mel")
        st = _f32(style, "style")
        nz = _f32(noise_z, "noise_z")
        d, ch = self.cfg["dim"], self.cfg["in_ch"]
        if cc.ndim != 3 or cc.shape[0] != 1 or cc.shape[2] != d:
            raise ValidationError(1, f"cat_condition: expected [1, T_total, {d}], got shape {list(cc.shape)}")
        if rm.ndim != 3 or rm.shape[0] != 1 or rm.shape[1] != ch:
            raise ValidationError(1, f"ref_mel: expected [1, {ch}, T_ref], got shape {list(rm.shape)}")
        if st.shape != (1, self.cfg["style_dim"]):
            raise ValidationError(1, f"style: expected [1, {self.cfg['style_dim']}], got shape {list(st.shape)}")
        T, Tr = cc.shape[1], rm.shape[2]
        if nz.shape != (1, ch, T):
            raise ValidationError(1, f"noise_z: expected shape [1, {ch}, {T}], got {list(nz.shape)}")
        out = np.empty((1, ch, max(T - Tr, 0)), np.float32)
        _check(lib.itts_cfm_solve_euler(self.h, cc.ctypes.data, T, rm.ctypes.data, Tr, st.ctypes.data,
                                        nz.ctypes.data, int(n_timesteps), C.c_float(cfg_rate), out.ctypes.data))
        return out

    def last_timing_ms(self) -> float:
        """Device time of the last solve_euler call (HIP events around the Euler loop)."""
        ms = C.c_float()
        _check(lib.itts_cfm_last_solve_ms(self.h, C.byref(ms)))
        return ms.value
