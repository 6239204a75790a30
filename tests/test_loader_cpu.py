"""The safetensors loader (Gpt::load_from_path, crates/core/src/models/gpt.rs:522) checks the
file the way the reference does before any device work: the header prefix and data section
(crates/core/src/models/loader.rs:1410-1458), then every tensor by name, shape and dtype
(tensor_array_shaped, loader.rs:316-331; Gpt::from_weights gpt.rs:477-515).  These cases
all fail before the device is touched, so they run without a GPU."""
import ctypes as C
import struct

import numpy as np
import pytest

import itts_hip as H
from itts_hip import synth


@pytest.fixture(scope="module")
def tiny_ckpt(tmp_path_factory):
    cfg = dict(synth.TINY_CONFIG, param_dtype=H.ITTS_F32)
    W = synth.make_weights(cfg, seed=3, init="rich")
    return W, tmp_path_factory.mktemp("ckpt")


def load(path):
    h = C.c_void_p()
    st = H.lib.itts_gpt_load_safetensors(str(path).encode(), C.byref(h))
    if st == H.ITTS_OK:
        H.lib.itts_gpt_destroy(h)
    return st, H.last_error()


def test_valid_checkpoint_passes_validation(tiny_ckpt):
    W, d = tiny_ckpt
    p = d / "ok.safetensors"
    synth.save_safetensors(W, str(p))
    st, msg = load(p)
    # without a GPU the decoder cannot be created: validation passed, the device step failed
    assert st in (H.ITTS_OK, H.ITTS_E_DEVICE), msg


@pytest.mark.parametrize("name", ["text_embedding.weight", "gpt.h.1.attn.c_proj.scales",
                                  "gpt.h.0.mlp.c_fc.bias", "final_norm.bias", "mel_head.biases"])
def test_missing_tensor(tiny_ckpt, name):
    W, d = tiny_ckpt
    p = d / "missing.safetensors"
    synth.save_safetensors(W, str(p), drop=(name,))
    st, msg = load(p)
    assert st == H.ITTS_E_WEIGHT
    assert msg == f"weight load error in `{name}`: missing required parameter tensor"


def test_wrong_shape(tiny_ckpt):
    W, d = tiny_ckpt
    p = d / "shape.safetensors"
    D = W.cfg["d_model"]
    synth.save_safetensors(W, str(p), override={"gpt.h.0.ln_2.bias": np.zeros(D + 1, np.float32)})
    st, msg = load(p)
    assert st == H.ITTS_E_WEIGHT
    assert msg == f"weight load error in `gpt.h.0.ln_2.bias`: expected shape [{D}], found [{D + 1}]"


def test_wrong_dtype(tiny_ckpt):
    W, d = tiny_ckpt
    p = d / "dtype.safetensors"
    synth.save_safetensors(W, str(p), override={"mel_head.bias": W.head.bias.astype(np.float16)})
    st, msg = load(p)
    assert st == H.ITTS_E_WEIGHT and msg.startswith("weight load error in `mel_head.bias`: unsupported dtype F16")


def test_mixed_param_dtypes_rejected(tiny_ckpt):
    W, d = tiny_ckpt
    p = d / "mixed.safetensors"
    s = W.layers[0].c_fc.scales.astype(np.float16)
    synth.save_safetensors(W, str(p), override={"gpt.h.0.mlp.c_fc.scales": s})
    st, msg = load(p)
    assert st == H.ITTS_E_WEIGHT and "gpt.h.0.mlp.c_fc.scales" in msg


def test_header_and_data_section(tiny_ckpt):
    W, d = tiny_ckpt
    good = d / "good.safetensors"
    synth.save_safetensors(W, str(good))
    raw = good.read_bytes()
    cases = {
        "short": (b"\x01\x02\x03", "safetensors file smaller than 8-byte header prefix"),
        "zero": (struct.pack("<Q", 0) + raw[8:], "invalid safetensors header length 0"),
        "huge": (struct.pack("<Q", 100_000_001) + raw[8:], "invalid safetensors header length 100000001"),
        "past_end": (struct.pack("<Q", len(raw)) + raw[8:], "safetensors header length exceeds file size"),
        "truncated": (raw[:-4], "safetensors data section length does not match file size"),
        "trailing": (raw + b"\x00" * 4, "safetensors data section length does not match file size"),
    }
    for name, (data, want) in cases.items():
        p = d / f"{name}.safetensors"
        p.write_bytes(data)
        st, msg = load(p)
        assert st == H.ITTS_E_WEIGHT, name
        assert msg == f"weight load error in `gpt_int8.safetensors`: {want}", (name, msg)
    # a header that is not the safetensors JSON object
    n = struct.unpack("<Q", raw[:8])[0]
    bad = bytearray(raw)
    bad[8] = ord("[")
    p = d / "json.safetensors"
    p.write_bytes(bytes(bad))
    st, msg = load(p)
    assert st == H.ITTS_E_WEIGHT and "safetensors header parse failed" in msg
    assert n > 0


def test_unreadable_path(tiny_ckpt):
    _, d = tiny_ckpt
    st, msg = load(d / "does_not_exist.safetensors")
    assert st == H.ITTS_E_WEIGHT and msg.startswith("weight load error in `gpt_int8.safetensors`: cannot open")
