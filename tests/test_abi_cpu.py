"""The C-ABI library loads without a GPU, exports every symbol include/itts_hip.h
declares, and its host-side entry points (quantiser, RNG, seen set, parameter
validation) agree with the oracle bit for bit."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import ito
import itts_hip as H

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "itts_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(itts_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", H.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (itts_[a-z0-9_]+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        getattr(H.lib, n)
    assert set(H.EXPORTED_SYMBOLS) == set(names)


def test_version_and_defaults():
    assert "gfx950" in H.version()
    c = H.lib.itts_config_default()
    assert (c.n_layer, c.d_model, c.n_head, c.d_ffn, c.mel_vocab, c.text_vocab, c.lang_vocab,
            c.mel_pos_len, c.text_pos_len, c.quant_bits) == (24, 1280, 20, 5120, 8194, 60510, 107,
                                                             1818, 602, 8)
    p = H.lib.itts_sampling_default()
    assert (p.greedy, p.top_k, p.max_mel_tokens) == (0, 3, 1500)
    assert abs(p.temperature - 0.8) < 1e-7 and abs(p.top_p - 0.8) < 1e-7
    assert p.repetition_penalty == 10.0


@pytest.mark.parametrize("bits,pd", [(8, H.ITTS_F16), (4, H.ITTS_F16), (8, H.ITTS_F32), (4, H.ITTS_F32)])
def test_library_quantizer_matches_oracle(bits, pd):
    rng = np.random.default_rng(bits * 10 + pd)
    w = (rng.standard_normal((300, 512)) * 0.02).astype(np.float32)
    w[3, :64] = 0.5                                     # constant group
    w[4, :] = np.linspace(-1, 1, 512, dtype=np.float32)
    a = H.quantize(w, bits, pd)
    b = ito.quantize(w, bits, pd)
    for x, y in zip(a, b):
        assert x.dtype == y.dtype and np.array_equal(x.view(np.uint8), y.view(np.uint8))


def test_rng_and_seen_match_oracle():
    for seed in (0, 7, 2**63 + 5, 2**64 - 1):
        r = H.SamplerRng(seed)
        s = C.c_uint64(ito.lib.ito_rng_init(seed))
        for _ in range(20):
            assert r.next_u64() == ito.lib.ito_rng_next_u64(C.byref(s))
            assert r.next_f32() == ito.lib.ito_rng_next_f32(C.byref(s))
    seen = H.SeenTokenBitSet()
    assert seen.contains(1) and seen.contains(8192) and not seen.contains(100)
    seen.insert(100)
    seen.insert(9000)        # ignored beyond 8255, as SeenTokenBitSet::insert
    assert seen.contains(100) and not seen.contains(9000)
    assert np.array_equal(H.SeenTokenBitSet().words, ito.seen_init())


def test_sampling_validation_matches_reference_ranges():
    H.SamplingParams().validate()
    bad = [dict(temperature=0.04), dict(top_p=0.001), dict(top_k=8195), dict(repetition_penalty=0.9),
           dict(max_mel_tokens=1816), dict(temperature=float("inf"))]
    for kw in bad:
        with pytest.raises(H.ValidationError) as e:
            H.SamplingParams(**kw).validate()
        assert e.value.message.split(":")[0] in kw
