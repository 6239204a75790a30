import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("index-tts-rs_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
    config.addinivalue_line("markers", "slow: full-size workload (seconds to minutes)")


@pytest.fixture(scope="session")
def tiny_weights():
    from itts_hip import synth

    return synth.make_weights(synth.TINY_CONFIG, seed=11, init="rich")


@pytest.fixture(scope="session")
def tiny_prompt(tiny_weights):
    from itts_hip import synth

    return synth.make_prompt(tiny_weights.cfg, n_cond=3, n_text=12, seed=5)


def _full(cfg_over, seed):
    import ito
    import itts_hip as H
    from itts_hip import synth

    print(f"[gpu] full-size decoder weights {cfg_over or ''} seed {seed}", flush=True)
    W = synth.make_weights(dict(synth.FULL_CONFIG, **cfg_over), seed=seed)
    ito.lib.ito_set_threads(16)
    g = H.Gpt(W)
    return W, g, ito.Model(W)


@pytest.fixture(scope="session")
def full_model():
    """The decoder at its real shape (int8 codes, fp16 group params, spec init): weights,
    the HIP decoder and the oracle over the same arrays."""
    W, g, M = _full({}, 11)
    yield W, g, M
    g.close()


@pytest.fixture(scope="session")
def full_int4():
    """The real shape with 4-bit codes."""
    W, g, M = _full({"quant_bits": 4}, 13)
    yield W, g, M
    g.close()


@pytest.fixture(scope="session")
def full_f32_params():
    """The real shape with F32 group parameters, the dtype of the shipped checkpoint."""
    import itts_hip as H

    W, g, M = _full({"param_dtype": H.ITTS_F32}, 19)
    yield W, g, M
    g.close()
