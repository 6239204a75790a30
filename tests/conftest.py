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
