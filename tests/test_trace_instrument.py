"""The phase-trace instrumentation still applies to the persistent step's source: every
anchor it patches is present once (a kernel edit that moves a phase barrier shows here)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_instrument_applies(tmp_path):
    out = tmp_path / "kp_trace.hip"
    r = subprocess.run([sys.executable, os.path.join(ROOT, "index-tts-rs_amd", "trace", "instrument.py"),
                        os.path.join(ROOT, "index-tts-rs_amd", "csrc", "kernels_persist.hip"), str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert "16 phase stamps" in r.stdout
    text = out.read_text()
    assert 'extern "C" int itts_trace_read' in text
    for i in (0, 1, 2, 3, 4, 5, 6, 9, 10, 11, 12, 13, 14, 15, 16, 17):
        assert f"STAMP({i});" in text
