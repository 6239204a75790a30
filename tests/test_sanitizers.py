"""Host code under AddressSanitizer and UBSan, on the CPU: the library's host side (ABI
runtime, safetensors loader, CFM host code) built with -fsanitize=address,undefined on
the host pass (index-tts-rs_amd `make asan`) runs the loader and ABI tests, and the oracle
built the same way with gcc (oracle `make asan`) runs the oracle tests.  Each suite runs
in a child python with the matching sanitizer runtime preloaded; any report aborts it."""
import glob
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


def _pytest(files, env):
    cmd = [sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu"] + \
          [os.path.join(ROOT, "tests", f) for f in files]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    return r.stdout


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc is needed to build the sanitizer variant of the library")
def test_library_host_code_under_asan_ubsan():
    subprocess.run(["make", "-s", "-j8", "-C", os.path.join(ROOT, "index-tts-rs_amd"), "asan"], check=True,
                   timeout=900)
    rt = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rt:
        pytest.skip("clang ASan runtime not found")
    env = dict(ENV, LD_PRELOAD=rt[-1],
               ITTS_HIP_LIB=os.path.join(ROOT, "index-tts-rs_amd", "lib_asan", "libitts_hip.so"))
    out = _pytest(["test_loader_cpu.py", "test_abi_cpu.py"], env)
    assert "passed" in out


def test_oracle_under_asan_ubsan():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "asan"], check=True, timeout=900)
    libs = [subprocess.run(["gcc", f"-print-file-name={n}"], capture_output=True, text=True).stdout.strip()
            for n in ("libasan.so", "libubsan.so")]
    if not all(os.path.isabs(p) and os.path.exists(p) for p in libs):
        pytest.skip("gcc sanitizer runtimes not found")
    env = dict(ENV, LD_PRELOAD=":".join(libs),
               ITO_LIB=os.path.join(ROOT, "oracle", "_build_asan", "libitts_oracle.so"))
    out = _pytest(["test_oracle_model.py", "test_oracle_sampler.py", "test_oracle_formats.py",
                   "test_oracle_replay.py", "test_oracle_streams.py", "test_oracle_independent.py",
                   "test_oracle_cfm.py"], env)
    assert "passed" in out
