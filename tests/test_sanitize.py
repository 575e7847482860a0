"""The library's host code and the CPU oracle under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only; tests/sanitize/).

host_fuzz: SDEC headers of versions 1-5 mutated 20000 times through
sde_model_read_header, the arena sizing of every parsed header and of
200000 random configurations (sde_model_weights_bytes), and 200000 random
KV configurations (sde_kv_config_validate / sde_kv_pool_bytes), each against
the harness's own restatement of the rules (128-bit sizes).  oracle_check:
the oracle's conversions, append / gather, attention and GEMV on random
shapes with exactly sized buffers.  Any sanitizer report fails the run.
"""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent / "sanitize"


@pytest.fixture(scope="module")
def built():
    if not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not available")
    if not shutil.which("gcc") or not shutil.which("make"):
        pytest.skip("gcc / make not available")
    env = dict(os.environ)
    env.setdefault("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
    r = subprocess.run(["make", "-s", "-C", str(HERE), "-j4"], capture_output=True, text=True,
                       env=env, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    return HERE / "_build"


def _run(cmd):
    env = dict(os.environ, UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=300)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    return out


def test_host_code_fuzz_under_sanitizers(built):
    out = _run([str(built / "host_fuzz"), "1", "1"])
    assert "host fuzz: all checks passed" in out


def test_oracle_under_sanitizers(built):
    out = _run([str(built / "oracle_check"), "300", "1"])
    assert "oracle check: 300 cases, all checks passed" in out
