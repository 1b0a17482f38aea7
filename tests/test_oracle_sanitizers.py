"""The CPU oracle under sanitizers (CPU only).

The oracle's own suites (sampler, speculative verification, numerics,
log-probabilities) run again in a child Python against a build of
oracle/tgs_oracle.c with AddressSanitizer and UndefinedBehaviorSanitizer
(tests/oracle_san/Makefile, every UB report fatal); and tgo_sample_batch /
tgo_spec_verify_batch run on 16 threads under ThreadSanitizer, their outputs
equal byte for byte to the same batches on one thread."""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SAN = os.path.join(HERE, "oracle_san")
SUITES = ["test_oracle_sampler.py", "test_oracle_spec.py", "test_oracle_numeric.py", "test_logprob_oracle.py"]


def _runtime(name):
    """The compiler's sanitizer runtime (a real file), or None."""
    r = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True)
    p = os.path.realpath(r.stdout.strip()) if r.returncode == 0 else ""
    return p if os.path.isfile(p) else None


def _make(target):
    if shutil.which("gcc") is None or shutil.which("make") is None:
        pytest.skip("needs gcc and make")
    r = subprocess.run(["make", "-s", "-C", SAN, target], capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip(f"sanitizer build unavailable: {r.stderr[-500:]}")


def test_oracle_suites_under_asan_and_ubsan():
    _make("asan")
    asan = _runtime("libasan.so")
    if asan is None:
        pytest.skip("no ASan runtime")
    env = dict(os.environ)
    env.update(LD_PRELOAD=asan, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               TGS_ORACLE_LIB=os.path.join(SAN, "build", "libtgs_oracle_asan.so"))
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        *[os.path.join(HERE, s) for s in SUITES]],
                       capture_output=True, text=True, env=env, cwd=ROOT, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-6000:]
    assert " passed" in r.stdout


def test_oracle_batches_under_tsan_on_16_threads():
    _make("tsan")
    exe = os.path.join(SAN, "build", "tsan_batch")
    if shutil.which("nm"):
        assert "__tsan_init" in subprocess.run(["nm", exe], capture_output=True, text=True).stdout
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1:exitcode=66")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-6000:]
    assert "ThreadSanitizer" not in out, out[-6000:]
    assert out.count(": ok") == 5, out
