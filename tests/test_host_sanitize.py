"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

tests/sanitize/Makefile builds, with g++/gcc -fsanitize=address,undefined:
  * host_check: the product's CSR -> BCSR host converter (csrc/abi.cpp, the
    replacement of convert_wrapper.cpp:27-180) checked against the C oracle
    on 1,600 random cases and its error paths;
  * liboracle_san.so: the C oracle, against which tests/test_oracle.py and
    tests/test_repack_oracle.py run in a child process with libasan preloaded.
"""
import os
import shutil
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SAN = os.path.join(HERE, "sanitize")
ROOT = os.path.dirname(HERE)


def _build():
    if not (shutil.which("g++") and shutil.which("gcc") and shutil.which("make")):
        pytest.skip("no host C/C++ toolchain")
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(libasan) or not os.path.exists(libasan):
        pytest.skip("libasan not available")
    r = subprocess.run(["make", "-s", "-C", SAN], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return libasan


def test_host_converter_under_asan_ubsan():
    _build()
    r = subprocess.run([os.path.join(SAN, "build", "host_check")], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ok" in r.stdout


def test_oracle_under_asan_ubsan():
    libasan = _build()
    env = dict(os.environ, LD_PRELOAD=libasan, ASAN_OPTIONS="detect_leaks=0",
               GRWS_ORACLE_LIB=os.path.join(SAN, "build", "liboracle_san.so"))
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(HERE, "test_oracle.py"), os.path.join(HERE, "test_repack_oracle.py")],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "passed" in r.stdout
