"""Host sanitizer runs (CPU only) of the test infrastructure's C code and of
the provider-selection header:

* the oracle (oracle/attn_oracle.c) with every exported function driven on
  small and edge shapes by tests/cpp/oracle_sanitize_check.c, built with
  AddressSanitizer + UndefinedBehaviorSanitizer, no recovery;
* tests/test_oracle.py re-run in a child process against an UBSan build of
  the oracle library (UBSan's runtime loads into an uninstrumented Python;
  ASan's must come first in the process, hence the separate driver above);
* include/mugen_attn_path.hpp through tests/cpp/path_select_check.cpp under
  ASan + UBSan, with the same output as the plain build."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")


def _cc(name):
    c = shutil.which(name)
    if c is None:
        pytest.skip(f"no {name}")
    return c


def test_oracle_asan_ubsan(tmp_path):
    exe = str(tmp_path / "oracle_sanitize_check")
    subprocess.run([_cc("gcc"), "-std=c11", "-fopenmp", "-ffp-contract=off", *SAN,
                    os.path.join(ROOT, "tests", "cpp", "oracle_sanitize_check.c"),
                    os.path.join(ROOT, "oracle", "attn_oracle.c"), "-o", exe, "-lm"], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, env=ENV, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "PASS", r.stderr[-4000:]
    assert "runtime error" not in r.stderr and "ERROR: AddressSanitizer" not in r.stderr, r.stderr[-4000:]


def test_oracle_tests_under_ubsan(tmp_path):
    so = str(tmp_path / "liboracle_attn_ubsan.so")
    subprocess.run([_cc("gcc"), "-std=c11", "-fopenmp", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
                    "-fsanitize=undefined", "-fno-sanitize-recover=all", "-g", "-O1",
                    os.path.join(ROOT, "oracle", "attn_oracle.c"), "-o", so, "-lm"], check=True)
    env = dict(ENV, MUGEN_ORACLE_LIB=so)
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_oracle.py")],
                       capture_output=True, text=True, env=env, cwd=ROOT, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "runtime error" not in r.stdout + r.stderr


def test_path_select_asan_ubsan(tmp_path):
    exe = str(tmp_path / "path_select_check")
    plain = str(tmp_path / "path_select_plain")
    src = os.path.join(ROOT, "tests", "cpp", "path_select_check.cpp")
    inc = os.path.join(ROOT, "include")
    subprocess.run([_cc("g++"), "-std=c++17", *SAN, "-I", inc, src, "-o", exe], check=True)
    subprocess.run([_cc("g++"), "-std=c++17", "-O1", "-I", inc, src, "-o", plain], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, env=ENV, timeout=60)
    assert r.returncode == 0, r.stderr[-3000:]
    assert r.stdout == subprocess.run([plain], capture_output=True, text=True, check=True).stdout
