"""CPU sanitizer runs (AddressSanitizer + UndefinedBehaviorSanitizer, gcc,
-fno-sanitize-recover) of the host code that reads untrusted input and of
the oracle:

- the pack header reader (hale-token_amd/csrc/pack_header.cpp, the code
  behind hale_pack_open's JSON parsing) over the malformed-header cases of
  test_pack.py plus truncations, structural substitutions and ~55k random
  mutations of a valid header (tests/native/pack_header_fuzz.cpp);
- the oracle (oracle/hale_oracle.c) built with both sanitizers and loaded
  in place of the default build while test_oracle.py and test_golden.py
  run (the exhaustive F16C comparison, a separate program, left out).
"""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(REPO, "hale-token_amd", "csrc")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]


def _runtime(name):
    path = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(path) or not os.path.exists(path):
        pytest.skip(f"{name} is not installed")
    return path


def test_pack_header_reader_under_asan_ubsan(tmp_path):
    _runtime("libasan.so")
    exe = tmp_path / "pack_header_fuzz"
    subprocess.run(["g++", "-std=c++17", "-O1", *SAN, "-I", CSRC, os.path.join(CSRC, "pack_header.cpp"),
                    os.path.join(HERE, "native", "pack_header_fuzz.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300,
                       env=dict(os.environ, ASAN_OPTIONS="detect_leaks=1", UBSAN_OPTIONS="print_stacktrace=1"))
    assert r.returncode == 0, r.stderr[-4000:]
    accepted, rejected = map(int, r.stdout.split())
    assert accepted >= 3 and rejected > 50000


def test_oracle_under_asan_ubsan(tmp_path):
    asan = _runtime("libasan.so")
    so = tmp_path / "libhale_oracle_san.so"
    subprocess.run(["gcc", "-O1", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC",
                    *SAN, "-shared", "-o", str(so), os.path.join(REPO, "oracle", "hale_oracle.c"), "-lm"],
                   check=True)
    env = dict(os.environ, HALE_ORACLE_LIB=str(so), LD_PRELOAD=asan,
               ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
                        "-k", "not f16c", os.path.join(HERE, "test_oracle.py"),
                        os.path.join(HERE, "test_golden.py")],
                       capture_output=True, text=True, timeout=900, env=env, cwd=REPO)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out
    assert " passed" in out


def test_sanitized_oracle_catches_an_overread(tmp_path):
    """The sanitized build is the one loaded and reports: decode_row asked
    for 64 q8_0 values from a 10-byte row reads past it."""
    asan = _runtime("libasan.so")
    so = tmp_path / "libhale_oracle_san.so"
    subprocess.run(["gcc", "-O1", "-std=c11", "-fopenmp", "-fPIC", *SAN, "-shared", "-o", str(so),
                    os.path.join(REPO, "oracle", "hale_oracle.c"), "-lm"], check=True)
    code = ("import sys; sys.path[:0] = ['oracle']\n"
            "import numpy as np, oracle as O\n"
            "row, out = np.zeros(10, np.uint8), np.zeros(64, np.float32)\n"
            "O.lib().orc_decode_row(O.Q8_0, row.ctypes.data_as(O._u8p), out.ctypes.data_as(O._fp), 64)\n")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120, cwd=REPO,
                       env=dict(os.environ, HALE_ORACLE_LIB=str(so), LD_PRELOAD=asan,
                                ASAN_OPTIONS="detect_leaks=0"))
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr
