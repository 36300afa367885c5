"""The device exp (glibc_expf.h) returns glibc's expf bits for every float.

Rust's f32::exp (src/ops/activation.rs:6,15) is glibc's expf on x86_64
Linux, and the oracle calls it directly; the GPU kernels use hale_expf.  The
same header compiled for the host is compared with glibc on all 2^32 inputs
(IEEE double arithmetic and fma give the same bits on host and device).
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_hale_expf_equals_glibc_expf_on_every_float(tmp_path):
    exe = tmp_path / "expf_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-mfma",
                    "-I", os.path.join(ROOT, "hale-token_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "expf_check.c"), "-o", str(exe), "-lm"],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert int(out.strip()) == 0
