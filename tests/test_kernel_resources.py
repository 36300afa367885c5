"""Resource check of every gfx950 kernel, from the compiler's own report.

`make resources` compiles each kernel unit's device code with the
library's flags and -Rpass-analysis=kernel-resource-usage.  A kernel that
needs scratch memory has spilled registers (or uses a stack): its spill
stores and reloads sit in the hot loop and wait on memory, as they did in
the whole-chain down kernel before its activation staging was sized per
variant.  No kernel of the library may use scratch, and the kernels whose
speed rests on a wave count keep it.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "hale-token_amd")
UNITS = ["kernels_decode", "kernels_prefill", "kernels_float", "kernels_attn"]

# (kernel name regex, least waves per SIMD the kernel is written for)
OCCUPANCY = [
    (r"k_grouped", 4),           # grouped prefill: four waves per SIMD (128 VGPRs)
    (r"k_gemvILi\d+ELi1ELi16E", 4),  # sixteen-wave gate/up: one work-group of 1024 threads per CU
    (r"k_down_combine", 2),      # eight-wave down + combine
    (r"k_down_tile", 4),         # sixteen-wave top-2 down: one work-group of 1024 threads per CU
]

REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]|"
                    r"Occupancy \[waves/SIMD\]|Dynamic Stack): (\S+)")


def parse(text):
    """{kernel: {field: value}} from one unit's resource remarks."""
    out, cur = {}, None
    for line in text.splitlines():
        m = REMARK.search(line)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = val
            out[cur] = {}
        elif cur is not None:
            out[cur][key] = val
    return out


@pytest.fixture(scope="module")
def report():
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    if not (os.path.exists(hipcc) or shutil.which("hipcc")) or not shutil.which("make"):
        pytest.skip("no hipcc to compile the kernels with")
    p = subprocess.run(["make", "-C", PKG, "-j4", "resources"], capture_output=True, text=True,
                       timeout=900)
    assert p.returncode == 0, p.stderr[-3000:]
    res = {}
    for u in UNITS:
        with open(os.path.join(PKG, "_build", u + ".res")) as f:
            res[u] = parse(f.read())
        assert res[u], f"no resource remarks for {u}"
    return res


def test_every_unit_reports_its_kernels(report):
    names = [k for u in UNITS for k in report[u]]
    for kernel in ("k_gemv", "k_down_combine", "k_down_chain", "k_down_tile", "k_route_logits", "k_grouped",
                   "k_group", "k_combine"):
        assert any(kernel in n for n in names), kernel


def test_no_kernel_uses_scratch(report):
    bad = [(u, k, r.get("ScratchSize [bytes/lane]"), r.get("VGPRs"))
           for u in UNITS for k, r in report[u].items()
           if int(r.get("ScratchSize [bytes/lane]", "0")) != 0 or r.get("Dynamic Stack") == "True"]
    assert not bad, f"kernels with scratch (spills): {bad}"


def test_occupancy_of_the_hot_kernels(report):
    seen = set()
    for u in UNITS:
        for k, r in report[u].items():
            for pat, least in OCCUPANCY:
                if re.search(pat, k):
                    seen.add(pat)
                    assert int(r["Occupancy [waves/SIMD]"]) >= least, (k, r)
    assert seen == {p for p, _ in OCCUPANCY}
