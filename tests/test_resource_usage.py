"""Register and scratch budgets of the kernels, from the compiler.

Compiles ``csrc/*.hip`` for gfx950 with the library's own flags and
``-Rpass-analysis=kernel-resource-usage``, and checks every kernel instance's
per-lane scratch (and, for stage 1, waves per SIMD) against the budgets the
kernels are designed to.  A change that makes a kernel spill (or spill more), or drops
the LDS-resident kernel below three waves per SIMD, fails here on the CPU,
before any GPU run.  Needs ``hipcc``; runs no GPU code.
"""
import concurrent.futures
import os
import re
import shutil
import subprocess

import pytest

from unum_ops_amd import build

SRC = os.path.join(build.HERE, "csrc", "stage1.hip")

# Per-lane scratch allowed for instances that spill (mangled-name fragment ->
# bytes); every instance not listed must use none.  None is listed: the
# LDS-resident kernel's eight-quad rows (fp32 and bf16 scores, and with the
# fused pool) fit their 168 VGPRs -- the row's 64 exponentials included --
# since each row's queries load at its start instead of a row ahead.
SCRATCH_BUDGET = {}


def _hipcc():
    return shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else None)


def _resource_usage(src, out):
    """{kernel: {"VGPRs", "ScratchSize", "Occupancy"}} of one source."""
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc is not installed")
    cmd = [hipcc, *build.HIP_FLAGS, *build.FILE_FLAGS.get(os.path.basename(src), []),
           "-Rpass-analysis=kernel-resource-usage", "--offload-device-only", "-c", src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stderr[-3000:]
    kernels = {}
    name = None
    for line in r.stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            kernels[name] = {}
            continue
        m = re.search(r"remark:\s+(ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]|VGPRs): (\d+)", line)
        if m and name is not None:
            kernels[name][m.group(1).split()[0]] = int(m.group(2))
    return kernels


OTHER = ["sparse_attn", "maxpool", "compress", "block_table"]


@pytest.fixture(scope="module")
def all_usage(tmp_path_factory):
    """Every source compiled at once (the compiles are independent)."""
    d = tmp_path_factory.mktemp("ru")
    names = ["stage1", *OTHER]
    with concurrent.futures.ThreadPoolExecutor(len(names)) as ex:
        futs = {n: ex.submit(_resource_usage, os.path.join(build.HERE, "csrc", n + ".hip"), d / (n + ".o"))
                for n in names}
        return {n: f.result() for n, f in futs.items()}


@pytest.fixture(scope="module")
def usage(all_usage):
    return all_usage["stage1"]


@pytest.mark.parametrize("name", OTHER)
def test_other_kernels_use_no_scratch(name, all_usage):
    usage = all_usage[name]
    assert usage, name
    spills = [(n, r["ScratchSize"]) for n, r in usage.items() if r["ScratchSize"] != 0]
    assert not spills, spills


def test_every_kernel_instance_reported(usage):
    kinds = {k: sum(1 for n in usage if k in n) for k in
             ("stage1_lds_kernel", "stage1_stream_kernel", "stage1_decode_kernel",
              "stage1_mfma_kernel", "stage1_generic_kernel")}
    assert all(v > 0 for v in kinds.values()), kinds
    assert all("ScratchSize" in v and "Occupancy" in v and "VGPRs" in v for v in usage.values())
    # The LDS-resident kernel's largest rows are known to need more than 128 VGPRs.
    assert max(v["VGPRs"] for n, v in usage.items() if "stage1_lds_kernel" in n) > 128


def test_scratch_within_budget(usage):
    over = []
    for name, r in usage.items():
        budget = next((b for frag, b in SCRATCH_BUDGET.items() if frag in name), 0)
        if r["ScratchSize"] > budget:
            over.append((name, r["ScratchSize"], budget))
    assert not over, over


def test_lds_kernel_keeps_three_waves_per_simd(usage):
    low = [(n, r["Occupancy"]) for n, r in usage.items() if "stage1_lds_kernel" in n and r["Occupancy"] < 3]
    assert not low, low
