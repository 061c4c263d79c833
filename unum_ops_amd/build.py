"""Build the gfx950 C-ABI library ``unum_ops_amd/libunum_ops_amd.so`` in-tree.

Every ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` to an
object (in parallel), then linked into one shared library next to this file.
The library links the HIP runtime by its soname ``libamdhip64.so.7``; torch
imports its own copy of that runtime first, so the process holds one runtime.

Usage: ``python -m unum_ops_amd.build`` (or ``__graft_entry__.build()``).
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libunum_ops_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"

# Packed fp32 VALU ops (v_pk_*_f32) are disabled for all device code: some of
# their forms have given wrong results on this hardware without any error.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]

# Extra flags per source.  Stage 1 never produces or consumes a NaN (masked
# scores are -inf and every exp argument is finite or -inf), so it is built
# without NaN semantics: fmaxf then needs no quieting and the DPP lane moves
# fold into the max/add of the cross-lane reductions.  Its MFMA results are
# read by the VALU right away (exponentials), so they are kept in VGPRs
# (-amdgpu-mfma-vgpr-form); values that feed only MFMAs may then live in the
# accumulation registers.
FILE_FLAGS = {
    "stage1.hip": ["-fno-honor-nans", "-mllvm", "-amdgpu-mfma-vgpr-form"],
    # Stage 2 keeps its P.V accumulators across the whole loop; in the
    # accumulation registers the compiler copied them out and back every stage.
    "sparse_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc():
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return cand


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose=True, jobs=None):
    """Compile every kernel source and link the shared library. Returns its path."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(BUILD_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        extra = FILE_FLAGS.get(os.path.basename(src), [])
        return _run([hipcc, *HIP_FLAGS, *extra, "-c", src, "-o", obj])

    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for (src, _), out in zip(zip(srcs, objs), ex.map(compile_one, zip(srcs, objs))):
            if verbose and out.strip():
                print(out, file=sys.stderr)
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
