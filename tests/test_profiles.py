"""The committed rocprof summaries describe the kernels as they are built now.

Every summary under ``profiles/`` that quotes a duration or traffic records
the sha256 (first 16 hex digits) of each kernel source it was measured on, and
the commands that produced it.  A kernel change without new profiles would
leave figures that no longer describe the build (bench.py then reports no
``traffic``); this test catches that on the CPU.
"""
import glob
import hashlib
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROFILES = sorted(glob.glob(os.path.join(ROOT, "profiles", "*.txt")))


def _sha16(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def test_profiles_exist():
    assert PROFILES, "no rocprof summaries under profiles/"


@pytest.mark.parametrize("path", PROFILES, ids=[os.path.basename(p) for p in PROFILES])
def test_profile_matches_sources(path):
    text = open(path).read()
    pins = re.findall(r"^source_sha256: ([0-9a-f]{16})\s+\(([^,)]+)", text, re.M)
    assert pins, f"{os.path.basename(path)} records no source_sha256"
    for sha, src in pins:
        src_path = os.path.join(ROOT, src.strip())
        assert os.path.exists(src_path), f"{os.path.basename(path)}: {src} does not exist"
        assert _sha16(src_path) == sha, (
            f"{os.path.basename(path)} was measured on {src} {sha}, the source is now {_sha16(src_path)}: "
            "regenerate the profile")
    assert re.search(r"rocprofv3 ", text), f"{os.path.basename(path)} gives no rocprofv3 command"
