"""The committed profile summaries describe kernels that exist: every kernel name in
profiles/*.md is a __global__ function of tabinfer_amd/csrc, and every summary gives the
commit it was measured at and the command that made it (CPU only)."""
import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _kernels_defined():
    names = set()
    for path in glob.glob(os.path.join(ROOT, "tabinfer_amd", "csrc", "*.hip")):
        with open(path) as f:
            src = f.read()
        names.update(re.findall(r"__global__\s+(?:__launch_bounds__\([^)]*\)\s+)?void\s+(k_\w+)\s*\(", src, re.S))
    return names


def _summaries():
    return sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md")))


def test_profiles_name_only_existing_kernels():
    defined = _kernels_defined()
    assert "k_fgemv" in defined and "k_attn_fused_pv" in defined
    missing = {}
    for path in _summaries():
        with open(path) as f:
            named = set(re.findall(r"\b(k_[a-z0-9_]+?)(?=[<\s`|(,;:]|\.(?!hip)|$)", f.read(), re.M))
        gone = sorted(n for n in named if n not in defined)
        if gone:
            missing[os.path.basename(path)] = gone
    assert not missing, missing


def test_profiles_are_stamped_with_their_commit_and_command():
    for path in _summaries():
        with open(path) as f:
            text = f.read()
        assert re.search(r"^Measured at commit [0-9a-f]{7,40}\b", text, re.M), path
        assert "rocprofv3 " in text and "bench.py" in text, path
