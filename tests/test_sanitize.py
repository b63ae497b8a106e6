"""The library's host-side C++ under AddressSanitizer and UndefinedBehaviorSanitizer, on the
CPU (no GPU code is built here):

- the .cpu.bin reader (tabinfer_amd/csrc/ti_cpubin.hip, host C++, with ti_error.hip) linked
  into tests/sanitize/fuzz_cpubin.cc: the corrupted-container cases of
  native/crates/n2-core/src/binfmt.rs:430-482, then seeded mutations of a valid container,
  every accessor run on whatever parses (binfmt.rs:234-257's rules hold or a report aborts);
- the N-API addon (tabinfer_amd/host/ti_node.cc) loaded into node with the sanitizer
  runtime preloaded, driven by tests/sanitize/fuzz_addon.js: every export called with wrong
  argument counts and types, container handles used after close and closed twice.

Both stop at their first failure. The sources are copied to .cc files in a temporary
directory and compiled there with g++."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "tabinfer_amd", "csrc")
SAN = os.path.join(ROOT, "tests", "sanitize")
INCLUDE = os.path.join(ROOT, "include")
GXX = shutil.which("g++")
NODE = shutil.which("node")
FLAGS = ["-O1", "-g", "-std=c++17", "-fno-omit-frame-pointer", "-fno-sanitize-recover=all"]
SANITIZE = ["-fsanitize=" + s for s in ("address", "undefined")]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:verify_asan_link_order=0:abort_on_error=1",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")

pytestmark = pytest.mark.skipif(GXX is None, reason="g++ is not installed")


def runtime(name):
    p = subprocess.run([GXX, "-print-file-name=" + name], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


@pytest.fixture(scope="module")
def fuzz_cpubin(tmp_path_factory):
    d = tmp_path_factory.mktemp("san")
    srcs = []
    for f in ("ti_cpubin", "ti_error"):
        dst = str(d / (f + ".cc"))
        shutil.copyfile(os.path.join(CSRC, f + ".hip"), dst)
        srcs.append(dst)
    exe = str(d / "fuzz_cpubin")
    cmd = [GXX] + FLAGS + SANITIZE + ["-I", INCLUDE, "-I", CSRC, os.path.join(SAN, "fuzz_cpubin.cc")] + srcs + ["-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_cpubin_reader_under_sanitizers(fuzz_cpubin, seed):
    r = subprocess.run([fuzz_cpubin, "60000", str(seed)], capture_output=True, text=True, timeout=300, env=ENV)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok 60000 iterations")
    parsed = int(r.stdout.split()[3])
    assert parsed > 100          # enough mutants parse for the accessors to be exercised


@pytest.mark.skipif(NODE is None or not os.path.exists("/usr/include/node/node_api.h"),
                    reason="node or its headers are not installed")
def test_addon_marshalling_under_sanitizers(tmp_path):
    lib = os.path.join(ROOT, "tabinfer_amd", "libtabinfer.so")
    if not os.path.exists(lib):
        pytest.fail("libtabinfer.so is not built: run python -m tabinfer_amd.build")
    asan, ubsan = runtime("libasan.so"), runtime("libubsan.so")
    if not asan or not ubsan:
        pytest.skip("the sanitizer runtimes are not installed")
    addon = str(tmp_path / "tabinfer.node")
    src = str(tmp_path / "ti_node.cc")
    shutil.copyfile(os.path.join(ROOT, "tabinfer_amd", "host", "ti_node.cc"), src)
    cmd = [GXX] + FLAGS + SANITIZE + ["-shared", "-fPIC", "-DNODE_GYP_MODULE_NAME=tabinfer", "-I", "/usr/include/node",
                                      "-I", INCLUDE, src, "-L", os.path.dirname(lib), "-ltabinfer",
                                      "-Wl,-rpath," + os.path.dirname(lib), "-o", addon]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    env = dict(ENV, LD_PRELOAD=asan + " " + ubsan)
    for seed in (1, 2):
        r = subprocess.run([NODE, "--expose-gc", os.path.join(SAN, "fuzz_addon.js"), addon, "6000", str(seed)],
                           capture_output=True, text=True, timeout=300, env=env)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
        assert '"ok":true' in r.stdout and '"exports":' in r.stdout
