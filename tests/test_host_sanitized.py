"""Memory safety of libsigcomp_host.so on corrupt inputs: the seeded mutation
fuzz of tests/host_fuzz.py, run against the product library in-process and
against an AddressSanitizer + UBSan build of the same source in a child
process (sanitizer runtimes preloaded into the interpreter)."""

import os
import shutil
import subprocess
import sys

import pytest

from conftest import REPO

SRC = REPO / "sigcomp_amd" / "csrc" / "sc_host.cpp"


def _runtime(name):
    gxx = shutil.which("g++")
    if gxx is None:
        return None
    path = subprocess.run([gxx, f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def test_fuzz_product_library_raises_only_documented_errors():
    from sigcomp_amd import _host
    if not _host.LIB_PATH.exists():
        pytest.skip("libsigcomp_host.so not built")
    sys.path.insert(0, str(REPO / "tests"))
    import host_fuzz
    stats = host_fuzz.run(seed=11, iters=150)
    # every parser saw both accepted and rejected inputs
    for name in ("parse", "rice", "reassemble", "scan", "index"):
        assert stats.get(name + "_ok", 0) > 0 and stats.get(name + "_err", 0) > 0, stats


@pytest.mark.parametrize("seed", [0, 1])
def test_fuzz_under_address_and_undefined_behaviour_sanitizers(tmp_path, seed):
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if asan is None or ubsan is None:
        pytest.skip("g++ sanitizer runtimes not available")
    lib = tmp_path / "libsigcomp_host_san.so"
    build = subprocess.run(["g++", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
                            "-fno-omit-frame-pointer", "-std=c++17", "-fPIC", "-shared", "-pthread",
                            f"-I{REPO / 'include'}", str(SRC), "-o", str(lib)], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-2000:]
    env = dict(os.environ, LD_PRELOAD=f"{asan} {ubsan}",
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    res = subprocess.run([sys.executable, str(REPO / "tests" / "host_fuzz.py"), "--lib", str(lib),
                          "--seed", str(seed), "--iters", "400"],
                         capture_output=True, text=True, env=env, timeout=600)
    report = (res.stdout + res.stderr)[-4000:]
    assert res.returncode == 0, report
    assert "AddressSanitizer" not in res.stderr and "runtime error" not in res.stderr, report
