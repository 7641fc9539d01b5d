"""The C ABI's host-side argument validation under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only).

The library sources are compiled with AddressSanitizer and
UndefinedBehaviorSanitizer on the host side only (each sanitizer flag scoped by
``-Xarch_host``; the link line also passes ``-fno-gpu-sanitize``), so the
gfx950 device code is built plain, and linked with
``tests/sanitize/abi_validation.cpp``, which calls every entry point with
arguments each check must reject (null pointers, negative or unsupported
sizes, short workspaces, an input past the allocation-free scratch) and the
size queries at the edges of ``int``.  None of those calls reaches a HIP API,
so the run needs no GPU; any sanitizer report fails the test.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from conftest import REPO

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CSRC = REPO / "fast-mimi_amd" / "csrc"
OUT = REPO / "fast-mimi_amd" / "_build" / "sanitize"


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
def test_abi_validation_under_asan_ubsan():
    OUT.mkdir(parents=True, exist_ok=True)
    exe = OUT / "abi_validation"
    sources = sorted(CSRC.glob("*.hip"))
    san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer"]
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", *san,
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", str(CSRC), "-I", str(REPO / "include")]

    def compile_one(src):
        obj = OUT / (src.stem + ".o")
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        proc = subprocess.run([HIPCC, *flags, *lang, "-c", str(src), "-o", str(obj)],
                              capture_output=True, text=True)
        assert proc.returncode == 0, f"{src.name}:\n{proc.stderr[-4000:]}"
        return str(obj)

    with ThreadPoolExecutor(max_workers=6) as pool:
        objects = list(pool.map(compile_one, sources + [REPO / "tests" / "sanitize" / "abi_validation.cpp"]))
    proc = subprocess.run([HIPCC, "--offload-arch=gfx950", "-fno-gpu-sanitize",
                           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                           *objects, "-o", str(exe)], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", HIP_VISIBLE_DEVICES="")
    run = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=120)
    report = run.stdout + run.stderr
    assert run.returncode == 0 and "runtime error" not in report and "AddressSanitizer" not in report, report
    assert "ok: 0 failure(s)" in run.stdout
