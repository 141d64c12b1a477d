"""The C ABI's host-side argument checks under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only).

Every ``csrc/*.hip`` file is compiled with the sanitizers on its host code
only (device code is built as usual and never runs), linked with the driver
``tests/sanitize/abi_checks.cpp``, and run without a GPU: each call in the
driver must be refused before it reaches the HIP runtime -- bad dtypes,
missing or misaligned tensors, non-unit innermost strides, and sizes whose
products overflow 64 bits. A sanitizer report (an out-of-bounds read of a
stride array, a signed overflow in a size check) fails the test as surely as
a wrong return code.
"""

from __future__ import annotations

import os
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "techjam_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"
CLANG = "/opt/rocm/llvm/bin/clang++"
# Sanitizers on the host side of each compilation only.
HOST_SANITIZE = ("-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined "
                 "-Xarch_host -fno-sanitize-recover=undefined -Xarch_host -fno-omit-frame-pointer").split()


@pytest.fixture(scope="module")
def abi_checks_exe(tmp_path_factory) -> Path:
    if not (Path(HIPCC).exists() and Path(CLANG).exists()):
        pytest.skip("ROCm compilers not found")
    out = tmp_path_factory.mktemp("sanitize")

    def compile_one(src: Path) -> Path:
        obj = out / (src.stem + ".o")
        cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *HOST_SANITIZE,
               f"-I{ROOT / 'include'}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-4000:]
        return obj

    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        objs = list(pool.map(compile_one, sorted(CSRC.glob("*.hip"))))
    driver = out / "abi_checks.o"
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
    res = subprocess.run([CLANG, "-O1", "-g", "-std=c++17", *san, "-D__HIP_PLATFORM_AMD__",
                          f"-I{ROOT / 'include'}", "-I/opt/rocm/include", "-c",
                          str(ROOT / "tests" / "sanitize" / "abi_checks.cpp"), "-o", str(driver)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    exe = out / "abi_checks"
    res = subprocess.run([CLANG, *san, *map(str, objs), str(driver), "-L/opt/rocm/lib", "-lamdhip64",
                          "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-4000:]
    return exe


def test_argument_checks_under_asan_and_ubsan(abi_checks_exe):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               HIP_VISIBLE_DEVICES="")  # the checks must not need a device
    res = subprocess.run([str(abi_checks_exe)], capture_output=True, text=True, env=env, timeout=120)
    report = res.stdout + res.stderr
    assert "runtime error" not in report and "AddressSanitizer" not in report, report[-4000:]
    assert res.returncode == 0, report[-4000:]
    assert "all argument checks held" in res.stdout


def test_driver_covers_every_entry_point():
    """Each ``extern "C"`` entry point of the library appears in the driver."""
    import re

    exported = set()
    for src in CSRC.glob("*.hip"):
        exported |= set(re.findall(r'extern "C" [\w\s\*]+?\b(tj_\w+)\(', src.read_text()))
    driver = (ROOT / "tests" / "sanitize" / "abi_checks.cpp").read_text()
    missing = sorted(name for name in exported if name + "(" not in driver)
    assert len(exported) >= 16 and not missing, missing

