"""The C ABI from C: tests/c_abi/nl_abi_check.c includes only
include/nlearn_hip.h and the HIP runtime API (no torch, no Python in the
process). On the CPU it must compile as strict C11; on a GPU it is linked
against the in-tree libnlearn_hip.so and run (exact GEMMs in four layouts, the
flash forward's first-row closed form and double-precision references for
flash and CE)."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "c_abi" / "nl_abi_check.c"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
CFLAGS = ["-std=c11", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
          f"-I{ROOT / 'include'}"]


def _cc():
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None or not (ROCM / "include" / "hip" / "hip_runtime_api.h").exists():
        pytest.skip("needs a C compiler and the HIP runtime headers")
    return cc


def test_header_is_strict_c11():
    cc = _cc()
    subprocess.run([cc, *CFLAGS, "-fsyntax-only", str(SRC)], check=True, timeout=120)


@pytest.mark.gpu
def test_c_program_through_the_abi(tmp_path):
    cc = _cc()
    lib_dir = ROOT / "nlearn_amd"
    assert (lib_dir / "libnlearn_hip.so").exists(), "build the library first"
    exe = tmp_path / "nl_abi_check"
    subprocess.run([cc, *CFLAGS, str(SRC), f"-L{lib_dir}", "-lnlearn_hip", f"-L{ROCM / 'lib'}", "-lamdhip64", "-lm",
                    f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{ROCM / 'lib'}", "-o", str(exe)], check=True, timeout=120)
    print("running", exe, flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("C ABI check: all passed")
