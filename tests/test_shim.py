"""The C++ launcher shims (include/ds4hip_launchers.h) compile against the
reference's call shapes, link to libds4hip.so and report errors through
ds4hip_get_last_error() — host-decided paths only, no GPU needed."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not on PATH")
def test_launcher_shims_compile_and_report(tmp_path):
    pkg = ROOT / "ds4cuda_amd"
    assert (pkg / "libds4hip.so").exists()
    exe = tmp_path / "shim_check"
    subprocess.run(["hipcc", "-std=c++17", "-O1", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "native" / "shim_check.cpp"), "-o", str(exe),
                    f"-L{pkg}", "-lds4hip", f"-Wl,-rpath,{pkg}"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, (out.returncode, out.stderr)
    assert "shim ok" in out.stdout
