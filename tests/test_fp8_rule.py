"""Exhaustive host check of the device FP8 scale rule and E4M3FN encoder
(ds4cuda_amd/csrc/ds4hip_common.h) against the correctly rounded log2 and the
oracle's nearest-code picker (tests/native/fp8_rule_check.cpp)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not on PATH")
def test_scale_rule_and_encoder_exhaustive(tmp_path):
    ora = ROOT / "oracle"
    assert (ora / "libds4oracle.so").exists()
    exe = tmp_path / "fp8_rule_check"
    subprocess.run(["hipcc", "-std=c++17", "-O2", "-pthread",
                    f"-I{ROOT / 'ds4cuda_amd' / 'csrc'}", f"-I{ora}",
                    str(ROOT / "tests" / "native" / "fp8_rule_check.cpp"), "-o", str(exe),
                    f"-L{ora}", "-lds4oracle", f"-Wl,-rpath,{ora}"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0, encoder mismatches 0" in out.stdout
