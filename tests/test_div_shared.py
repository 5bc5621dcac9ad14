"""The per-element division of the head norms (`data * weight / rms`, fused_per_head_norm_rope.wgsl:40;
div_shared in gemma4-webgpu_amd/csrc/ref_math.h): one correctly rounded reciprocal per head row, then
Markstein's correction per element. tests/div_check.c compares it bit for bit with the IEEE quotient
over random operand pairs across every exponent, every divisor significand in [1, 2), signed zeros and
the fast path's threshold. The GPU tests then compare every norm's output with the oracle's IEEE
division."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
GCC = shutil.which("gcc")


@pytest.mark.skipif(GCC is None, reason="gcc is not installed")
def test_shared_divisor_division_is_the_ieee_quotient(tmp_path):
    exe = tmp_path / "div_check"
    subprocess.run([GCC, "-O2", "-ffp-contract=off", str(ROOT / "tests" / "div_check.c"), "-o", str(exe), "-lm"],
                   check=True)
    r = subprocess.run([str(exe), "20000000"], capture_output=True, text=True, timeout=300)
    print(r.stdout.strip())
    assert r.returncode == 0, r.stdout
    assert "mismatches 0" in r.stdout
