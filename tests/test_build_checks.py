"""Compile-time checks of the decode kernels' launch shapes (host-side syntax passes of hipcc,
no GPU): the static LDS of every one-workgroup-per-CU shape plus its dynamic request must fit
a workgroup's 160 KiB, and a request that would not fit is a build error, not a queue abort at
run time."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SOURCE = ROOT / "lightdelta_amd" / "csrc" / "gdn_decode.hip"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")


def syntax_check(*defines: str) -> subprocess.CompletedProcess:
    cmd = [HIPCC, "--offload-arch=gfx950", "-std=c++17", "--cuda-host-only", "-fsyntax-only",
           f"-I{ROOT / 'include'}", f"-I{SOURCE.parent}", *defines, str(SOURCE)]
    return subprocess.run(cmd, capture_output=True, text=True, timeout=300)


def test_solo_shapes_fit_a_workgroup():
    result = syntax_check()
    assert result.returncode == 0, result.stderr[-2000:]


def test_oversized_solo_request_fails_to_build():
    """150 KiB of dynamic LDS beside any verify kernel's static LDS exceeds 160 KiB."""
    result = syntax_check("-DLD_SOLO_LDS_BYTES=(150*1024)")
    assert result.returncode != 0
    assert "exceed a workgroup's 160 KiB" in result.stderr
