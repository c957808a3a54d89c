"""The measurement programs under mnemocuda_amd/probes/ (figures quoted in the design notes)
still compile for gfx950 against the current kernel sources (CPU only: hipcc cross-compiles)."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PROBES = sorted((ROOT / "mnemocuda_amd" / "probes").glob("*.hip"))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", PROBES, ids=[p.name for p in PROBES])
def test_probe_compiles(src, tmp_path):
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", str(ROOT / "mnemocuda_amd" / "csrc"), str(src), "-o", str(tmp_path / src.stem)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
