"""CPU-side checks of the C ABI: the library loads, exports exactly what the headers
declare, and its host logic and argument checks work without a GPU (no call below
reaches a HIP API)."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from mnemocuda_amd import lib as mlib

ROOT = Path(__file__).resolve().parents[1]
HEADERS = [ROOT / "include" / "mnemo_kernels.h", ROOT / "include" / "mnemo_host.h", ROOT / "include" / "mnemo_model.h"]


def header_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[a-zA-Z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, re.M):
            if m.group(1) not in ("defined",):
                names.add(m.group(1))
    return names


@pytest.fixture(scope="module")
def L():
    if not mlib.LIB_PATH.exists():
        pytest.fail("libmnemo_hip.so not built (run __graft_entry__.build())")
    return mlib.load_library()


def test_headers_match_binding_table():
    assert header_functions() == set(mlib.EXPORTS)


def test_library_exports_every_declared_symbol(L):
    out = subprocess.run(["nm", "-D", "--defined-only", str(mlib.LIB_PATH)], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = set(mlib.EXPORTS) - exported
    assert not missing, missing


def test_version_string(L):
    assert b"gfx950" in L.mnemo_version()


def test_down_type_heuristic(L):
    """forward.c:866-872: down is Q6_K iff bytes > 1.2 x the Q4_K size of [H][EFF]."""
    H, EFF = 4096, 1536
    q4 = (H * EFF + 255) // 256 * 144
    q6 = (H * EFF + 255) // 256 * 210
    assert L.mnemo_down_type_id(q6, H, EFF) == 14
    assert L.mnemo_down_type_id(q4, H, EFF) == 12
    assert L.mnemo_down_type_id(int(q4 * 1.2), H, EFF) == 12
    assert L.mnemo_down_type_id(int(q4 * 1.2) + 1, H, EFF) == 14


def test_dispatcher_rejects_unsupported_type(L, capfd):
    # type 13 (Q5_K) takes the reference's warning-and-no-op branch (forward.c:169-171)
    assert L.mnemo_matvec(None, None, None, 4, 256, 13, None) == 3
    assert "unsupported type_id 13" in capfd.readouterr().err


@pytest.mark.parametrize("call", [
    lambda L: L.cuda_matvec_q4k(None, None, None, 8, 256, None),
    lambda L: L.cuda_matvec_q6k(1, 1, 1, 8, 0, None),
    lambda L: L.cuda_matvec_q4k(1, 1, 1, 8, 1 << 20, None),
    lambda L: L.mnemo_matvec_dual(1, 12, 1, 13, 1, 1, 1, 8, 256, None),
    lambda L: L.cuda_topk_softmax(1, 1, 1, 128, 17, None),
    lambda L: L.cuda_quantize_mmq_q8_1(16, 16, 100, 4, None),
    lambda L: L.cuda_gemm_q4k(16, 16, 16, 64, 300, 4, None),
    lambda L: L.cuda_matvec_f32(None, 1, 1, 4, 4, None),
])
def test_bad_arguments_are_reported_without_launching(L, call, capfd):
    assert L.mnemo_last_error() == 0
    call(L)
    code = L.mnemo_last_error()
    assert code in (1, 3)
    assert "[mnemo]" in capfd.readouterr().err
    assert L.mnemo_last_error() == 0  # reading clears


def test_expert_fwd_rejects_bad_down_type(L):
    assert L.mnemo_expert_fwd(16, 1, 1, 4096, 1536, 13, 1.0, 16, 16, 16, 16, None) == 3
    assert L.mnemo_expert_fwd(None, 1, 1, 4096, 1536, 12, 1.0, 16, 16, 16, 16, None) == 1
