"""The MoE decode entry point that allocates nothing (mnemo_moe_decode_rmsnorm_noalloc,
called through the C-ABI) against the workspace entry point it mirrors
(mnemo_moe_decode_rmsnorm): the same kernels on the library's own device array, so the
routing and the added delta must agree bit for bit -- on two calls in a row, the second with
smaller sizes (the array keeps the first call's contents) -- and sizes beyond the array are
rejected before any launch."""
import ctypes as C

import numpy as np
import pytest
import torch

from mnemocuda_amd import synth
from tests.gpu_util import case, dev, host

pytestmark = pytest.mark.gpu


def _ptr(t):
    return C.c_void_p(t.data_ptr())


def _inputs(rng, H, EFF, E, k, DT):
    table = synth.expert_table(rng, E, H, EFF, DT)
    router = (rng.standard_normal((E, H)) / np.sqrt(H)).astype(np.float32)
    x = (3.0 * rng.standard_normal(H)).astype(np.float32)
    nw = (1.0 + 0.25 * rng.standard_normal(H)).astype(np.float32)
    out0 = rng.standard_normal(H).astype(np.float32)
    return dev(table), dev(router), dev(x), dev(nw), out0


@pytest.mark.parametrize("order", ["large_then_small"])
def test_noalloc_matches_workspace_entry_point(gpu, order):
    lib = gpu.load_library()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    for H, EFF, E, k, DT in [(4096, 1536, 128, 8, 14), (1024, 512, 16, 4, 12)]:
        rng = np.random.default_rng(H + E)
        table, router, x, nw, out0 = _inputs(rng, H, EFF, E, k, DT)
        lay = synth.expert_layout(H, EFF, DT)
        eps = 1e-6
        # the workspace entry point
        ws = torch.zeros(gpu.ops.moe_decode_workspace_bytes(H, EFF, E, k), dtype=torch.uint8, device="cuda")
        out_ws, idx_ws, w_ws = dev(out0), torch.full((k,), -1, dtype=torch.int32, device="cuda"), \
            torch.zeros(k, device="cuda")
        case(f"moe_decode_rmsnorm (workspace) H={H} EFF={EFF} E={E} k={k} down={DT}")
        gpu.ops.moe_decode_rmsnorm(router, table, *lay, DT, x, nw, eps, H, EFF, E, k, ws, out_ws, idx_ws, w_ws)
        # the entry point without allocation, through the C-ABI
        out_na, idx_na, w_na = dev(out0), torch.full((k,), -1, dtype=torch.int32, device="cuda"), \
            torch.zeros(k, device="cuda")
        case(f"moe_decode_rmsnorm_noalloc H={H} EFF={EFF} E={E} k={k} down={DT}")
        rc = lib.mnemo_moe_decode_rmsnorm_noalloc(_ptr(router), _ptr(table), *lay, DT, _ptr(x), _ptr(nw),
                                                  C.c_float(eps), H, EFF, E, k, _ptr(out_na), _ptr(idx_na),
                                                  _ptr(w_na), stream)
        assert rc == 0, lib.mnemo_last_error_string()
        lib.mnemo_last_error()
        assert torch.equal(idx_na, idx_ws)
        assert torch.equal(w_na, w_ws)
        assert torch.equal(out_na, out_ws), float((out_na - out_ws).abs().max())
        assert not torch.equal(out_na, dev(out0))  # it added something


def test_noalloc_rejects_oversize(gpu):
    lib = gpu.load_library()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    H, EFF, E, k = 16384, 8192, 128, 16  # needs ~3.2 MB of workspace
    assert gpu.ops.moe_decode_workspace_bytes(H, EFF, E, k) > 1703936
    out = torch.zeros(H, device="cuda")
    before = out.clone()
    rc = lib.mnemo_moe_decode_rmsnorm_noalloc(None, None, 0, 0, 0, 0, 14, None, _ptr(out), C.c_float(1e-6), H, EFF,
                                              E, k, _ptr(out), None, None, stream)
    assert rc != 0
    assert b"scratch" in lib.mnemo_last_error_string()
    lib.mnemo_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, before)
