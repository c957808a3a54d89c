"""GPU checks of the model directory upload and the embedding lookup: every resident tensor
and expert layer lands byte-exact at its device address; the embedding rows decode exactly
as the oracle's dequantisation (F32, Q4_K, Q6_K; host and device token ids); a GEMV reads
the uploaded weights in place (MnemoCUDA src/engine.c:860-890, forward.c:1145-1280)."""
import ctypes as C

import numpy as np
import pytest
import torch

from mnemocuda_amd import model as mm
from tests.conftest import rel_l2
from tests.gpu_util import case, dev, host
from tests.model_fixture import F32, Q4K, Q6K, write_model

pytestmark = pytest.mark.gpu

_hip = None


def d2h(ptr: int, n: int) -> bytes:
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
    torch.cuda.synchronize()
    buf = C.create_string_buffer(n)
    assert _hip.hipMemcpy(buf, C.c_void_p(ptr), C.c_size_t(n), 2) == 0  # device to host
    return buf.raw


@pytest.mark.parametrize("embd_type", [Q4K, Q6K, F32])
def test_upload_and_embedding(gpu, oracle, tmp_path, embd_type):
    meta = write_model(tmp_path / "m", embd_type=embd_type, vocab=300, hidden=512)
    case(f"model upload embd_type={embd_type}")
    m = mm.Model(tmp_path / "m")
    m.upload(with_experts=True)
    for name, (t, rows, cols, raw) in meta["tensors"].items():
        info, ptr = m.tensor(name)
        assert ptr % 256 == 0 and info.size == len(raw)
        assert d2h(ptr, len(raw)) == raw, name
    for layer, raw in meta["experts"].items():
        assert d2h(m.experts(layer), len(raw)) == raw
    # embedding rows
    t, vocab, hidden, raw = meta["tensors"]["token_embd.weight"]
    _, ptr = m.tensor("token_embd.weight")
    table = oracle.dequant(t, np.frombuffer(raw, np.uint8), vocab, hidden) if t != F32 else \
        np.frombuffer(raw, np.float32).reshape(vocab, hidden)
    out = torch.full((hidden,), np.nan, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    for token in (0, 1, 137, vocab - 1):
        tok.fill_(token)
        gpu.ops.embedding_lookup(ptr, t, tok, vocab, out, hidden)
        assert np.array_equal(host(out), table[token]), token
    tok.fill_(vocab + 5)  # outside the table: the nearest row
    gpu.ops.embedding_lookup(ptr, t, tok, vocab, out, hidden)
    assert np.array_equal(host(out), table[vocab - 1])
    if t == Q4K:
        out2 = torch.empty(hidden, device="cuda")
        gpu.ops.embedding_lookup_q4k(ptr, out2, 137, hidden, hidden // 256 * 144)
        assert np.array_equal(host(out2), table[137])
    # a GEMV straight on the uploaded weights
    _, wq = m.tensor("blk.1.attn_q.weight")
    tq, rq, cq, rawq = meta["tensors"]["blk.1.attn_q.weight"]
    x = np.random.default_rng(3).standard_normal(cq).astype(np.float32)
    y = torch.empty(rq, device="cuda")
    xd = dev(x)
    gpu.load_library().cuda_matvec_q4k(C.c_void_p(wq), C.c_void_p(xd.data_ptr()), C.c_void_p(y.data_ptr()), rq, cq,
                                       None)
    assert rel_l2(host(y), oracle.gemv(Q4K, np.frombuffer(rawq, np.uint8), x, rq, cq)) < 1e-3
    m.close()


def test_embedding_hidden_not_multiple_of_256(gpu, oracle, rng):
    """a 300-value row (two Q4_K blocks, the second partly used)."""
    from mnemocuda_amd import synth
    vocab, hidden = 5, 300
    raw = synth.weights(rng, Q4K, vocab, hidden)
    table = oracle.dequant(Q4K, raw, vocab, hidden)
    case("embedding ragged hidden")
    out = torch.full((hidden + 4,), 7.0, device="cuda")
    tok = torch.tensor([3], dtype=torch.int32, device="cuda")
    gpu.ops.embedding_lookup(dev(raw), Q4K, tok, vocab, out, hidden)
    got = host(out)
    assert np.array_equal(got[:hidden], table[3]) and np.all(got[hidden:] == 7.0)
