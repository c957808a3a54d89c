"""Torch-tensor wrappers over the C ABI (one call = one C entry point).

Tensors must be CUDA (HIP) tensors on the current device; weights are uint8 tensors that
hold raw GGUF blocks.  Calls are enqueued on torch's current stream.  Nothing here
computes on the host: a missing library or a CPU tensor raises MnemoError.
"""
from __future__ import annotations

import torch

from .lib import MnemoError, check, load_library

TYPE_F32, TYPE_Q4K, TYPE_Q6K = 0, 12, 14
BLOCK_BYTES = {TYPE_Q4K: 144, TYPE_Q6K: 210}


def _dev(t: torch.Tensor, name: str, dtype: torch.dtype | None = None) -> int:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise MnemoError(f"{name} must be a GPU tensor")
    if dtype is not None and t.dtype != dtype:
        raise MnemoError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise MnemoError(f"{name} must be contiguous")
    return t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def row_bytes(type_id: int, n_cols: int) -> int:
    if type_id == TYPE_F32:
        return 4 * n_cols
    return (n_cols + 255) // 256 * BLOCK_BYTES[type_id]


def _check_w(w: torch.Tensor, type_id: int, rows: int, cols: int, name: str = "W") -> int:
    p = _dev(w, name)
    need = rows * row_bytes(type_id, cols)
    if w.numel() * w.element_size() < need:
        raise MnemoError(f"{name}: {w.numel() * w.element_size()} bytes < {need} needed for "
                         f"{rows}x{cols} type {type_id}")
    return p


def _check_rc(lib, rc: int, what: str) -> None:
    """Raise for a non-zero return code; also consumes the library's per-thread error slot
    so that a later call does not report this error again."""
    lib.mnemo_last_error()
    if rc:
        raise MnemoError(f"{what}: error {rc}: {lib.mnemo_last_error_string().decode()}")


def init() -> None:
    lib = load_library()
    lib.cuda_kernels_init()
    check(lib, "cuda_kernels_init")


def matvec(w, x, y, rows, cols, type_id):
    """Reference dispatcher matvec() (forward.c:160-173) via mnemo_matvec."""
    lib = load_library()
    _check_w(w, type_id, rows, cols)
    e = lib.mnemo_matvec(w.data_ptr(), _dev(x, "x", torch.float32), _dev(y, "y", torch.float32),
                         rows, cols, type_id, _stream())
    _check_rc(lib, e, "mnemo_matvec")


def matvec_q4k(w, x, y, rows, cols):
    lib = load_library()
    lib.cuda_matvec_q4k(_check_w(w, TYPE_Q4K, rows, cols), _dev(x, "x", torch.float32),
                        _dev(y, "y", torch.float32), rows, cols, _stream())
    check(lib, "cuda_matvec_q4k")


def matvec_q6k(w, x, y, rows, cols):
    lib = load_library()
    lib.cuda_matvec_q6k(_check_w(w, TYPE_Q6K, rows, cols), _dev(x, "x", torch.float32),
                        _dev(y, "y", torch.float32), rows, cols, _stream())
    check(lib, "cuda_matvec_q6k")


def matvec_q4k_add(w, x, residual, y, rows, cols):
    lib = load_library()
    lib.cuda_matvec_q4k_add(_check_w(w, TYPE_Q4K, rows, cols), _dev(x, "x", torch.float32),
                            _dev(residual, "residual", torch.float32), _dev(y, "y", torch.float32),
                            rows, cols, _stream())
    check(lib, "cuda_matvec_q4k_add")


def matvec_q4k_qkv(wq, wk, wv, x, q, k, v, q_rows, kv_rows, cols):
    lib = load_library()
    lib.cuda_matvec_q4k_qkv(_check_w(wq, TYPE_Q4K, q_rows, cols, "wq"),
                            _check_w(wk, TYPE_Q4K, kv_rows, cols, "wk"),
                            _check_w(wv, TYPE_Q4K, kv_rows, cols, "wv"), _dev(x, "x", torch.float32),
                            _dev(q, "q", torch.float32), _dev(k, "k", torch.float32),
                            _dev(v, "v", torch.float32), q_rows, kv_rows, cols, _stream())
    check(lib, "cuda_matvec_q4k_qkv")


def matvec_q4k_dual(wa, wb, x, ya, yb, rows, cols):
    lib = load_library()
    lib.cuda_matvec_q4k_dual(_check_w(wa, TYPE_Q4K, rows, cols, "wa"), _check_w(wb, TYPE_Q4K, rows, cols, "wb"),
                             _dev(x, "x", torch.float32), _dev(ya, "ya", torch.float32),
                             _dev(yb, "yb", torch.float32), rows, cols, _stream())
    check(lib, "cuda_matvec_q4k_dual")


def matvec_dual(wa, ta, wb, tb, x, ya, yb, rows, cols):
    lib = load_library()
    lib.mnemo_matvec_dual(_check_w(wa, ta, rows, cols, "wa"), ta, _check_w(wb, tb, rows, cols, "wb"), tb,
                          _dev(x, "x", torch.float32), _dev(ya, "ya", torch.float32),
                          _dev(yb, "yb", torch.float32), rows, cols, _stream())
    check(lib, "mnemo_matvec_dual")


def matvec_qkv(wq, tq, wk, tk, wv, tv, x, oq, ok, ov, q_rows, kv_rows, cols):
    lib = load_library()
    lib.mnemo_matvec_qkv(_check_w(wq, tq, q_rows, cols, "wq"), tq, _check_w(wk, tk, kv_rows, cols, "wk"), tk,
                         _check_w(wv, tv, kv_rows, cols, "wv"), tv, _dev(x, "x", torch.float32),
                         _dev(oq, "oq", torch.float32), _dev(ok, "ok", torch.float32),
                         _dev(ov, "ov", torch.float32), q_rows, kv_rows, cols, _stream())
    check(lib, "mnemo_matvec_qkv")


def matvec_qkv_rmsnorm(wq, tq, wk, tk, wv, tv, x, norm_w, eps, oq, ok, ov, q_rows, kv_rows, cols):
    """matvec_qkv of rms_norm(x) * norm_w, the norm computed inside the projection launch."""
    lib = load_library()
    if x.numel() < cols or norm_w.numel() < cols:
        raise MnemoError("matvec_qkv_rmsnorm: x or norm_w too small")
    lib.mnemo_matvec_qkv_rmsnorm(_check_w(wq, tq, q_rows, cols, "wq"), tq, _check_w(wk, tk, kv_rows, cols, "wk"), tk,
                                 _check_w(wv, tv, kv_rows, cols, "wv"), tv, _dev(x, "x", torch.float32),
                                 _dev(norm_w, "norm_w", torch.float32), float(eps), _dev(oq, "oq", torch.float32),
                                 _dev(ok, "ok", torch.float32), _dev(ov, "ov", torch.float32), q_rows, kv_rows, cols,
                                 _stream())
    check(lib, "mnemo_matvec_qkv_rmsnorm")


def matvec_q4k_scaled_add(w, x, y, rows, cols, scale):
    lib = load_library()
    lib.cuda_matvec_q4k_scaled_add(_check_w(w, TYPE_Q4K, rows, cols), _dev(x, "x", torch.float32),
                                   _dev(y, "y", torch.float32), rows, cols, float(scale), _stream())
    check(lib, "cuda_matvec_q4k_scaled_add")


def matvec_q6k_scaled_add(w, x, y, rows, cols, scale):
    lib = load_library()
    lib.mnemo_matvec_q6k_scaled_add(_check_w(w, TYPE_Q6K, rows, cols), _dev(x, "x", torch.float32),
                                    _dev(y, "y", torch.float32), rows, cols, float(scale), _stream())
    check(lib, "mnemo_matvec_q6k_scaled_add")


def matvec_swiglu_scaled_add(w, type_id, gate, up, y, rows, cols, scale):
    lib = load_library()
    lib.mnemo_matvec_swiglu_scaled_add(_check_w(w, type_id, rows, cols), type_id,
                                       _dev(gate, "gate", torch.float32), _dev(up, "up", torch.float32),
                                       _dev(y, "y", torch.float32), rows, cols, float(scale), _stream())
    check(lib, "mnemo_matvec_swiglu_scaled_add")


def matvec_f32(w, x, y, rows, cols):
    lib = load_library()
    lib.cuda_matvec_f32(_dev(w, "W", torch.float32), _dev(x, "x", torch.float32), _dev(y, "y", torch.float32),
                        rows, cols, _stream())
    check(lib, "cuda_matvec_f32")


def topk_softmax(scores, idx, w, n_experts, k):
    lib = load_library()
    lib.cuda_topk_softmax(_dev(scores, "scores", torch.float32), _dev(idx, "idx", torch.int32),
                          _dev(w, "w", torch.float32), n_experts, k, _stream())
    check(lib, "cuda_topk_softmax")


def swiglu(g, u, out, n):
    lib = load_library()
    lib.cuda_swiglu(_dev(g, "g", torch.float32), _dev(u, "u", torch.float32), _dev(out, "out", torch.float32),
                    n, _stream())
    check(lib, "cuda_swiglu")


def scaled_add(out, x, scale, n):
    lib = load_library()
    lib.cuda_scaled_add(_dev(out, "out", torch.float32), _dev(x, "x", torch.float32), float(scale), n, _stream())
    check(lib, "cuda_scaled_add")


def quantize_q8_1(src, dst, K, N):
    lib = load_library()
    if dst.numel() * dst.element_size() < N * (K // 128) * 144:
        raise MnemoError("quantize_q8_1: dst too small")
    lib.cuda_quantize_mmq_q8_1(_dev(src, "src", torch.float32), _dev(dst, "dst"), K, N, _stream())
    check(lib, "cuda_quantize_mmq_q8_1")


def gemm(w, type_id, act, out, M, K, N):
    lib = load_library()
    _check_w(w, type_id, M, K)
    if act.numel() * act.element_size() < N * (K // 128) * 144:
        raise MnemoError("gemm: activation buffer too small")
    if out.numel() < M * N:
        raise MnemoError("gemm: output too small")
    fn = lib.cuda_gemm_q4k if type_id == TYPE_Q4K else lib.mnemo_gemm_q6k
    fn(w.data_ptr(), _dev(act, "act"), _dev(out, "out", torch.float32), M, K, N, _stream())
    check(lib, "gemm")


def expert_fwd(expert, gate_sz, up_sz, H, EFF, down_type, weight, x, gate_buf, up_buf, moe_out):
    lib = load_library()
    e = lib.mnemo_expert_fwd(_dev(expert, "expert"), gate_sz, up_sz, H, EFF, down_type, float(weight),
                             _dev(x, "x", torch.float32), _dev(gate_buf, "gate_buf", torch.float32),
                             _dev(up_buf, "up_buf", torch.float32), _dev(moe_out, "moe_out", torch.float32),
                             _stream())
    _check_rc(lib, e, "mnemo_expert_fwd")


def moe_prefill_workspace_bytes(T, hidden, eff, n_experts, k) -> int:
    return int(load_library().mnemo_moe_prefill_workspace_bytes(T, hidden, eff, n_experts, k))


def moe_prefill(experts, expert_stride, gate_off, up_off, down_off, down_type, x, topk_idx, topk_w,
                T, hidden, eff, n_experts, k, workspace, out):
    """Grouped-expert prefill: out[t] += sum_slot w * down(silu(gate x_t) * up x_t)."""
    lib = load_library()
    need = expert_stride * (n_experts - 1) + down_off + row_bytes(down_type, eff) * hidden \
        if down_type in BLOCK_BYTES else 0  # an unknown type is reported by the library
    if experts.numel() * experts.element_size() < need:
        raise MnemoError("moe_prefill: expert table too small")
    if topk_idx.numel() < T * k or topk_w.numel() < T * k or x.numel() < T * hidden or out.numel() < T * hidden:
        raise MnemoError("moe_prefill: routing, x or out too small")
    e = lib.mnemo_moe_prefill(_dev(experts, "experts"), expert_stride, gate_off, up_off, down_off, down_type,
                              _dev(x, "x", torch.float32), _dev(topk_idx, "topk_idx", torch.int32),
                              _dev(topk_w, "topk_w", torch.float32), T, hidden, eff, n_experts, k,
                              _dev(workspace, "workspace"), workspace.numel() * workspace.element_size(),
                              _dev(out, "out", torch.float32), _stream())
    _check_rc(lib, e, "mnemo_moe_prefill")


def moe_decode_workspace_bytes(hidden, eff, n_experts, k) -> int:
    return int(load_library().mnemo_moe_decode_workspace_bytes(hidden, eff, n_experts, k))


def moe_decode(router_w, experts, expert_stride, gate_off, up_off, down_off, down_type, x, hidden, eff,
               n_experts, k, workspace, out, topk_idx=None, topk_w=None):
    """One token's MoE block with device-side dispatch: out += sum_slot w * expert(x)."""
    lib = load_library()
    need = expert_stride * (n_experts - 1) + down_off + row_bytes(down_type, eff) * hidden \
        if down_type in BLOCK_BYTES else 0
    if experts.numel() * experts.element_size() < need:
        raise MnemoError("moe_decode: expert table too small")
    if router_w.numel() < n_experts * hidden or x.numel() < hidden or out.numel() < hidden:
        raise MnemoError("moe_decode: router, x or out too small")
    e = lib.mnemo_moe_decode(_dev(router_w, "router_w", torch.float32), _dev(experts, "experts"), expert_stride,
                             gate_off, up_off, down_off, down_type, _dev(x, "x", torch.float32), hidden, eff,
                             n_experts, k, _dev(workspace, "workspace"),
                             workspace.numel() * workspace.element_size(), _dev(out, "out", torch.float32),
                             None if topk_idx is None else _dev(topk_idx, "topk_idx", torch.int32),
                             None if topk_w is None else _dev(topk_w, "topk_w", torch.float32), _stream())
    _check_rc(lib, e, "mnemo_moe_decode")


def moe_decode_rmsnorm(router_w, experts, expert_stride, gate_off, up_off, down_off, down_type, x, norm_w, eps,
                       hidden, eff, n_experts, k, workspace, out, topk_idx=None, topk_w=None):
    """moe_decode of rms_norm(x) * norm_w with the norm computed by the router and gate/up
    launches; x is the raw hidden state and may be out itself."""
    lib = load_library()
    need = expert_stride * (n_experts - 1) + down_off + row_bytes(down_type, eff) * hidden \
        if down_type in BLOCK_BYTES else 0
    if experts.numel() * experts.element_size() < need:
        raise MnemoError("moe_decode_rmsnorm: expert table too small")
    if router_w.numel() < n_experts * hidden or x.numel() < hidden or out.numel() < hidden \
            or norm_w.numel() < hidden:
        raise MnemoError("moe_decode_rmsnorm: router, x, norm_w or out too small")
    e = lib.mnemo_moe_decode_rmsnorm(
        _dev(router_w, "router_w", torch.float32), _dev(experts, "experts"), expert_stride, gate_off, up_off,
        down_off, down_type, _dev(x, "x", torch.float32), _dev(norm_w, "norm_w", torch.float32), float(eps), hidden,
        eff, n_experts, k, _dev(workspace, "workspace"), workspace.numel() * workspace.element_size(),
        _dev(out, "out", torch.float32), None if topk_idx is None else _dev(topk_idx, "topk_idx", torch.int32),
        None if topk_w is None else _dev(topk_w, "topk_w", torch.float32), _stream())
    _check_rc(lib, e, "mnemo_moe_decode_rmsnorm")


def sample_token(logits, vocab, temperature, top_p, seed, out):
    """Next token from logits[vocab] (greedy for temperature <= 0, else top-p) into out[0]."""
    lib = load_library()
    if logits.numel() < vocab or out.numel() < 1:
        raise MnemoError("sample_token: logits or out too small")
    lib.cuda_sample_token(_dev(logits, "logits", torch.float32), vocab, float(temperature), float(top_p),
                          int(seed) & 0xFFFFFFFFFFFFFFFF, _dev(out, "out", torch.int32), _stream())
    check(lib, "cuda_sample_token")


def sample_workspace_bytes() -> int:
    return int(load_library().mnemo_sample_workspace_bytes())


def sample_token_ws(logits, vocab, temperature, top_p, seed, workspace, out):
    """sample_token with the vocabulary scan over 64 workgroups (workspace of
    sample_workspace_bytes() bytes)."""
    lib = load_library()
    if logits.numel() < vocab or out.numel() < 1:
        raise MnemoError("sample_token_ws: logits or out too small")
    rc = lib.mnemo_sample_token_ws(_dev(logits, "logits", torch.float32), vocab, float(temperature), float(top_p),
                                   int(seed) & 0xFFFFFFFFFFFFFFFF, _dev(workspace, "workspace"),
                                   workspace.numel() * workspace.element_size(), _dev(out, "out", torch.int32),
                                   _stream())
    _check_rc(lib, rc, "mnemo_sample_token_ws")


# ---------------------------------------------------------------- attention chain
F32 = torch.float32


def _opt(t, name, dtype=None) -> int | None:
    return None if t is None else _dev(t, name, dtype)


def rms_norm(x, w, out, eps: float, residual=None):
    """out = x * rsqrt(mean(x^2) + eps) * w (cuda_rms_norm); with residual, also residual = x
    (cuda_rms_norm_residual)."""
    lib = load_library()
    n = x.numel()
    if w.numel() < n or out.numel() < n or (residual is not None and residual.numel() < n):
        raise MnemoError("rms_norm: buffers too small")
    if residual is None:
        lib.cuda_rms_norm(_dev(x, "x", F32), _dev(w, "w", F32), _dev(out, "out", F32), n, float(eps), _stream())
        check(lib, "cuda_rms_norm")
    else:
        lib.cuda_rms_norm_residual(_dev(x, "x", F32), _dev(w, "w", F32), _dev(out, "out", F32),
                                   _dev(residual, "residual", F32), n, float(eps), _stream())
        check(lib, "cuda_rms_norm_residual")


def rms_norm_batched(x, w, out, head_dim: int, eps: float):
    lib = load_library()
    lib.cuda_rms_norm_batched(_dev(x, "x", F32), _dev(w, "w", F32), _dev(out, "out", F32), head_dim,
                              x.numel() // head_dim, float(eps), _stream())
    check(lib, "cuda_rms_norm_batched")


def rms_norm_qk(q, k, qw, kw, head_dim: int, eps: float):
    lib = load_library()
    lib.cuda_rms_norm_qk(_dev(q, "q", F32), _dev(k, "k", F32), _dev(qw, "qw", F32), _dev(kw, "kw", F32), head_dim,
                         q.numel() // head_dim, k.numel() // head_dim, float(eps), _stream())
    check(lib, "cuda_rms_norm_qk")


def residual_add(a, b, out):
    lib = load_library()
    lib.cuda_residual_add(_dev(a, "a", F32), _dev(b, "b", F32), _dev(out, "out", F32), a.numel(), _stream())
    check(lib, "cuda_residual_add")


def rope(q, k, head_dim: int, pos: int, theta: float):
    lib = load_library()
    lib.cuda_rope(_dev(q, "q", F32), _dev(k, "k", F32), head_dim, int(pos), float(theta), q.numel() // head_dim,
                  k.numel() // head_dim, _stream())
    check(lib, "cuda_rope")


def f32_to_f16_dual(a, b, oa, ob):
    lib = load_library()
    lib.cuda_f32_to_f16_dual(_dev(a, "a", F32), _dev(b, "b", F32), _dev(oa, "oa", torch.float16),
                             _dev(ob, "ob", torch.float16), a.numel(), _stream())
    check(lib, "cuda_f32_to_f16_dual")


def f32_to_int8_kv_dual(k, v, ok, ov, ks, vs, head_dim: int):
    lib = load_library()
    lib.cuda_f32_to_int8_kv_dual(_dev(k, "k", F32), _dev(v, "v", F32), _dev(ok, "ok", torch.int8),
                                 _dev(ov, "ov", torch.int8), _dev(ks, "ks", F32), _dev(vs, "vs", F32), head_dim,
                                 k.numel() // head_dim, _stream())
    check(lib, "cuda_f32_to_int8_kv_dual")


def attention(q, kc, vc, out, n_heads: int, head_dim: int, n_kv_heads: int, seq_len: int, scale: float,
              ks=None, vs=None):
    """cuda_attention_f16kv (kc/vc float16) or cuda_attention_int8kv (int8 with scales)."""
    lib = load_library()
    gqa = n_heads // n_kv_heads
    if kc.dtype == torch.float16:
        lib.cuda_attention_f16kv(_dev(q, "q", F32), _dev(kc, "kc"), _dev(vc, "vc"), _dev(out, "out", F32), n_heads,
                                 head_dim, n_kv_heads, int(seq_len), gqa, float(scale), _stream())
        check(lib, "cuda_attention_f16kv")
    else:
        lib.cuda_attention_int8kv(_dev(q, "q", F32), _dev(kc, "kc", torch.int8), _dev(vc, "vc", torch.int8),
                                  _dev(ks, "ks", F32), _dev(vs, "vs", F32), _dev(out, "out", F32), n_heads, head_dim,
                                  n_kv_heads, int(seq_len), gqa, float(scale), _stream())
        check(lib, "cuda_attention_int8kv")


def attention_reserve(n_slots: int) -> None:
    """mnemo_attention_reserve: at least n_slots free workspace slots for captured
    cuda_attention_* calls on the current GPU (allocates; not under capture)."""
    lib = load_library()
    _check_rc(lib, lib.mnemo_attention_reserve(int(n_slots)), "mnemo_attention_reserve")


def attn_prep(q, k, v, qw, kw, head_dim: int, eps: float, theta: float, pos_dev, kc, vc, ks=None, vs=None,
              v_layout: int = 0):
    """QK norm (when qw/kw are given) + RoPE + KV store at cache row pos_dev[0], one launch
    (v_layout 1: V in the blocked layout of attention_decode)."""
    lib = load_library()
    kv_type = 0 if kc.dtype == torch.float16 else 1
    rc = lib.mnemo_attn_prep(_dev(q, "q", F32), _dev(k, "k", F32), _dev(v, "v", F32), _opt(qw, "qw", F32),
                             _opt(kw, "kw", F32), head_dim, q.numel() // head_dim, k.numel() // head_dim, float(eps),
                             float(theta), _dev(pos_dev, "pos_dev", torch.int32), _dev(kc, "kc"), _dev(vc, "vc"),
                             _opt(ks, "ks", F32), _opt(vs, "vs", F32), kv_type, int(v_layout), _stream())
    _check_rc(lib, rc, "mnemo_attn_prep")


def attention_dev(q, kc, vc, out, n_heads: int, head_dim: int, n_kv_heads: int, pos_dev, scale: float,
                  ks=None, vs=None):
    """attention over positions 0..pos_dev[0] (length read on the device)."""
    lib = load_library()
    kv_type = 0 if kc.dtype == torch.float16 else 1
    rc = lib.mnemo_attention(_dev(q, "q", F32), _dev(kc, "kc"), _dev(vc, "vc"), _opt(ks, "ks", F32),
                             _opt(vs, "vs", F32), kv_type, _dev(out, "out", F32), n_heads, head_dim, n_kv_heads,
                             _dev(pos_dev, "pos_dev", torch.int32), float(scale), _stream())
    _check_rc(lib, rc, "mnemo_attention")


def attention_decode_workspace_bytes(n_kv_heads: int, max_ctx: int) -> int:
    return int(load_library().mnemo_attention_decode_workspace_bytes(n_kv_heads, max_ctx))


def v_cache_bytes(n_kv_heads: int, head_dim: int, max_ctx: int, kv_type: int, v_layout: int) -> int:
    return int(load_library().mnemo_v_cache_bytes(n_kv_heads, head_dim, max_ctx, kv_type, v_layout))


def attention_decode(q, kc, vc, out, n_heads: int, head_dim: int, n_kv_heads: int, max_ctx: int, pos_dev,
                     scale: float, ws, ks=None, vs=None, v_layout: int = 0):
    """GQA-batched split-position attention over positions 0..pos_dev[0] (matrix cores)."""
    lib = load_library()
    kv_type = 0 if kc.dtype == torch.float16 else 1
    rc = lib.mnemo_attention_decode(_dev(q, "q", F32), _dev(kc, "kc"), _dev(vc, "vc"), _opt(ks, "ks", F32),
                                    _opt(vs, "vs", F32), kv_type, int(v_layout), _dev(out, "out", F32), n_heads,
                                    head_dim,
                                    n_kv_heads, int(max_ctx), _dev(pos_dev, "pos_dev", torch.int32), float(scale),
                                    _dev(ws, "ws"), ws.numel() * ws.element_size(), _stream())
    _check_rc(lib, rc, "mnemo_attention_decode")


def attention_decode_prep(q, k, v, qw, kw, eps: float, theta: float, kc, vc, out, n_heads: int, head_dim: int,
                          n_kv_heads: int, max_ctx: int, pos_dev, scale: float, ws, ks=None, vs=None,
                          v_layout: int = 0):
    """attn_prep + attention_decode in the same two launches: q, k, v raw (left unchanged),
    the new K / V rows stored at pos_dev[0], attention over 0..pos_dev[0]."""
    lib = load_library()
    kv_type = 0 if kc.dtype == torch.float16 else 1
    if q.numel() < n_heads * head_dim or k.numel() < n_kv_heads * head_dim or v.numel() < n_kv_heads * head_dim:
        raise MnemoError("attention_decode_prep: q, k or v too small")
    rc = lib.mnemo_attention_decode_prep(
        _dev(q, "q", F32), _dev(k, "k", F32), _dev(v, "v", F32), _opt(qw, "qw", F32), _opt(kw, "kw", F32),
        float(eps), float(theta), _dev(kc, "kc"), _dev(vc, "vc"), _opt(ks, "ks", F32), _opt(vs, "vs", F32), kv_type,
        int(v_layout), _dev(out, "out", F32), n_heads, head_dim, n_kv_heads, int(max_ctx),
        _dev(pos_dev, "pos_dev", torch.int32), float(scale), _dev(ws, "ws"), ws.numel() * ws.element_size(),
        _stream())
    _check_rc(lib, rc, "mnemo_attention_decode_prep")


# ---------------------------------------------------------------- embedding
def embedding_lookup(table, type_id: int, token_dev, n_vocab: int, out, hidden: int):
    """out[:hidden] = dequantised row token_dev[0] of table (F32 / Q4_K / Q6_K).  table is a
    GPU tensor or a raw device pointer (int)."""
    lib = load_library()
    tp = table if isinstance(table, int) else _dev(table, "table")
    rc = lib.mnemo_embedding_lookup(tp, int(type_id), _dev(token_dev, "token_dev", torch.int32), int(n_vocab),
                                    _dev(out, "out", F32), int(hidden), _stream())
    _check_rc(lib, rc, "mnemo_embedding_lookup")


def embedding_lookup_q4k(table, out, token_id: int, hidden: int, row_bytes: int):
    """cuda_embedding_lookup_q4k (reference signature)."""
    lib = load_library()
    tp = table if isinstance(table, int) else _dev(table, "table")
    lib.cuda_embedding_lookup_q4k(tp, _dev(out, "out", F32), int(token_id), int(hidden), int(row_bytes), _stream())
    check(lib, "cuda_embedding_lookup_q4k")
