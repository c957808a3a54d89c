"""CPU oracle for the quantized-matmul hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this
package; the product library never loads it.  ``load()`` returns the C restatement
(mnemo_oracle.c) with typed numpy-friendly wrappers; ``oracle_np`` is the independent
numpy restatement the C code is cross-checked against.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libmnemo_oracle.so"


def build() -> Path:
    r = subprocess.run(["make", "-C", str(HERE)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")
    return LIB


class Oracle:
    def __init__(self, path: Path = LIB):
        if not path.exists():
            build()
        L = C.CDLL(str(path))
        P = C.c_void_p
        L.mo_f16_to_f32.restype = C.c_float
        L.mo_f16_to_f32.argtypes = [C.c_uint16]
        L.mo_f32_to_f16.restype = C.c_uint16
        L.mo_f32_to_f16.argtypes = [C.c_float]
        L.mo_get_scale_min_k4.argtypes = [C.c_int, P, P, P]
        for n in ("mo_dequant_q4k", "mo_dequant_q6k"):
            getattr(L, n).argtypes = [P, P, C.c_int, C.c_int]
        L.mo_dequant.restype = C.c_int
        L.mo_dequant.argtypes = [C.c_int, P, P, C.c_int, C.c_int]
        L.mo_gemv.restype = C.c_int
        L.mo_gemv.argtypes = [C.c_int, P, P, P, C.c_int, C.c_int]
        L.mo_gemv_f32acc.restype = C.c_int
        L.mo_gemv_f32acc.argtypes = [C.c_int, P, P, P, C.c_int, C.c_int, C.c_int]
        L.mo_matvec_f32.argtypes = [P, P, P, C.c_int, C.c_int]
        L.mo_topk_softmax.argtypes = [P, C.c_int, C.c_int, P, P]
        L.mo_swiglu.argtypes = [P, P, P, C.c_int]
        L.mo_scaled_add.argtypes = [P, P, C.c_float, C.c_int]
        L.mo_quantize_q8_1_mmq.argtypes = [P, P, C.c_int, C.c_int]
        L.mo_dequant_q8_1_mmq.argtypes = [P, P, C.c_int, C.c_int]
        L.mo_gemm_q8_1.restype = C.c_int
        L.mo_gemm_q8_1.argtypes = [C.c_int, P, P, P, C.c_int, C.c_int, C.c_int]
        L.mo_sample_token.restype = C.c_int
        L.mo_sample_token.argtypes = [P, C.c_int, C.c_float, C.c_float, C.c_ulonglong, P, P]
        L.mo_xoroshiro_next.restype = C.c_uint64
        L.mo_xoroshiro_next.argtypes = [P, P]
        F = C.c_float
        L.mo_rms_norm.argtypes = [P, P, P, C.c_int, F]
        L.mo_rms_norm_residual.argtypes = [P, P, P, P, C.c_int, F]
        L.mo_rms_norm_heads.argtypes = [P, P, P, C.c_int, C.c_int, F]
        L.mo_residual_add.argtypes = [P, P, P, C.c_int]
        L.mo_rope_freq.restype = F
        L.mo_rope_freq.argtypes = [C.c_int, C.c_int, F]
        L.mo_rope.argtypes = [P, P, C.c_int, C.c_int, F, C.c_int, C.c_int]
        L.mo_kv_quant_int8.argtypes = [P, P, P, C.c_int, C.c_int]
        L.mo_attention.restype = C.c_int
        L.mo_attention.argtypes = [P, P, P, P, P, C.c_int, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, F]
        self.L = L

    @staticmethod
    def _p(a: np.ndarray):
        return a.ctypes.data_as(C.c_void_p)

    def f16_to_f32(self, h: int) -> float:
        return self.L.mo_f16_to_f32(h)

    def f32_to_f16(self, f: float) -> int:
        return self.L.mo_f32_to_f16(f)

    def scale_min_k4(self, j: int, scales12: np.ndarray) -> tuple[int, int]:
        s = np.ascontiguousarray(scales12, np.uint8)
        sc, m = np.zeros(1, np.uint8), np.zeros(1, np.uint8)
        self.L.mo_get_scale_min_k4(j, self._p(s), self._p(sc), self._p(m))
        return int(sc[0]), int(m[0])

    def dequant(self, type_id: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint8)
        out = np.zeros((rows, cols), np.float32)
        if self.L.mo_dequant(type_id, self._p(w), self._p(out), rows, cols):
            raise ValueError(type_id)
        return out

    def gemv(self, type_id: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(rows, np.float64)
        if self.L.mo_gemv(type_id, self._p(w), self._p(x), self._p(y), rows, cols):
            raise ValueError(type_id)
        return y

    def gemv_f32acc(self, type_id, w, x, rows, cols, nthreads=0) -> np.ndarray:
        y = np.zeros(rows, np.float32)
        if self.L.mo_gemv_f32acc(type_id, self._p(w), self._p(x), self._p(y), rows, cols, nthreads):
            raise ValueError(type_id)
        return y

    def matvec_f32(self, w: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
        w = np.ascontiguousarray(w, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(rows, np.float64)
        self.L.mo_matvec_f32(self._p(w), self._p(x), self._p(y), rows, cols)
        return y

    def topk_softmax(self, scores: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
        s = np.ascontiguousarray(scores, np.float32)
        idx = np.zeros(k, np.int32)
        w = np.zeros(k, np.float32)
        self.L.mo_topk_softmax(self._p(s), s.size, k, self._p(idx), self._p(w))
        return idx, w

    def swiglu(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        out = np.zeros_like(g)
        self.L.mo_swiglu(self._p(g), self._p(u), self._p(out), g.size)
        return out

    def quantize_q8_1(self, src: np.ndarray) -> np.ndarray:
        src = np.ascontiguousarray(src, np.float32)
        n, k = src.shape
        out = np.zeros((n, k // 128, 144), np.uint8)
        self.L.mo_quantize_q8_1_mmq(self._p(src), self._p(out), k, n)
        return out

    def dequant_q8_1(self, blocks: np.ndarray, k: int, n: int) -> np.ndarray:
        b = np.ascontiguousarray(blocks, np.uint8)
        out = np.zeros((n, k), np.float32)
        self.L.mo_dequant_q8_1_mmq(self._p(b), self._p(out), k, n)
        return out

    def gemm(self, type_id: int, w: np.ndarray, act: np.ndarray, M: int, K: int, N: int) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint8)
        a = np.ascontiguousarray(act, np.uint8)
        out = np.zeros((N, M), np.float64)
        if self.L.mo_gemm_q8_1(type_id, self._p(w), self._p(a), self._p(out), M, K, N):
            raise ValueError(type_id)
        return out

    def sample_token(self, logits: np.ndarray, temperature: float, top_p: float, seed: int):
        z = np.ascontiguousarray(logits, np.float32)
        u = C.c_float(0.0)
        ns = C.c_float(0.0)
        tok = self.L.mo_sample_token(self._p(z), z.size, C.c_float(temperature), C.c_float(top_p),
                                     C.c_ulonglong(seed), C.byref(u), C.byref(ns))
        return int(tok), float(u.value), float(ns.value)

    def xoroshiro_next(self, s0: int, s1: int) -> tuple[int, int, int]:
        a, b = C.c_uint64(s0), C.c_uint64(s1)
        v = self.L.mo_xoroshiro_next(C.byref(a), C.byref(b))
        return int(v), int(a.value), int(b.value)

    def moe_prefill(self, table: np.ndarray, stride: int, gate_off: int, up_off: int, down_off: int,
                    down_type: int, x: np.ndarray, idx: np.ndarray, w: np.ndarray, hidden: int, eff: int,
                    n_experts: int) -> np.ndarray:
        """sum over slots of w * down(silu(gate x) * up x) per token, with x and the SwiGLU
        activations quantized to Q8_1: the reference's token-sequential MoE prefill
        (src/forward.c:1783-1830, per expert src/forward.c:876-893) in the GEMM semantics
        (mo_gemm_q8_1).  Pairs are grouped per expert only to batch the oracle GEMMs; each
        output row depends on its own token alone.  Returns the fp64 delta [T][hidden]."""
        T, k = idx.shape
        xq = self.quantize_q8_1(np.ascontiguousarray(x, np.float32).reshape(T, hidden))
        out = np.zeros((T, hidden), np.float64)
        gsz = up_off - gate_off
        for e in range(n_experts):
            tok, slot = np.nonzero(idx == e)
            if tok.size == 0:
                continue
            base = e * stride
            wg = table[base + gate_off: base + gate_off + gsz]
            wu = table[base + up_off: base + up_off + gsz]
            wd = table[base + down_off: base + stride]
            g = self.gemm(12, wg, xq[tok], eff, hidden, tok.size).astype(np.float32)
            u = self.gemm(12, wu, xq[tok], eff, hidden, tok.size).astype(np.float32)
            act = self.swiglu(g, u).reshape(tok.size, eff)
            d = self.gemm(down_type, wd, self.quantize_q8_1(act), hidden, eff, tok.size)
            np.add.at(out, tok, w[tok, slot][:, None].astype(np.float64) * d)
        return out

    # ---------------------------------------------------------------- attention chain
    @staticmethod
    def _f32(a) -> np.ndarray:
        return np.ascontiguousarray(a, np.float32)

    def rms_norm(self, x, w, eps: float) -> np.ndarray:
        x, w = self._f32(x), self._f32(w)
        out = np.zeros_like(x)
        self.L.mo_rms_norm(self._p(x), self._p(w), self._p(out), x.size, eps)
        return out

    def rms_norm_residual(self, x, w, eps: float):
        x, w = self._f32(x), self._f32(w)
        normed, res = np.zeros_like(x), np.zeros_like(x)
        self.L.mo_rms_norm_residual(self._p(x), self._p(w), self._p(normed), self._p(res), x.size, eps)
        return normed, res

    def rms_norm_heads(self, x, w, head_dim: int, eps: float) -> np.ndarray:
        x, w = self._f32(x), self._f32(w)
        out = np.zeros_like(x)
        self.L.mo_rms_norm_heads(self._p(x), self._p(w), self._p(out), head_dim, x.size // head_dim, eps)
        return out

    def residual_add(self, a, b) -> np.ndarray:
        a, b = self._f32(a), self._f32(b)
        out = np.zeros_like(a)
        self.L.mo_residual_add(self._p(a), self._p(b), self._p(out), a.size)
        return out

    def rope_freq(self, j: int, head_dim: int, theta: float) -> float:
        return self.L.mo_rope_freq(j, head_dim, theta)

    def rope(self, q, k, head_dim: int, pos: int, theta: float):
        q, k = self._f32(q).copy(), self._f32(k).copy()
        self.L.mo_rope(self._p(q), self._p(k), head_dim, pos, theta, q.size // head_dim, k.size // head_dim)
        return q, k

    def kv_quant_int8(self, x, head_dim: int):
        x = self._f32(x)
        out = np.zeros(x.size, np.int8)
        sc = np.zeros(x.size // head_dim, np.float32)
        self.L.mo_kv_quant_int8(self._p(x), self._p(out), self._p(sc), head_dim, x.size // head_dim)
        return out, sc

    def attention(self, q, kv_k, kv_v, n_heads: int, head_dim: int, n_kv_heads: int, seq_len: int,
                  scale: float, k_scales=None, v_scales=None) -> np.ndarray:
        """kv_k / kv_v: uint16 f16 bits (kv_type 0) or int8 with [pos][kv head] scales."""
        q = self._f32(q)
        kt = 0 if kv_k.dtype == np.uint16 else 1
        kk, vv = np.ascontiguousarray(kv_k), np.ascontiguousarray(kv_v)
        ks = self._f32(k_scales) if k_scales is not None else np.zeros(1, np.float32)
        vs = self._f32(v_scales) if v_scales is not None else np.zeros(1, np.float32)
        out = np.zeros(n_heads * head_dim, np.float32)
        if self.L.mo_attention(self._p(q), self._p(kk), self._p(vv), self._p(ks), self._p(vs), kt, self._p(out),
                               n_heads, head_dim, n_kv_heads, seq_len, n_heads // n_kv_heads, scale):
            raise ValueError("attention arguments")
        return out


_oracle: Oracle | None = None


def load() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


# ---------------------------------------------------------------- CPU baseline
def _has_avx512() -> bool:
    try:
        flags = next(l for l in open("/proc/cpuinfo") if l.startswith("flags")).split()
    except (OSError, StopIteration):
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512dq", "avx512vl"))


class Baseline:
    """The vectorised CPU GEMV bench.py times (cpu_baseline.c), built for x86-64-v4 and
    x86-64-v3; the AVX-512 build is used where the host CPU has it."""

    def __init__(self):
        level = "v4" if _has_avx512() else "v3"
        path = HERE / "_build" / f"libmnemo_baseline_{level}.so"
        if not path.exists():
            build()
        self.level = level
        self.L = C.CDLL(str(path))
        self.L.mo_base_gemv.restype = C.c_int
        self.L.mo_base_gemv.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]

    def gemv(self, type_id: int, w: np.ndarray, x: np.ndarray, rows: int, cols: int, nthreads: int = 0) -> np.ndarray:
        w = np.ascontiguousarray(w, np.uint8)
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(rows, np.float32)
        if self.L.mo_base_gemv(type_id, w.ctypes.data, x.ctypes.data, y.ctypes.data, rows, cols, nthreads):
            raise ValueError((type_id, cols))
        return y


_baseline: Baseline | None = None


def load_baseline() -> Baseline:
    global _baseline
    if _baseline is None:
        _baseline = Baseline()
    return _baseline
