"""ctypes binding of libmnemo_hip.so (include/mnemo_kernels.h + include/mnemo_host.h).

Every exported symbol is declared here with its C signature; ``EXPORTS`` is the list the
CPU test compares against the headers.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmnemo_hip.so"

vp, fp, ip = C.c_void_p, C.c_void_p, C.c_void_p  # device pointers travel as void*
i32, f32, sz = C.c_int, C.c_float, C.c_size_t
stream_t = C.c_void_p

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    "mnemo_last_error": (i32, []),
    "mnemo_last_error_string": (C.c_char_p, []),
    "mnemo_version": (C.c_char_p, []),
    "cuda_kernels_init": (None, []),
    "cuda_matvec_q4k": (None, [vp, fp, fp, i32, i32, stream_t]),
    "cuda_matvec_q4k_add": (None, [vp, fp, fp, fp, i32, i32, stream_t]),
    "cuda_matvec_q4k_qkv": (None, [vp, vp, vp, fp, fp, fp, fp, i32, i32, i32, stream_t]),
    "cuda_matvec_q4k_dual": (None, [vp, vp, fp, fp, fp, i32, i32, stream_t]),
    "cuda_matvec_q4k_scaled_add": (None, [vp, fp, fp, i32, i32, f32, stream_t]),
    "cuda_matvec_q6k": (None, [vp, fp, fp, i32, i32, stream_t]),
    "mnemo_matvec_q6k_scaled_add": (None, [vp, fp, fp, i32, i32, f32, stream_t]),
    "mnemo_matvec_dual": (None, [vp, i32, vp, i32, fp, fp, fp, i32, i32, stream_t]),
    "mnemo_matvec_qkv": (None, [vp, i32, vp, i32, vp, i32, fp, fp, fp, fp, i32, i32, i32, stream_t]),
    "mnemo_matvec_qkv_rmsnorm": (None, [vp, i32, vp, i32, vp, i32, fp, fp, f32, fp, fp, fp, i32, i32, i32,
                                         stream_t]),
    "mnemo_matvec_swiglu_scaled_add": (None, [vp, i32, fp, fp, fp, i32, i32, f32, stream_t]),
    "cuda_matvec_f32": (None, [fp, fp, fp, i32, i32, stream_t]),
    "cuda_topk_softmax": (None, [fp, ip, fp, i32, i32, stream_t]),
    "cuda_swiglu": (None, [fp, fp, fp, i32, stream_t]),
    "cuda_scaled_add": (None, [fp, fp, f32, i32, stream_t]),
    "cuda_quantize_mmq_q8_1": (None, [fp, vp, i32, i32, stream_t]),
    "cuda_gemm_q4k": (None, [vp, vp, fp, i32, i32, i32, stream_t]),
    "mnemo_gemm_q6k": (None, [vp, vp, fp, i32, i32, i32, stream_t]),
    "cuda_sample_token": (None, [fp, i32, f32, f32, C.c_ulonglong, ip, stream_t]),
    "mnemo_sample_workspace_bytes": (sz, []),
    "mnemo_sample_token_ws": (i32, [fp, i32, f32, f32, C.c_ulonglong, vp, sz, ip, stream_t]),
    "mnemo_moe_prefill_workspace_bytes": (sz, [i32, i32, i32, i32, i32]),
    "mnemo_moe_prefill": (i32, [vp, sz, sz, sz, sz, i32, fp, ip, fp, i32, i32, i32, i32, i32, vp, sz, fp,
                                stream_t]),
    "mnemo_moe_decode_workspace_bytes": (sz, [i32, i32, i32, i32]),
    "mnemo_moe_decode": (i32, [fp, vp, sz, sz, sz, sz, i32, fp, i32, i32, i32, i32, vp, sz, fp, ip, fp, stream_t]),
    "mnemo_moe_decode_rmsnorm": (i32, [fp, vp, sz, sz, sz, sz, i32, fp, fp, f32, i32, i32, i32, i32, vp, sz, fp,
                                        ip, fp, stream_t]),
    "mnemo_moe_decode_rmsnorm_noalloc": (i32, [fp, vp, sz, sz, sz, sz, i32, fp, fp, f32, i32, i32, i32, i32, fp, ip,
                                                fp, stream_t]),
    # attention chain
    "cuda_rms_norm": (None, [fp, fp, fp, i32, f32, stream_t]),
    "cuda_rms_norm_residual": (None, [fp, fp, fp, fp, i32, f32, stream_t]),
    "cuda_rms_norm_batched": (None, [fp, fp, fp, i32, i32, f32, stream_t]),
    "cuda_rms_norm_qk": (None, [fp, fp, fp, fp, i32, i32, i32, f32, stream_t]),
    "cuda_residual_add": (None, [fp, fp, fp, i32, stream_t]),
    "cuda_rope": (None, [fp, fp, i32, i32, f32, i32, i32, stream_t]),
    "cuda_f32_to_f16_dual": (None, [fp, fp, vp, vp, i32, stream_t]),
    "cuda_get_rope_kernel_ptr": (vp, []),
    "cuda_get_f16dual_kernel_ptr": (vp, []),
    "cuda_get_attn_f16kv_kernel_ptr": (vp, []),
    "mnemo_attention_reserve": (i32, [i32]),
    "mnemo_attention_slot_bytes": (sz, []),
    "cuda_f32_to_int8_kv_dual": (None, [fp, fp, vp, vp, fp, fp, i32, i32, stream_t]),
    "cuda_attention_f16kv": (None, [vp, vp, vp, fp, i32, i32, i32, i32, i32, f32, stream_t]),
    "cuda_attention_int8kv": (None, [fp, vp, vp, fp, fp, fp, i32, i32, i32, i32, i32, f32, stream_t]),
    "mnemo_attn_prep": (i32, [fp, fp, fp, fp, fp, i32, i32, i32, f32, f32, ip, vp, vp, fp, fp, i32, i32, stream_t]),
    "mnemo_v_cache_bytes": (sz, [i32, i32, i32, i32, i32]),
    "mnemo_attention": (i32, [fp, vp, vp, fp, fp, i32, fp, i32, i32, i32, ip, f32, stream_t]),
    "mnemo_attention_decode_workspace_bytes": (sz, [i32, i32]),
    "mnemo_attention_decode": (i32, [fp, vp, vp, fp, fp, i32, i32, fp, i32, i32, i32, i32, ip, f32, vp, sz,
                                     stream_t]),
    "mnemo_attention_decode_prep": (i32, [fp, fp, fp, fp, fp, f32, f32, vp, vp, fp, fp, i32, i32, fp, i32, i32, i32,
                                          i32, ip, f32, vp, sz, stream_t]),
    "cuda_embedding_lookup_q4k": (None, [vp, fp, i32, i32, i32, stream_t]),
    "mnemo_embedding_lookup": (i32, [vp, i32, ip, i32, fp, i32, stream_t]),
    # model directory (mnemo_model.h); structs travel as void*
    "mnemo_parse_config": (i32, [C.c_char_p, vp]),
    "mnemo_parse_resident_manifest": (i32, [C.c_char_p, vp, i32, vp]),
    "mnemo_parse_expert_manifest": (i32, [C.c_char_p, i32, vp]),
    "mnemo_row_bytes": (sz, [i32, i32]),
    "mnemo_model_open": (i32, [C.c_char_p, vp]),
    "mnemo_model_config_of": (vp, [vp]),
    "mnemo_model_n_tensors": (i32, [vp]),
    "mnemo_model_tensor_at": (i32, [vp, i32, vp]),
    "mnemo_model_expert_layer": (i32, [vp, i32, vp]),
    "mnemo_model_upload": (i32, [vp, i32]),
    "mnemo_model_tensor": (i32, [vp, C.c_char_p, vp, vp]),
    "mnemo_model_experts": (i32, [vp, i32, vp]),
    "mnemo_model_close": (None, [vp]),
    # host composition (mnemo_host.h)
    "mnemo_matvec": (i32, [vp, fp, fp, i32, i32, i32, stream_t]),
    "mnemo_down_type_id": (i32, [sz, i32, i32]),
    "mnemo_expert_fwd": (i32, [vp, sz, sz, i32, i32, i32, f32, fp, fp, fp, fp, stream_t]),
}
EXPORTS = sorted(SIGNATURES)


class MnemoError(RuntimeError):
    pass


_lib: C.CDLL | None = None


def load_library(path: Path | str | None = None) -> C.CDLL:
    """Load libmnemo_hip.so and declare every signature.  Raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise MnemoError(f"{p} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                         "or `python mnemocuda_amd/build.py`")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(lib: C.CDLL, what: str) -> None:
    e = lib.mnemo_last_error()
    if e:
        raise MnemoError(f"{what}: error {e}: {lib.mnemo_last_error_string().decode()}")
