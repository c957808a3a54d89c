"""The split model directory (include/mnemo_model.h) from Python: ctypes structures and a
small wrapper around mnemo_model_open / upload / tensor lookups."""
from __future__ import annotations

import ctypes as C

from .lib import MnemoError, load_library


class ModelConfig(C.Structure):
    _fields_ = [("prefix", C.c_char * 32), ("hidden_size", C.c_int), ("n_layers", C.c_int), ("n_heads", C.c_int),
                ("n_kv_heads", C.c_int), ("head_dim", C.c_int), ("eff", C.c_int), ("n_experts", C.c_int),
                ("experts_per_tok", C.c_int), ("context_length", C.c_int), ("full_attention_interval", C.c_int),
                ("vocab_size", C.c_int), ("rope_theta", C.c_float), ("rms_eps", C.c_float)]


class TensorInfo(C.Structure):
    _fields_ = [("name", C.c_char * 128), ("offset", C.c_size_t), ("size", C.c_size_t), ("type_id", C.c_int),
                ("n_dims", C.c_int), ("dims", C.c_longlong * 4)]


class ExpertLayerInfo(C.Structure):
    _fields_ = [("expert_size", C.c_size_t), ("gate_size", C.c_size_t), ("up_size", C.c_size_t),
                ("down_size", C.c_size_t), ("down_type_id", C.c_int), ("n_experts", C.c_int)]


def _rc(lib, rc: int, what: str) -> None:
    lib.mnemo_last_error()
    if rc:
        raise MnemoError(f"{what}: error {rc}: {lib.mnemo_last_error_string().decode()}")


def parse_config(text: str) -> ModelConfig:
    lib = load_library()
    cfg = ModelConfig()
    _rc(lib, lib.mnemo_parse_config(text.encode(), C.addressof(cfg)), "parse_config")
    return cfg


def parse_resident_manifest(text: str) -> list[TensorInfo]:
    lib = load_library()
    n = C.c_int(0)
    _rc(lib, lib.mnemo_parse_resident_manifest(text.encode(), None, 0, C.addressof(n)), "parse_resident_manifest")
    arr = (TensorInfo * max(n.value, 1))()
    _rc(lib, lib.mnemo_parse_resident_manifest(text.encode(), C.addressof(arr), n.value, C.addressof(n)),
        "parse_resident_manifest")
    return list(arr[:n.value])


def parse_expert_manifest(text: str, layer: int) -> ExpertLayerInfo:
    lib = load_library()
    info = ExpertLayerInfo()
    _rc(lib, lib.mnemo_parse_expert_manifest(text.encode(), layer, C.addressof(info)), "parse_expert_manifest")
    return info


class Model:
    """mnemo_model_open(dir); upload() places resident tensors and expert layers on the
    current device; tensor(name) / experts(layer) return device pointers (int)."""

    def __init__(self, path: str):
        self.lib = load_library()
        h = C.c_void_p()
        _rc(self.lib, self.lib.mnemo_model_open(str(path).encode(), C.addressof(h)), "model_open")
        self.h = h

    @property
    def config(self) -> ModelConfig:
        p = self.lib.mnemo_model_config_of(self.h)
        return ModelConfig.from_buffer_copy(C.string_at(p, C.sizeof(ModelConfig)))

    def tensors(self) -> list[TensorInfo]:
        out = []
        for i in range(self.lib.mnemo_model_n_tensors(self.h)):
            t = TensorInfo()
            _rc(self.lib, self.lib.mnemo_model_tensor_at(self.h, i, C.addressof(t)), "model_tensor_at")
            out.append(t)
        return out

    def expert_layer(self, layer: int) -> ExpertLayerInfo:
        info = ExpertLayerInfo()
        _rc(self.lib, self.lib.mnemo_model_expert_layer(self.h, layer, C.addressof(info)), "model_expert_layer")
        return info

    def upload(self, with_experts: bool = True) -> None:
        _rc(self.lib, self.lib.mnemo_model_upload(self.h, int(with_experts)), "model_upload")

    def tensor(self, name: str) -> tuple[TensorInfo, int]:
        info, ptr = TensorInfo(), C.c_void_p()
        _rc(self.lib, self.lib.mnemo_model_tensor(self.h, name.encode(), C.addressof(info), C.addressof(ptr)),
            "model_tensor")
        return info, ptr.value or 0

    def experts(self, layer: int) -> int:
        ptr = C.c_void_p()
        _rc(self.lib, self.lib.mnemo_model_experts(self.h, layer, C.addressof(ptr)), "model_experts")
        return ptr.value

    def close(self) -> None:
        if self.h:
            self.lib.mnemo_model_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
