"""Writes a small split model directory in the reference's format (docs/model-format.md):
config.json, resident_manifest.json + resident_weights.bin, expert_manifest.json and
experts/layer_XX.bin, with seeded Q4_K / Q6_K / F32 tensors from mnemocuda_amd.synth."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from mnemocuda_amd import synth

Q4K, Q6K, F32 = 12, 14, 0


def row_bytes(t, n):
    return {Q4K: (n + 255) // 256 * 144, Q6K: (n + 255) // 256 * 210, F32: 4 * n}[t]


def tensor_bytes(rng, t, rows, cols):
    if t == F32:
        return rng.standard_normal(rows * cols).astype(np.float32).tobytes()
    return synth.weights(rng, t, rows, cols).tobytes()


def write_model(d: Path, *, hidden=512, layers=2, heads=8, kv_heads=2, head_dim=64, eff=256, experts=4, vocab=300,
                embd_type=Q4K, prefix="qwen3moe", manifest_layers="top", down_type=Q6K, seed=7,
                extra_config=None) -> dict:
    rng = np.random.default_rng(seed)
    d = Path(d)
    (d / "experts").mkdir(parents=True, exist_ok=True)
    cfg = {f"{prefix}.embedding_length": hidden, f"{prefix}.block_count": layers,
           f"{prefix}.attention.head_count": heads, f"{prefix}.attention.head_count_kv": kv_heads,
           f"{prefix}.attention.key_length": head_dim, f"{prefix}.expert_feed_forward_length": eff,
           f"{prefix}.expert_count": experts, f"{prefix}.expert_used_count": 2,
           f"{prefix}.rope.freq_base": 5e5, "tokenizer.ggml.tokens_count": vocab,
           "general.name": "tiny \"test\" model", "general.tags": ["a", {"b": 1}]}
    cfg.update(extra_config or {})
    (d / "config.json").write_text(json.dumps(cfg, indent=1))
    tensors, blob, off = [], bytearray(), 0
    spec = [("token_embd.weight", embd_type, vocab, hidden), ("output_norm.weight", F32, 1, hidden),
            ("output.weight", Q6K, vocab, hidden)]
    for l in range(layers):
        spec += [(f"blk.{l}.attn_norm.weight", F32, 1, hidden), (f"blk.{l}.attn_q.weight", Q4K, heads * head_dim, hidden),
                 (f"blk.{l}.attn_k.weight", Q4K, kv_heads * head_dim, hidden),
                 (f"blk.{l}.attn_v.weight", Q6K, kv_heads * head_dim, hidden),
                 (f"blk.{l}.attn_output.weight", Q4K, hidden, heads * head_dim),
                 (f"blk.{l}.ffn_gate_inp.weight", F32, experts, hidden)]
    data = {}
    for name, t, rows, cols in spec:
        b = tensor_bytes(rng, t, rows, cols)
        blob += b"\0" * 40  # gaps between tensors, as a real file may have
        off = len(blob)
        blob += b
        data[name] = (t, rows, cols, b)
        tensors.append({"name": name, "offset": off, "size": len(b), "type_id": t, "dims": [cols, rows]})
    (d / "resident_weights.bin").write_bytes(bytes(blob))
    (d / "resident_manifest.json").write_text(json.dumps({"version": 1, "tensors": tensors}))
    gsz = row_bytes(Q4K, hidden) * eff
    dsz = row_bytes(down_type, eff) * hidden
    esz = 2 * gsz + dsz
    man = {}
    experts_data = {}
    for l in range(layers):
        e = b"".join(tensor_bytes(rng, Q4K, eff, hidden) + tensor_bytes(rng, Q4K, eff, hidden) +
                     tensor_bytes(rng, down_type, hidden, eff) for _ in range(experts))
        (d / "experts" / f"layer_{l:02d}.bin").write_bytes(e)
        experts_data[l] = e
        man[str(l)] = {"expert_size": esz, "gate_size": gsz, "up_size": gsz, "down_size": dsz}
    if manifest_layers == "top":
        (d / "expert_manifest.json").write_text(json.dumps(man))
    elif manifest_layers == "nested":
        (d / "expert_manifest.json").write_text(json.dumps({"format": 1, "layers": man}))
    return {"tensors": data, "experts": experts_data, "expert_size": esz, "gate_size": gsz, "down_size": dsz}
