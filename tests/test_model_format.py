"""CPU checks of the split model directory reader (include/mnemo_model.h) against the
format of MnemoCUDA docs/model-format.md and the loader src/engine.c:376-460, 524-736:
required keys and defaults, prefix detection, whole-key matching, manifest fields,
expert-size rules and the validation errors.  Nothing here touches a GPU."""
import json

import pytest

from mnemocuda_amd import model as mm
from mnemocuda_amd.lib import MnemoError
from tests.model_fixture import F32, Q4K, Q6K, write_model


def test_config_required_defaults_and_prefix():
    text = json.dumps({"qwen3moe.embedding_length": 4096, "qwen3moe.block_count": 94,
                       "qwen3moe.attention.head_count": 64, "qwen3moe.attention.head_count_kv": 4})
    c = mm.parse_config(text)
    assert (c.prefix, c.hidden_size, c.n_layers, c.n_heads, c.n_kv_heads) == (b"qwen3moe", 4096, 94, 64, 4)
    # defaults of src/engine.c:411-444
    assert (c.eff, c.head_dim, c.n_experts, c.experts_per_tok, c.context_length, c.vocab_size) == \
        (1536, 128, 128, 8, 40960, 151936)
    assert c.rope_theta == 1e6 and abs(c.rms_eps - 1e-6) < 1e-12 and c.full_attention_interval == 0
    t2 = json.dumps({"llama.embedding_length": 2048, "llama.block_count": 16, "llama.attention.head_count": 32,
                     "llama.attention.head_count_kv": 8, "llama.rope.freq_base": 10000.0, "vocab_size": 32000})
    c2 = mm.parse_config(t2)
    assert c2.prefix == b"llama" and c2.rope_theta == 10000.0 and c2.vocab_size == 32000


def test_config_whole_key_match_and_missing():
    # a nested object that contains a key with the same text must not be taken for it
    text = json.dumps({"meta": {"qwen3moe.embedding_length": 1}, "qwen3moe.embedding_length": 4096,
                       "qwen3moe.block_count": 2, "qwen3moe.attention.head_count": 4,
                       "qwen3moe.attention.head_count_kv": 2,
                       "qwen3moe.expert_feed_forward_length_extra": 7})
    c = mm.parse_config(text)
    assert c.hidden_size == 4096 and c.eff == 1536
    with pytest.raises(MnemoError, match="head_count_kv"):
        mm.parse_config(json.dumps({"qwen3moe.embedding_length": 4096, "qwen3moe.block_count": 2,
                                    "qwen3moe.attention.head_count": 4}))
    with pytest.raises(MnemoError):
        mm.parse_config("[1, 2]")
    with pytest.raises(MnemoError, match="head counts"):
        mm.parse_config(json.dumps({"qwen3moe.embedding_length": 64, "qwen3moe.block_count": 2,
                                    "qwen3moe.attention.head_count": 6, "qwen3moe.attention.head_count_kv": 4}))


@pytest.mark.parametrize("key,value,match", [
    ("expert_count", 0, "expert count"), ("expert_count", -3, "expert count"), ("expert_count", 513, "expert count"),
    ("expert_used_count", 0, "expert_used_count"), ("expert_used_count", 200, "expert_used_count"),
    ("expert_feed_forward_length", 0, "expert_feed_forward_length"), ("attention.key_length", -128, "key_length"),
    ("attention.key_length", 129, "key_length"), ("context_length", 0, "context_length")])
def test_config_rejects_invalid_sizes(key, value, match):
    """Sizes the loader divides or indexes by are range-checked (an expert_count of 0 would
    otherwise divide the expert file size by zero)."""
    cfg = {"qwen3moe.embedding_length": 4096, "qwen3moe.block_count": 2, "qwen3moe.attention.head_count": 4,
           "qwen3moe.attention.head_count_kv": 2, f"qwen3moe.{key}": value}
    with pytest.raises(MnemoError, match=match):
        mm.parse_config(json.dumps(cfg))


def test_resident_manifest_fields():
    big = 2**40 + 3  # offsets beyond 2^32 (and exact beyond 2^53 would need integers: parsed as such)
    text = json.dumps({"version": 2, "tensors": [
        {"name": "token_embd.weight", "offset": 0, "size": 144, "type_id": 12, "dims": [256, 1]},
        {"dims": [4096], "type_id": 0, "size": 16384, "offset": big, "name": "blk.0.attn_norm.weight",
         "extra": {"x": [1, 2, {"y": "z"}]}},
        {"name": 'a"b\u00e9', "offset": 1, "size": 2, "type_id": 14, "dims": []}]})  # json escapes " and é
    t = mm.parse_resident_manifest(text)
    assert [x.name for x in t] == [b"token_embd.weight", b"blk.0.attn_norm.weight", 'a"b\u00e9'.encode()]
    assert t[1].offset == big and t[1].size == 16384 and t[1].type_id == 0
    assert t[0].n_dims == 2 and list(t[0].dims[:2]) == [256, 1] and t[2].n_dims == 0
    assert mm.parse_resident_manifest(json.dumps({"tensors": []})) == []
    with pytest.raises(MnemoError, match="tensors"):
        mm.parse_resident_manifest(json.dumps({"x": []}))
    with pytest.raises(MnemoError):
        mm.parse_resident_manifest('{"tensors": [{"name": "a", "offset": 1,')
    with pytest.raises(MnemoError, match="type_id"):
        mm.parse_resident_manifest(json.dumps({"tensors": [{"name": "a", "offset": 0, "size": 1}]}))


def test_expert_manifest_top_and_nested():
    layer = {"expert_size": 100, "gate_size": 30, "up_size": 30, "down_size": 40}
    top = json.dumps({"1": layer, "10": {"expert_size": 7}})
    i = mm.parse_expert_manifest(top, 1)
    assert (i.expert_size, i.gate_size, i.up_size, i.down_size) == (100, 30, 30, 40)
    assert mm.parse_expert_manifest(top, 10).expert_size == 7  # "1" does not match "10"
    assert mm.parse_expert_manifest(top, 2).expert_size == 0
    nested = json.dumps({"format": 1, "layers": {"3": layer}})
    assert mm.parse_expert_manifest(nested, 3).down_size == 40


def test_model_open_and_layers(tmp_path):
    meta = write_model(tmp_path / "m", manifest_layers="top")
    m = mm.Model(tmp_path / "m")
    c = m.config
    assert (c.hidden_size, c.n_layers, c.vocab_size, c.rope_theta) == (512, 2, 300, 5e5)
    names = [t.name.decode() for t in m.tensors()]
    assert names[:3] == ["token_embd.weight", "output_norm.weight", "output.weight"] and len(names) == 3 + 2 * 6
    e = m.expert_layer(1)
    assert (e.expert_size, e.gate_size, e.down_size, e.down_type_id, e.n_experts) == \
        (meta["expert_size"], meta["gate_size"], meta["down_size"], Q6K, 4)
    with pytest.raises(MnemoError):
        m.expert_layer(2)
    m.close()


def test_model_open_without_manifest_uses_file_size_and_thirds(tmp_path):
    meta = write_model(tmp_path / "m", manifest_layers=None, down_type=Q4K)
    m = mm.Model(tmp_path / "m")
    e = m.expert_layer(0)
    assert e.expert_size == meta["expert_size"]
    assert e.gate_size == e.up_size == e.expert_size // 3 and e.down_size == e.expert_size - 2 * (e.expert_size // 3)
    m.close()


def test_model_open_validation(tmp_path):
    write_model(tmp_path / "m")
    man = json.loads((tmp_path / "m" / "resident_manifest.json").read_text())
    man["tensors"][1]["offset"] = (tmp_path / "m" / "resident_weights.bin").stat().st_size  # past the end
    (tmp_path / "m" / "resident_manifest.json").write_text(json.dumps(man))
    with pytest.raises(MnemoError, match="outside resident_weights.bin"):
        mm.Model(tmp_path / "m")
    write_model(tmp_path / "n")
    with open(tmp_path / "n" / "experts" / "layer_01.bin", "ab") as f:
        f.write(b"\0")
    with pytest.raises(MnemoError, match="layer_01.bin"):
        mm.Model(tmp_path / "n")
    write_model(tmp_path / "o")
    em = json.loads((tmp_path / "o" / "expert_manifest.json").read_text())
    em["0"]["down_size"] = em["0"]["expert_size"]
    (tmp_path / "o" / "expert_manifest.json").write_text(json.dumps(em))
    with pytest.raises(MnemoError, match="gate \\+ up \\+ down"):
        mm.Model(tmp_path / "o")
    with pytest.raises(MnemoError, match="cannot read"):
        mm.Model(tmp_path / "missing")


def test_row_bytes():
    from mnemocuda_amd import load_library
    L = load_library()
    assert L.mnemo_row_bytes(Q4K, 4096) == 16 * 144 and L.mnemo_row_bytes(Q6K, 1536) == 6 * 210
    assert L.mnemo_row_bytes(F32, 10) == 40 and L.mnemo_row_bytes(8, 64) == 0 and L.mnemo_row_bytes(Q4K, 300) == 2 * 144
