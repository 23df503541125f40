"""Safetensors input (host side, no GPU): header parsing and its checks, sharded indexes, layer bytes,
and the Qwen3 checkpoint mapping with strict / non-strict key handling.

Files are written by the `safetensors` package (an implementation independent of this repository's
parser), bf16 through torch; the header checks follow the
format (the reference parser: packages/core/src/io/safetensor/parser.ts:28-172), the index
sharded.ts:20-96, the key handling from
nn/module.ts:572-660.
"""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from kandle_amd.io import host_array, load_safetensor, parse_header_size, parse_safetensor_file
from kandle_amd.model_utils import Qwen3Config, init_qwen3_weights, qwen3_weights_from_safetensor


def _bf16_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


def test_parse_single_file_bits_and_shapes(tmp_path):
    rng = np.random.default_rng(0)
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    bits = rng.integers(0, 0x7F80, size=(4, 2, 3), dtype=np.uint16)
    i32 = np.arange(7, dtype=np.int32)
    path = str(tmp_path / "m.safetensors")
    save_file({"a.f32": torch.from_numpy(f32), "b.bf16": _bf16_tensor(bits), "c.i32": torch.from_numpy(i32)}, path,
              metadata={"format": "pt"})
    g = load_safetensor(path)
    assert not g.sharded and g.metadata == {"format": "pt"}
    assert set(g.layers) == {"a.f32", "b.bf16", "c.i32"}
    a, b, c = g.get_layer("a.f32"), g.get_layer("b.bf16"), g.get_layer("c.i32")
    assert (a.original_dtype, a.dtype, a.shape) == ("F32", "float32", (3, 5))
    assert (b.original_dtype, b.dtype, b.shape, b.byte_size) == ("BF16", "bfloat16", (4, 2, 3), 48)
    np.testing.assert_array_equal(a.numpy(), f32)
    np.testing.assert_array_equal(b.numpy(), bits)           # native bf16 bits, no widening
    np.testing.assert_array_equal(c.numpy(), i32)
    # the reference's widening on request: bits << 16
    np.testing.assert_array_equal(host_array(b, "float32").view(np.uint32), bits.astype(np.uint32) << 16)
    # F32 -> bf16 rounds to nearest even: 1 + 2^-8 (half an ulp) -> 1 (0x3F80, even); 1 + 3*2^-8
    # (halfway between 0x3F81 and 0x3F82) -> 0x3F82 (even)
    ties = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32)
    save_file({"t": torch.from_numpy(ties)}, str(tmp_path / "t.safetensors"))
    t = load_safetensor(str(tmp_path / "t.safetensors")).get_layer("t")
    np.testing.assert_array_equal(host_array(t, "bfloat16"), np.array([0x3F80, 0x3F82], np.uint16))
    g.close()


def _raw_file(path, header: bytes, data: bytes = b"", size_field=None):
    n = len(header) if size_field is None else size_field
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Q", n) + header + data)


def test_header_checks(tmp_path):
    assert parse_header_size(struct.pack("<Q", 123)) == 123
    with pytest.raises(ValueError, match="exceeds the format's cap"):
        parse_header_size(struct.pack("<Q", 1 << 33))
    with pytest.raises(ValueError, match="exceeds the format's cap"):
        parse_header_size(struct.pack("<Q", 100 * 1024 * 1024 + 1))
    with pytest.raises(ValueError, match="file too small"):
        parse_header_size(b"\x01\x02")
    p = str(tmp_path / "x.safetensors")
    _raw_file(p, b"{not json")
    with pytest.raises(ValueError, match="not valid UTF-8 JSON"):
        parse_safetensor_file(p)
    _raw_file(p, b"", size_field=0)
    with pytest.raises(ValueError, match="empty header"):
        parse_safetensor_file(p)
    _raw_file(p, b"{}", size_field=64)
    with pytest.raises(ValueError, match="incomplete"):
        parse_safetensor_file(p)
    hdr = json.dumps({"w": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 12]}}).encode()
    _raw_file(p, hdr, b"\0" * 12)
    with pytest.raises(ValueError, match="tensor 'w' \\(F32, shape \\(2, 2\\)\\) needs 16 bytes but its data_offsets span 12"):
        parse_safetensor_file(p)
    hdr = json.dumps({"w": {"dtype": "F8_E4M3", "shape": [2], "data_offsets": [0, 2]}}).encode()
    _raw_file(p, hdr, b"\0" * 2)
    with pytest.raises(ValueError, match="dtype 'F8_E4M3', which this loader does not read"):
        parse_safetensor_file(p)
    hdr = json.dumps({"w": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}).encode()
    _raw_file(p, hdr, b"\0" * 8)   # truncated data area
    with pytest.raises(ValueError, match="occupies bytes \\[0, 16\\) of a 8-byte data area"):
        parse_safetensor_file(p)
    for bad, what in (({"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}, "shape"),
                      ({"dtype": "F32", "shape": [1], "data_offsets": [0]}, "data_offsets"),
                      ({"dtype": "F32", "shape": [1], "data_offsets": [8, 4]}, "span -4")):
        _raw_file(p, json.dumps({"w": bad}).encode(), b"\0" * 8)
        with pytest.raises(ValueError, match=what):
            parse_safetensor_file(p)
    _raw_file(p, b"[1, 2]")
    with pytest.raises(ValueError, match="not an object"):
        parse_safetensor_file(p)
    # hostile shapes: a product past 2^64 (no int64 wrap to 0 bytes), a dim past 2^63
    for shape in ([2 ** 62, 4], [2 ** 64 + 1]):
        _raw_file(p, json.dumps({"w": {"dtype": "F32", "shape": shape, "data_offsets": [0, 0]}}).encode())
        with pytest.raises(ValueError, match="needs"):
            parse_safetensor_file(p)
    for meta in ([1, 2], "text", {"k": 3}):
        _raw_file(p, json.dumps({"__metadata__": meta}).encode())
        with pytest.raises(ValueError, match="__metadata__ must be an object"):
            parse_safetensor_file(p)
    # entries that describe no tensor (no data_offsets) are skipped, as in the reference
    hdr = json.dumps({"__metadata__": {"k": "v"}, "junk": 3, "w": {"dtype": "I32", "shape": [], "data_offsets": [0, 4]}}).encode()
    _raw_file(p, hdr, struct.pack("<i", -5))
    f = parse_safetensor_file(p)
    assert list(f.layers) == ["w"] and f.metadata == {"k": "v"} and int(f.layers["w"].numpy()) == -5
    f.close()


def _write_sharded(tmp_path, tensors: dict, split: int):
    names = list(tensors)
    shards = {"model-00001-of-00002.safetensors": names[:split], "model-00002-of-00002.safetensors": names[split:]}
    wm, total = {}, 0
    for shard, keys in shards.items():
        save_file({k: tensors[k] for k in keys}, str(tmp_path / shard))
        for k in keys:
            wm[k] = shard
            total += tensors[k].numel() * tensors[k].element_size()
    with open(tmp_path / "model.safetensors.index.json", "w") as fh:
        json.dump({"metadata": {"total_size": total}, "weight_map": wm}, fh)
    return total


def test_sharded_index(tmp_path):
    rng = np.random.default_rng(1)
    ts = {f"t{i}": torch.from_numpy(rng.standard_normal((i + 1, 3)).astype(np.float32)) for i in range(5)}
    total = _write_sharded(tmp_path, ts, 2)
    g = load_safetensor(str(tmp_path))          # directory: the index is preferred
    assert g.sharded and g.total_size == total and len(g.files) == 2
    for k, v in ts.items():
        np.testing.assert_array_equal(g.get_layer(k).numpy(), v.numpy())
    g.close()
    with open(tmp_path / "model.safetensors.index.json", "w") as fh:
        json.dump({"weight_map": {"t0": "model-00001-of-00002.safetensors", "zz": "model-00001-of-00002.safetensors"}}, fh)
    with pytest.raises(ValueError, match="Layer not found in shard model-00001-of-00002.safetensors: zz"):
        load_safetensor(str(tmp_path / "model.safetensors.index.json"))
    with open(tmp_path / "model.safetensors.index.json", "w") as fh:
        json.dump({"weights": {}}, fh)
    with pytest.raises(ValueError, match="weight_map must be an object"):
        load_safetensor(str(tmp_path / "model.safetensors.index.json"))


def _tiny_cfg(**kw):
    base = dict(vocab_size=64, hidden_size=32, intermediate_size=48, num_hidden_layers=2, num_attention_heads=2,
                num_key_value_heads=1, head_dim=32)
    base.update(kw)
    return Qwen3Config(**base)


def test_qwen3_checkpoint_mapping(tmp_path):
    cfg = _tiny_cfg()
    w = init_qwen3_weights(cfg, seed=3)
    path = str(tmp_path / "model.safetensors")
    save_file({k: _bf16_tensor(v) for k, v in w.items()}, path)
    with load_safetensor(path) as g:
        got, res = qwen3_weights_from_safetensor(g, cfg)
        assert sorted(res.loaded_keys) == sorted(w) and not res.missing_keys and not res.unexpected_keys
        for k in w:
            np.testing.assert_array_equal(got[k], w[k])
        del got
    # a missing key and an unexpected key: strict raises with the reference's message, non-strict reports
    w2 = dict(w)
    w2.pop("model.layers.1.mlp.up_proj.weight")
    w2["model.rotary.inv_freq"] = np.zeros(4, np.uint16)
    save_file({k: _bf16_tensor(v) for k, v in w2.items()}, path)
    with load_safetensor(path) as g:
        with pytest.raises(ValueError, match=r"Missing keys: \[model.layers.1.mlp.up_proj.weight\]\n"
                                             r"  Unexpected keys: \[model.rotary.inv_freq\]"):
            qwen3_weights_from_safetensor(g, cfg)
        _, res = qwen3_weights_from_safetensor(g, cfg, strict=False)
        assert res.missing_keys == ["model.layers.1.mlp.up_proj.weight"]
        assert res.unexpected_keys == ["model.rotary.inv_freq"]
    # key_mapper: a checkpoint saved with another prefix
    save_file({"base." + k: _bf16_tensor(v) for k, v in w.items()}, path)
    with load_safetensor(path) as g:
        _, res = qwen3_weights_from_safetensor(g, cfg, key_mapper=lambda k: k[len("base."):])
        assert len(res.loaded_keys) == len(w)
    # a tied model may store lm_head.weight (ignored); an untied one requires it
    save_file({**{k: _bf16_tensor(v) for k, v in w.items()},
               "lm_head.weight": _bf16_tensor(w["model.embed_tokens.weight"][::-1].copy())}, path)
    with load_safetensor(path) as g:
        got, res = qwen3_weights_from_safetensor(g, cfg)
        assert "lm_head.weight" not in got and not res.unexpected_keys
        got, res = qwen3_weights_from_safetensor(g, _tiny_cfg(tie_word_embeddings=False))
        np.testing.assert_array_equal(got["lm_head.weight"], w["model.embed_tokens.weight"][::-1])
        del got
    # shape mismatch
    w3 = dict(w)
    w3["model.norm.weight"] = np.zeros(31, np.uint16)
    save_file({k: _bf16_tensor(v) for k, v in w3.items()}, path)
    with load_safetensor(path) as g:
        with pytest.raises(ValueError, match=r"model.norm.weight: checkpoint shape \[31\] does not match"):
            qwen3_weights_from_safetensor(g, cfg)


def test_qwen3_config_from_hf_json(tmp_path):
    d = {"architectures": ["Qwen3ForCausalLM"], "hidden_size": 1024, "intermediate_size": 3072,
         "num_hidden_layers": 28, "num_attention_heads": 16, "num_key_value_heads": 8, "head_dim": 128,
         "rms_norm_eps": 1e-6, "rope_theta": 1000000, "vocab_size": 151936, "tie_word_embeddings": True,
         "max_position_embeddings": 40960, "torch_dtype": "bfloat16"}
    with open(tmp_path / "config.json", "w") as fh:
        json.dump(d, fh)
    assert Qwen3Config.from_json_file(str(tmp_path / "config.json")) == Qwen3Config()


def test_save_safetensors_round_trip(tmp_path):
    """save_safetensors writes what both this loader and the safetensors package read back
    bit for bit: bf16 bit patterns, float32, int32, an empty tensor and the metadata map, with the
    header padded to 8 bytes and no gaps in the data area."""
    from safetensors.torch import load_file

    from kandle_amd.io import save_safetensors

    rng = np.random.default_rng(5)
    t = {"w.bf16": rng.integers(0, 1 << 16, (7, 5), dtype=np.uint16),
         "b.f32": rng.standard_normal(9).astype(np.float32),
         "ids.i32": np.array([3, -1, 151935], np.int32),
         "empty": np.zeros((0, 4), np.float32)}
    p = str(tmp_path / "m.safetensors")
    save_safetensors(p, t, metadata={"format": "pt"})
    with open(p, "rb") as f:
        n = parse_header_size(f.read(8))
    assert n % 8 == 0
    g = load_safetensor(p)
    assert g.metadata == {"format": "pt"}
    want = {"w.bf16": "bfloat16", "b.f32": "float32", "ids.i32": "int32", "empty": "float32"}
    for k, v in t.items():
        np.testing.assert_array_equal(host_array(g.layers[k], want[k]), v)
    r = load_file(p)
    assert r["w.bf16"].dtype == torch.bfloat16
    np.testing.assert_array_equal(r["w.bf16"].view(torch.int16).numpy().view(np.uint16), t["w.bf16"])
    np.testing.assert_array_equal(r["b.f32"].numpy(), t["b.f32"])
    np.testing.assert_array_equal(r["ids.i32"].numpy(), t["ids.i32"])
    with pytest.raises(ValueError, match="no safetensors dtype"):
        save_safetensors(str(tmp_path / "bad.safetensors"), {"x": np.zeros(2, np.complex64)})
