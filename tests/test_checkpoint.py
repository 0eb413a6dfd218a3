"""The checkpoint loader's checks (Config::read, src/model.rs:29-73;
Weights::open, src/checkpoint.rs:310-386; Weights::checked, :405-409)
through yue2_hip_checkpoint_config, which needs no device: valid single-file
and sharded checkpoints, then each malformed case the reference rejects,
with its message."""
import json
import struct

import numpy as np
import pytest

from yue2_rs_amd import synthetic
from yue2_rs_amd.api import Config, Yue2Error

from ckpt_files import ar_tensors, config_json, safetensors_bytes, write_checkpoint

SMALL = Config(hidden_size=64, num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1, head_dim=64,
               intermediate_size=128, vocab_size=300, max_position_embeddings=512, rms_norm_eps=1e-6,
               rope_theta=1e6)


@pytest.fixture(scope="module")
def ck():
    return synthetic.checkpoint(SMALL, seed=1)


@pytest.mark.parametrize("dtype,shards", [("BF16", 1), ("F32", 1), ("F16", 3), ("BF16", 4)])
def test_valid_checkpoints_read(tmp_path, ck, dtype, shards):
    d = write_checkpoint(tmp_path / "m", ck, dtype=dtype, shards=shards)
    got = Config.read_dir(d)
    f32 = lambda c: [np.float32(v) if isinstance(v, float) else v for v in vars(c).values()]
    assert f32(got) == f32(SMALL)


def test_defaults_of_missing_config_fields(tmp_path, ck):
    """Absent fields take Config::read's defaults (src/model.rs:35-48)."""
    cfg = config_json(SMALL)
    del cfg["rope_theta"], cfg["model_type"], cfg["latent_type"]
    d = write_checkpoint(tmp_path / "m", ck, config=cfg)
    assert Config.read_dir(d).rope_theta == 1e6


def _err(d):
    with pytest.raises(Yue2Error) as e:
        Config.read_dir(d)
    return str(e.value)


def test_rejections(tmp_path, ck):
    ts = ar_tensors(ck)
    # a missing tensor, a wrong shape
    d = write_checkpoint(tmp_path / "a", ck, tensors=[t for t in ts if t[0] != "model.layers.1.mlp.up_proj.weight"])
    assert "Missing checkpoint tensor model.layers.1.mlp.up_proj.weight" in _err(d)
    bad = [(n, dt, (sh[1], sh[0]) if n == "lm_head.weight" else sh, b) for n, dt, sh, b in ts]
    d = write_checkpoint(tmp_path / "b", ck, tensors=bad)
    assert "Tensor lm_head.weight: expected [300, 64], found [64, 300]" in _err(d)
    # an unsupported dtype
    bad = [(n, "I8" if n == "model.norm.weight" else dt, sh, b) for n, dt, sh, b in ts]
    d = write_checkpoint(tmp_path / "c", ck, tensors=bad)
    assert "Unsupported dtype I8 for model.norm.weight" in _err(d)
    # the model type and an invalid configuration
    d = write_checkpoint(tmp_path / "d", ck, config=config_json(SMALL, model_type="llama"))
    assert "Expected YuE2 VAE-latent model" in _err(d)
    d = write_checkpoint(tmp_path / "e", ck, config=config_json(SMALL, num_key_value_heads=3))
    assert "Invalid transformer configuration" in _err(d)


@pytest.mark.parametrize("field,value,message", [
    ("latent_dim", 0, "Invalid transformer configuration"),
    ("max_latent_frames", 0, "Invalid transformer configuration"),
    ("timestep_shift", 0.0, "Invalid transformer configuration"),
    ("timestep_shift", -1.5, "Invalid transformer configuration"),
    ("model_type", 7, "Expected JSON string"),
    ("latent_type", ["vae"], "Expected JSON string"),
    ("hidden_size", "64", "Expected unsigned JSON integer"),
    ("rope_theta", True, "Expected JSON number"),
    ("tie_word_embeddings", 1, "Expected JSON boolean"),
])
def test_config_field_rejections(tmp_path, ck, field, value, message):
    """Config::read's other checks (src/model.rs:44-71) and the JSON kind
    errors of its accessors (src/json.rs:26-80): a present key of the wrong
    kind is an error, never its default."""
    d = write_checkpoint(tmp_path / "m", ck, config=config_json(SMALL, **{field: value}))
    assert message in _err(d)


def test_config_nonfinite_timestep_shift(tmp_path, ck):
    d = write_checkpoint(tmp_path / "m", ck)
    text = (d / "config.json").read_text()
    (d / "config.json").write_text(text[:-1] + ', "timestep_shift": 1e999}')
    assert "Invalid transformer configuration" in _err(d)


def test_malformed_files(tmp_path, ck):
    ts = ar_tensors(ck)
    d = write_checkpoint(tmp_path / "a", ck)
    (d / "model.safetensors").write_bytes(b"\x01\x02")
    assert "Short safetensors file" in _err(d)
    (d / "model.safetensors").write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    assert "Invalid safetensors header size" in _err(d)
    # a tensor whose extent disagrees with its shape, and two that overlap
    raw = bytearray(safetensors_bytes(ts))
    hlen = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + hlen])
    header["model.norm.weight"]["data_offsets"][1] += 4
    h = json.dumps(header).encode()
    (d / "model.safetensors").write_bytes(struct.pack("<Q", len(h)) + h + raw[8 + hlen:])
    assert "Invalid tensor extent model.norm.weight" in _err(d)
    header = json.loads(raw[8:8 + hlen])
    a = header["model.layers.0.input_layernorm.weight"]["data_offsets"]
    header["model.layers.0.q_norm.weight"] = {"dtype": "F32", "shape": [16], "data_offsets": [a[0], a[0] + 64]}
    h = json.dumps(header).encode()
    (d / "model.safetensors").write_bytes(struct.pack("<Q", len(h)) + h + raw[8 + hlen:])
    assert "Overlapping safetensors tensors" in _err(d)
    # a shard path outside the directory
    d2 = write_checkpoint(tmp_path / "b", ck, shards=2)
    idx = json.loads((d2 / "model.safetensors.index.json").read_text())
    idx["weight_map"]["lm_head.weight"] = "../model.safetensors"
    (d2 / "model.safetensors.index.json").write_text(json.dumps(idx))
    assert "Invalid shard path" in _err(d2)
