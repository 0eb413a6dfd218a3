"""Write a synthetic checkpoint directory in the layout the reference's
Model::open reads (src/model.rs:418-451, src/checkpoint.rs:310-386):
config.json plus model.safetensors, or shards named by
model.safetensors.index.json.  Tensor names follow the reference's loader."""
import json
import struct
from pathlib import Path

import numpy as np


def safetensors_bytes(tensors):
    """tensors: list of (name, dtype string, shape, raw bytes)."""
    header, blobs, off = {}, [], 0
    for name, dt, shape, data in tensors:
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        off += len(data)
        blobs.append(data)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    return struct.pack("<Q", len(h)) + h + b"".join(blobs)


def ar_tensors(ck, dtype="BF16"):
    """The AR decode path's tensors of a synthetic Checkpoint, as
    (name, dtype, shape, bytes).  dtype F32/F16 stores the BF16 values
    widened (exact), so the loader's rounding gives the same BF16 back."""
    def mat(a):
        if dtype == "BF16":
            return "BF16", a.shape, np.ascontiguousarray(a, np.uint16).tobytes()
        f = (a.astype(np.uint32) << 16).view(np.float32)
        if dtype == "F32":
            return "F32", a.shape, f.tobytes()
        return "F16", a.shape, f.astype(np.float16).tobytes()

    def vec(v):
        return "F32", v.shape, np.ascontiguousarray(v, np.float32).tobytes()

    out = [("model.embed_tokens.weight", *mat(ck.embed_tokens)), ("lm_head.weight", *mat(ck.lm_head)),
           ("model.norm.weight", *vec(ck.final_norm))]
    for i, w in enumerate(ck.layers):
        p = f"model.layers.{i}"
        for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
            out.append((f"{p}.self_attn.{n}.weight", *mat(getattr(w, n))))
        for n in ("gate_proj", "up_proj", "down_proj"):
            out.append((f"{p}.mlp.{n}.weight", *mat(getattr(w, n))))
        out.append((f"{p}.input_layernorm.weight", *vec(w.input_layernorm)))
        out.append((f"{p}.self_attn.q_norm.weight", *vec(w.q_norm)))
        out.append((f"{p}.self_attn.k_norm.weight", *vec(w.k_norm)))
        out.append((f"{p}.post_attention_layernorm.weight", *vec(w.post_attention_layernorm)))
    return out


def config_json(c, **extra):
    d = {"model_type": "yue2", "latent_type": "vae", "hidden_size": c.hidden_size,
         "num_hidden_layers": c.num_hidden_layers, "num_attention_heads": c.num_attention_heads,
         "num_key_value_heads": c.num_key_value_heads, "head_dim": c.head_dim,
         "intermediate_size": c.intermediate_size, "vocab_size": c.vocab_size,
         "max_position_embeddings": c.max_position_embeddings, "rms_norm_eps": c.rms_norm_eps,
         "rope_theta": c.rope_theta, "tie_word_embeddings": False}
    d.update(extra)
    return d


def write_checkpoint(directory, ck, dtype="BF16", shards=1, tensors=None, config=None):
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    (d / "config.json").write_text(json.dumps(config if config is not None else config_json(ck.config)))
    ts = tensors if tensors is not None else ar_tensors(ck, dtype)
    if shards == 1:
        (d / "model.safetensors").write_bytes(safetensors_bytes(ts))
        return d
    weight_map = {}
    for s in range(shards):
        part = ts[s::shards]
        name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        (d / name).write_bytes(safetensors_bytes(part))
        weight_map.update({t[0]: name for t in part})
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    return d
