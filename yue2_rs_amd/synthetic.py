"""Synthetic checkpoints and prompts for the benchmark configurations.

The real YuE2 checkpoint is downloaded by the reference and is not available
offline, so the benchmark models are random-init: BF16 weights ~N(0, 0.02)
from the library's counter-based generator, all norm gammas 1.  Prompts are
uniform token ids from MT19937 (the reference's generator,
src/sampling.rs:10-42): id = next_u32() mod vocab.  VAE decoders are written
as checkpoint directories in the layout Vae::open reads (src/vae.rs:635-669)
with numpy-generated FP32 weights.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

from .api import Checkpoint, Config, LayerWeights, NarWeights, lib

# Tensor ids of the generator (one independent stream per tensor).
EMBED, LM_HEAD, LAYER_BASE, PER_LAYER = 0, 1, 16, 8
NAR_BASE = 1 << 16  # the NAR pathway's tensors
PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

REDUCED = Config(hidden_size=1024, num_hidden_layers=2, num_attention_heads=16, num_key_value_heads=4,
                 head_dim=64, intermediate_size=2816, vocab_size=32768, max_position_embeddings=24576,
                 rms_norm_eps=1e-6, rope_theta=10000.0)
# The reference's Config defaults (src/model.rs:35-44): the YuE2 shape.
YUE2 = Config(hidden_size=2048, num_hidden_layers=28, num_attention_heads=16, num_key_value_heads=8,
              head_dim=128, intermediate_size=6144, vocab_size=184704, max_position_embeddings=24576,
              rms_norm_eps=1e-6, rope_theta=1e6)
CLASS_3B = Config(hidden_size=3072, num_hidden_layers=28, num_attention_heads=24, num_key_value_heads=8,
                  head_dim=128, intermediate_size=8192, vocab_size=84000, max_position_embeddings=24576,
                  rms_norm_eps=1e-6, rope_theta=10000.0)
# A 1B-class shape with no step kernel of its own (the generic head_dim-64
# kernel runs it): 4 query heads per KV head, contexts up to 16384.
CLASS_1B_ANY = Config(hidden_size=2048, num_hidden_layers=16, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=64, intermediate_size=8192, vocab_size=128256, max_position_embeddings=16384,
                      rms_norm_eps=1e-6, rope_theta=500000.0)
# An 8B-class shape (the generic head_dim-128 kernel): hidden 4096, 32 x 128
# query heads, 4 per KV head, SwiGLU 14336.
CLASS_8B_ANY = Config(hidden_size=4096, num_hidden_layers=32, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, intermediate_size=14336, vocab_size=128256, max_position_embeddings=16384,
                      rms_norm_eps=1e-6, rope_theta=500000.0)


def bf16_normal(shape, seed: int, tensor: int, std: float = 0.02, threads: int = 0) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    lib().yue2_hip_synthetic_bf16(out.ctypes.data, out.size, seed, tensor, std, threads)
    return out


def shapes(c: Config) -> dict:
    H, D, I = c.hidden_size, c.head_dim, c.intermediate_size
    q, kv = c.num_attention_heads * D, c.num_key_value_heads * D
    return {"q_proj": (q, H), "k_proj": (kv, H), "v_proj": (kv, H), "o_proj": (H, q),
            "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}


def checkpoint(c: Config, seed: int = 0, std: float = 0.02, threads: int = 0) -> Checkpoint:
    """Random-init checkpoint of config c (weights ~N(0, std) in BF16, norms 1)."""
    H, D, V = c.hidden_size, c.head_dim, c.vocab_size
    embed = bf16_normal((V, H), seed, EMBED, std, threads)
    head = bf16_normal((V, H), seed, LM_HEAD, std, threads)
    layers = []
    sh = shapes(c)
    for l in range(c.num_hidden_layers):
        mats = {n: bf16_normal(sh[n], seed, LAYER_BASE + l * PER_LAYER + j, std, threads)
                for j, n in enumerate(PROJECTIONS)}
        layers.append(LayerWeights(**mats, input_layernorm=np.ones(H, np.float32),
                                   q_norm=np.ones(D, np.float32), k_norm=np.ones(D, np.float32),
                                   post_attention_layernorm=np.ones(H, np.float32)))
    return Checkpoint(c, embed, head, np.ones(H, np.float32), layers)


def nar_weights(c: Config, seed: int = 0, std: float = 0.02, latent_dim: int = 64,
                max_latent_frames: int = 24576, timestep_shift: float = 1.0, threads: int = 0) -> NarWeights:
    """Random-init NAR pathway for config c: BF16 weights ~N(0, std), biases
    BF16-exact ~N(0, std) as float32, latent position rows ~N(0, std), norms 1."""
    H, D = c.hidden_size, c.head_dim
    t = iter(range(NAR_BASE, NAR_BASE + 64))

    def mat(shape):
        return bf16_normal(shape, seed, next(t), std, threads)

    def bias(n):
        b = bf16_normal((n,), seed, next(t), std, threads)
        return (b.astype(np.uint32) << 16).view(np.float32)

    layers = []
    sh = shapes(c)
    for l in range(c.num_hidden_layers):
        mats = {n: bf16_normal(sh[n], seed, NAR_BASE + 256 + l * PER_LAYER + j, std, threads)
                for j, n in enumerate(PROJECTIONS)}
        layers.append(LayerWeights(**mats, input_layernorm=np.ones(H, np.float32),
                                   q_norm=np.ones(D, np.float32), k_norm=np.ones(D, np.float32),
                                   post_attention_layernorm=np.ones(H, np.float32)))
    return NarWeights(latent_dim, max_latent_frames, timestep_shift,
                      mat((H, latent_dim)), bias(H), mat((latent_dim, H)), bias(latent_dim),
                      mat((H, 256)), bias(H), mat((H, H)), bias(H), mat((max_latent_frames, H)), layers)


class MT19937:
    """std::mt19937 seeded as src/sampling.rs:15-24."""

    def __init__(self, seed: int):
        s = [0] * 624
        s[0] = seed & 0xFFFFFFFF
        for i in range(1, 624):
            s[i] = (1812433253 * (s[i - 1] ^ (s[i - 1] >> 30)) + i) & 0xFFFFFFFF
        self.s, self.i = s, 624

    def next_u32(self) -> int:
        s = self.s
        if self.i == 624:
            for i in range(624):
                bits = (s[i] & 0x80000000) | (s[(i + 1) % 624] & 0x7FFFFFFF)
                s[i] = s[(i + 397) % 624] ^ (bits >> 1) ^ (0x9908B0DF if bits & 1 else 0)
            self.i = 0
        y = s[self.i]
        self.i += 1
        y ^= y >> 11
        y ^= (y << 7) & 0x9D2C5680
        y ^= (y << 15) & 0xEFC60000
        y ^= y >> 18
        return y


def prompt(n: int, vocab: int, seed: int = 0) -> np.ndarray:
    """n uniform token ids: MT19937(seed).next_u32() mod vocab."""
    g = MT19937(seed)
    return np.array([g.next_u32() % vocab for _ in range(n)], dtype=np.int32)


# An Oobleck decoder at the reference's default downsampling ratio (1920,
# src/vae.rs:643; 48 kHz audio from 25 latent frames per second) with the
# common Oobleck widths 128 x (1, 2, 4, 8, 16).  The YuE2 VAE's own config
# ships with its checkpoint, which is not available offline.
VAE_1920 = dict(channels=128, c_mults=(1, 2, 4, 8, 16), strides=(2, 4, 4, 6, 10), latent=64, out_channels=2,
                core=512, halo=16)


def vae(seed=0, channels=8, c_mults=(2, 4), strides=(2, 4), latent=16, out_channels=2, snake=True,
        final_tanh=True, core=8, halo=6):
    """(config.json dict, {tensor name: FP32 array}) of a random-init decoder
    under the reference's tensor names (network, src/vae.rs:470-546; residual
    units, :427-466): weight-norm pairs with g in [0.5, 1.5), biases
    ~N(0, 0.01), SnakeBeta log-parameters ~N(0, 0.04)."""
    rng = np.random.default_rng(seed)
    cfg = {"model_type": "yue2_vae", "latent_dim": latent, "sample_rate": 48000, "audio_channels": out_channels,
           "downsampling_ratio": int(np.prod(strides)), "decode_core_frames": core, "decode_halo_frames": halo,
           "decoder_config": {"channels": channels, "c_mults": list(c_mults), "strides": list(strides),
                              "latent_dim": latent, "out_channels": out_channels, "use_snake": snake,
                              "final_tanh": final_tanh}}
    t = {}

    def conv(name, cin, cout, k, transpose=False, bias=True):
        shape = (cin, cout, k) if transpose else (cout, cin, k)
        t[f"{name}.weight_v"] = rng.standard_normal(shape).astype(np.float32)
        t[f"{name}.weight_g"] = rng.uniform(0.5, 1.5, (shape[0], 1, 1)).astype(np.float32)
        if bias:
            t[f"{name}.bias"] = (0.1 * rng.standard_normal(cout)).astype(np.float32)

    def act(name, c):
        if snake:
            t[f"{name}.alpha"] = (0.2 * rng.standard_normal(c)).astype(np.float32)
            t[f"{name}.beta"] = (0.2 * rng.standard_normal(c)).astype(np.float32)

    mults = [1] + list(c_mults)
    conv("decoder.layers.0", latent, channels * mults[-1], 7)
    index = 1
    for i in range(len(mults) - 1, 0, -1):
        cin, cout, s = channels * mults[i], channels * mults[i - 1], strides[i - 1]
        p = f"decoder.layers.{index}.layers"
        act(f"{p}.0", cin)
        conv(f"{p}.1", cin, cout, 2 * s, transpose=True)
        for r in (2, 3, 4):
            act(f"{p}.{r}.layers.0", cout)
            conv(f"{p}.{r}.layers.1", cout, cout, 7)
            act(f"{p}.{r}.layers.2", cout)
            conv(f"{p}.{r}.layers.3", cout, cout, 1)
        index += 1
    act(f"decoder.layers.{index}", channels)
    conv(f"decoder.layers.{index + 1}", channels, out_channels, 7, bias=False)
    return cfg, t


def safetensors_bytes(tensors):
    """A safetensors file: tensors is a list of (name, dtype string, shape,
    raw bytes), stored in that order."""
    header, off = {}, 0
    for name, dt, shape, data in tensors:
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        off += len(data)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    return struct.pack("<Q", len(h)) + h + b"".join(d for _, _, _, d in tensors)


def write_vae(directory, cfg, tensors) -> Path:
    """config.json and model.safetensors (FP32) of a VAE decoder."""
    path = Path(directory)
    path.mkdir(parents=True, exist_ok=True)
    (path / "config.json").write_text(json.dumps(cfg))
    items = [(n, "F32", a.shape, np.ascontiguousarray(a, np.float32).tobytes()) for n, a in sorted(tensors.items())]
    (path / "model.safetensors").write_bytes(safetensors_bytes(items))
    return path
