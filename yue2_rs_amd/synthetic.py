"""Synthetic checkpoints and prompts for the benchmark configurations.

The real YuE2 checkpoint is downloaded by the reference and is not available
offline, so the benchmark models are random-init: BF16 weights ~N(0, 0.02)
from the library's counter-based generator, all norm gammas 1.  Prompts are
uniform token ids from MT19937 (the reference's generator,
src/sampling.rs:10-42): id = next_u32() mod vocab.
"""
from __future__ import annotations

import numpy as np

from .api import Checkpoint, Config, LayerWeights, NarWeights, lib

# Tensor ids of the generator (one independent stream per tensor).
EMBED, LM_HEAD, LAYER_BASE, PER_LAYER = 0, 1, 16, 8
NAR_BASE = 1 << 16  # the NAR pathway's tensors
PROJECTIONS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

REDUCED = Config(hidden_size=1024, num_hidden_layers=2, num_attention_heads=16, num_key_value_heads=4,
                 head_dim=64, intermediate_size=2816, vocab_size=32768, max_position_embeddings=24576,
                 rms_norm_eps=1e-6, rope_theta=10000.0)
CLASS_3B = Config(hidden_size=3072, num_hidden_layers=28, num_attention_heads=24, num_key_value_heads=8,
                  head_dim=128, intermediate_size=8192, vocab_size=84000, max_position_embeddings=24576,
                  rms_norm_eps=1e-6, rope_theta=10000.0)


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
