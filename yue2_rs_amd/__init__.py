"""yue2_rs_amd -- MI355X (gfx950) implementation of YuE2's autoregressive
decode step behind the reference's model-step API, with the matrix-core
prefill, the NAR velocity stack and the VAE decoder around it.

The compute path is libyue2_hip.so (hand-written HIP kernels, C ABI in
include/yue2_hip.h); this package binds it with ctypes.
"""
from .api import (PHASE_ABC, PHASE_NONE, PHASE_SEMANTIC, Cache, Checkpoint, Config, Decoder,
                  Generated, LayerWeights, Model, NarWeights, Sampling, Vae, Yue2Error, available, choose,
                  generate, lib, synchronize)

__all__ = ["PHASE_ABC", "PHASE_NONE", "PHASE_SEMANTIC", "Cache", "Checkpoint", "Config", "Decoder",
           "Generated", "LayerWeights", "Model", "NarWeights", "Sampling", "Vae", "Yue2Error", "available",
           "choose", "generate", "lib", "synchronize"]
