"""Python binding of include/yue2_hip.h, shaped like the reference's Rust API.

Model.open / Model.forward / Model.forward_phase / Model.prefill_phase /
Cache / Sampling / generate mirror src/model.rs and src/sampling.rs; errors
raise Yue2Error carrying the library's code and message (the reference's
InvalidData errors).  Everything runs on the HIP library; there is no CPU
path, and loading fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libyue2_hip.so"

PHASE_NONE, PHASE_ABC, PHASE_SEMANTIC = 0, 1, 2
ERRORS = {
    -1: "AR input exceeds cache/model context",
    -2: "Token outside model vocabulary",
    -3: "Vocabulary does not support native music protocol",
    -4: "Model produced invalid logits",
    -5: "Empty sampling distribution",
    -6: "Invalid sampling configuration",
    -7: "Prefix + requested generation budget exceeds 24576",
    -8: "Guidance requires negative prefix",
    -9: "Incomplete codec vocabulary",
    -10: "allocation failed",
    -11: "Invalid transformer configuration",
    -12: "device error",
    -13: "invalid argument",
    -14: "top-k survivors exceed the device sort capacity",
}


class Yue2Error(RuntimeError):
    def __init__(self, code: int, message: str = ""):
        self.code = code
        super().__init__(f"{message or ERRORS.get(code, 'error')} (code {code})")


class _Config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
        "head_dim", "intermediate_size", "vocab_size", "max_position_embeddings")] + [
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float)]


class _LayerWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj",
        "input_layernorm", "q_norm", "k_norm", "post_attention_layernorm")]


class _NarWeights(C.Structure):
    _fields_ = [("latent_dim", C.c_int32), ("max_latent_frames", C.c_int32), ("timestep_shift", C.c_float)] + [
        (n, C.c_void_p) for n in ("vae2llm", "llm2vae", "time_in", "time_out", "latent_pos", "vae2llm_bias",
                                  "llm2vae_bias", "time_in_bias", "time_out_bias")] + [
        ("layers", C.POINTER(_LayerWeights))]


class _Sampling(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int32),
                ("repetition_penalty", C.c_float), ("penalty_window", C.c_int32),
                ("min_tokens", C.c_int32), ("max_tokens", C.c_int32)]


class _GpuWeight(C.Structure):
    _fields_ = [("raw", C.c_void_p), ("mapping", C.c_size_t), ("rows", C.c_size_t),
                ("cols", C.c_size_t), ("dtype", C.c_int32), ("rounded", C.c_int32)]


class _GpuLayer(C.Structure):
    _fields_ = [("weights", _GpuWeight * 7), ("norms", C.c_void_p * 4), ("key", C.c_void_p),
                ("value", C.c_void_p)]


_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    """Load libyue2_hip.so (built by yue2_rs_amd.build); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FileNotFoundError(f"{LIB_PATH} is missing: run python -m yue2_rs_amd.build")
    L = C.CDLL(str(LIB_PATH))
    vp, i32, u64, sz, f32 = C.c_void_p, C.c_int32, C.c_uint64, C.c_size_t, C.c_float
    sig = {
        "yue2_hip_available": (i32, []),
        "yue2_hip_vector_default": (i32, []),
        "yue2_hip_name": (C.c_char_p, []),
        "yue2_physical_memory": (u64, []),
        "yue2_hip_vector": (i32, [vp, vp, sz, i32, i32, i32, vp, sz, sz]),
        "yue2_hip_ar_stack": (i32, [vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, sz, sz, sz, f32, vp, vp]),
        "yue2_hip_cached_attention": (i32, [vp, vp, vp, vp, sz, sz, sz, sz, sz, sz]),
        "yue2_hip_gemm": (i32, [vp, vp, vp, sz, sz, sz, i32, sz, sz, sz, C.c_float]),
        "yue2_hip_linear": (i32, [vp, vp, sz, i32, i32, vp, sz, sz, sz]),
        "yue2_hip_attention": (i32, [vp, vp, vp, vp, sz, sz, sz, sz, sz, C.c_int64, C.c_float]),
        "yue2_hip_release_cache": (None, [sz]),
        "yue2_hip_clear_weights": (None, []),
        "yue2_hip_release_model": (None, []),
        "yue2_hip_config_validate": (i32, [vp]),
        "yue2_hip_sampling_validate": (i32, [vp]),
        "yue2_hip_model_open": (vp, [vp, vp, vp, vp, vp]),
        "yue2_hip_model_open_dir": (vp, [C.c_char_p]),
        "yue2_hip_checkpoint_config": (i32, [C.c_char_p, vp]),
        "yue2_hip_model_free": (None, [vp]),
        "yue2_hip_cache_new": (vp, [vp, i32]),
        "yue2_hip_cache_free": (None, [vp]),
        "yue2_hip_cache_length": (i32, [vp]),
        "yue2_hip_cache_load": (i32, [vp, vp, vp, i32, i32]),
        "yue2_hip_cache_export": (i32, [vp, vp, vp, i32, i32, i32]),
        "yue2_hip_model_set_prefill": (i32, [vp, i32]),
        "yue2_hip_forward": (i32, [vp, vp, vp, i32, i32, vp]),
        "yue2_hip_prefill": (i32, [vp, vp, vp, i32, i32, vp]),
        "yue2_hip_prefill_mfma": (i32, [vp, vp, vp, i32, i32, vp]),
        "yue2_hip_nar_load": (i32, [vp, vp]),
        "yue2_hip_velocity": (i32, [vp, vp, vp, i32, C.c_double, i32, vp]),
        "yue2_hip_synthesize": (i32, [vp, vp, i32, vp, i32, C.c_uint64, i32, vp]),
        "yue2_hip_vae_open": (vp, [C.c_char_p]),
        "yue2_hip_vae_free": (None, [vp]),
        "yue2_hip_vae_info": (i32, [vp, vp]),
        "yue2_hip_vae_output_length": (C.c_int64, [vp, i32]),
        "yue2_hip_vae_required_halo": (i32, [vp, i32]),
        "yue2_hip_vae_decode": (i32, [vp, vp, i32, vp]),
        "yue2_hip_vae_decode_tiled": (i32, [vp, vp, i32, i32, i32, vp]),
        "yue2_hip_selftest_conv": (i32, [i32, i32, i32, i32, i32, i32, i32, vp, i32, vp, vp, vp]),
        "yue2_hip_selftest_gemm": (i32, [vp, vp, vp, i32, i32, i32]),
        "yue2_hip_decoder_new": (vp, [vp, vp, vp, vp, u64, i32, f32, i32]),
        "yue2_hip_decoder_free": (None, [vp]),
        "yue2_hip_decoder_run": (i32, [vp, vp, i32, vp, vp]),
        "yue2_hip_decoder_logits": (i32, [vp, vp]),
        "yue2_hip_generate": (i32, [vp, vp, i32, vp, u64, i32, vp, i32, f32, i32, vp, vp, vp]),
        "yue2_hip_choose": (i32, [vp, i32, vp, vp, i32, i32, i32, i32, vp, vp]),
        "yue2_hip_choose_noalloc": (i32, [vp, i32, vp, vp, i32, i32, i32, i32, vp, vp]),
        "yue2_hip_last_error": (C.c_char_p, []),
        "yue2_hip_synchronize": (i32, []),
        "yue2_hip_synthetic_bf16": (None, [vp, sz, u64, u64, f32, i32]),
        "yue2_hip_selftest_math": (i32, [i32, vp, vp, sz]),
        "yue2_hip_norm_fallbacks": (i32, [vp]),
        "yue2_hip_model_advance_sequence": (i32, [vp, i32]),
        "yue2_hip_decoder_time_kernel": (i32, [vp, i32, i32, vp, vp]),
        "yue2_hip_trace_step": (i32, [vp, vp, vp, i32, vp, i32, vp, vp]),
        "yue2_hip_model_set_step_kernel": (i32, [vp, i32]),
        "yue2_hip_bench_gemv": (i32, [i32, i32, i32, i32, i32, vp, vp]),
        "yue2_hip_bench_attention": (i32, [i32, i32, i32, i32, vp, vp]),
        "yue2_hip_bench_copy": (i32, [C.c_int64, i32, vp]),
        "yue2_hip_bench_gemm": (i32, [i32, i32, i32, i32, i32, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _ptr(a: Optional[np.ndarray]) -> Optional[int]:
    return None if a is None else a.ctypes.data


def _check(code: int) -> int:
    if code < 0:
        raise Yue2Error(code, lib().yue2_hip_last_error().decode())
    return code


def available() -> bool:
    return bool(lib().yue2_hip_available())


def synchronize() -> None:
    _check(lib().yue2_hip_synchronize())


@dataclass
class Config:
    """Config (src/model.rs:11-27) with the reference's defaults."""
    hidden_size: int = 2048
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 6144
    vocab_size: int = 184704
    max_position_embeddings: int = 24576
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6

    def c(self) -> _Config:
        return _Config(**{f: getattr(self, f) for f, _ in _Config._fields_})

    def validate(self) -> None:
        cfg = self.c()
        _check(lib().yue2_hip_config_validate(C.byref(cfg)))

    @classmethod
    def read_dir(cls, path) -> "Config":
        """Config::read plus the checkpoint's header and tensor checks, without
        a device; raises Yue2Error with the reference's message."""
        cfg = _Config()
        _check(lib().yue2_hip_checkpoint_config(str(path).encode(), C.byref(cfg)))
        return cls(**{f: getattr(cfg, f) for f, _ in _Config._fields_})


@dataclass
class Sampling:
    """Sampling (src/protocol.rs:143-165) with Sampling::default values."""
    temperature: float = 1.0
    top_p: float = 0.95
    top_k: int = 100
    repetition_penalty: float = 1.2
    penalty_window: int = 50
    min_tokens: int = 200
    max_tokens: int = 9000

    def c(self) -> _Sampling:
        return _Sampling(self.temperature, self.top_p, self.top_k, self.repetition_penalty,
                         self.penalty_window, self.min_tokens, self.max_tokens)

    def validate(self) -> None:
        """Sampling::validate (src/protocol.rs:191-207): raises Yue2Error(-6)."""
        s = self.c()
        _check(lib().yue2_hip_sampling_validate(C.byref(s)))


@dataclass
class LayerWeights:
    q_proj: np.ndarray
    k_proj: np.ndarray
    v_proj: np.ndarray
    o_proj: np.ndarray
    gate_proj: np.ndarray
    up_proj: np.ndarray
    down_proj: np.ndarray
    input_layernorm: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray
    post_attention_layernorm: np.ndarray


@dataclass
class NarWeights:
    """Host weights of the NAR (acoustic) pathway (Model::open,
    src/model.rs:418-451): per layer the AR layer's tensor set, the linears
    vae2llm [H, latent], llm2vae [latent, H], time_embedder.mlp.0 [H, 256]
    and .2 [H, H] as uint16 BF16 arrays with float32 biases, and
    latent_pos_embed.pe [max_latent_frames, H] as uint16 BF16."""
    latent_dim: int
    max_latent_frames: int
    timestep_shift: float
    vae2llm: np.ndarray
    vae2llm_bias: np.ndarray
    llm2vae: np.ndarray
    llm2vae_bias: np.ndarray
    time_in: np.ndarray
    time_in_bias: np.ndarray
    time_out: np.ndarray
    time_out_bias: np.ndarray
    latent_pos: np.ndarray
    layers: list = field(default_factory=list)


@dataclass
class Checkpoint:
    """Host weights of one AR model: BF16 matrices as uint16 arrays [out, in],
    norm gammas as float32 arrays."""
    config: Config
    embed_tokens: np.ndarray
    lm_head: np.ndarray
    final_norm: np.ndarray
    layers: list = field(default_factory=list)


class Model:
    """Model (src/model.rs:398-610) with device-resident weights."""

    def __init__(self, handle: int, config: Config, checkpoint: Checkpoint):
        self._h = handle
        self.config = config
        self._ckpt = checkpoint  # host arrays stay alive with the model

    @classmethod
    def open(cls, checkpoint: Checkpoint) -> "Model":
        L = lib()
        cfg = checkpoint.config.c()
        layers = (_LayerWeights * len(checkpoint.layers))()
        for i, w in enumerate(checkpoint.layers):
            for f, _ in _LayerWeights._fields_:
                setattr(layers[i], f, _ptr(getattr(w, f)))
        h = L.yue2_hip_model_open(C.byref(cfg), _ptr(checkpoint.embed_tokens), _ptr(checkpoint.lm_head),
                                  _ptr(checkpoint.final_norm), layers)
        if not h:
            raise Yue2Error(-12, L.yue2_hip_last_error().decode())
        return cls(h, checkpoint.config, checkpoint)

    @classmethod
    def open_dir(cls, path) -> "Model":
        """Model::open from a checkpoint directory (config.json + safetensors)."""
        L = lib()
        h = L.yue2_hip_model_open_dir(str(path).encode())
        if not h:
            raise Yue2Error(-11, L.yue2_hip_last_error().decode())
        cfg = _Config()
        _check(L.yue2_hip_checkpoint_config(str(path).encode(), C.byref(cfg)))
        config = Config(**{f: getattr(cfg, f) for f, _ in _Config._fields_})
        return cls(h, config, None)

    def close(self) -> None:
        """Model's Drop.  Its caches and decoders may be closed before or
        after it (the library detaches them): a detached decoder's calls
        raise, a detached cache can still be exported."""
        if self._h:
            lib().yue2_hip_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward_phase(self, ids: Sequence[int], cache: "Cache", phase: int = PHASE_NONE) -> np.ndarray:
        """Model::forward_phase: logits of the last row (vocab_size f32)."""
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.config.vocab_size, dtype=np.float32)
        _check(lib().yue2_hip_forward(self._h, cache._h, _ptr(arr), len(arr), phase, _ptr(out)))
        return out

    def forward(self, ids: Sequence[int], cache: "Cache") -> np.ndarray:
        """Model::forward (full vocabulary head)."""
        return self.forward_phase(ids, cache, PHASE_NONE)

    def prefill_phase(self, ids: Sequence[int], capacity: int, phase: int = PHASE_NONE):
        """Model::prefill_phase: (Cache, logits of the last prompt row)."""
        cache = Cache(self, capacity)
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.config.vocab_size, dtype=np.float32)
        _check(lib().yue2_hip_prefill(self._h, cache._h, _ptr(arr), len(arr), phase, _ptr(out)))
        return cache, out

    def prefill_mfma(self, ids: Sequence[int], capacity: int, phase: int = PHASE_NONE):
        """Model::prefill_phase on the matrix cores (MFMA GEMMs + flash
        attention): (Cache, logits of the last prompt row).  Agrees with
        prefill_phase within a tolerance, not bit for bit."""
        cache = Cache(self, capacity)
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.config.vocab_size, dtype=np.float32)
        _check(lib().yue2_hip_prefill_mfma(self._h, cache._h, _ptr(arr), len(arr), phase, _ptr(out)))
        return cache, out

    def load_nar(self, w: "NarWeights") -> None:
        """Upload the NAR pathway (its host arrays stay referenced by the model)."""
        layers = (_LayerWeights * len(w.layers))()
        for i, lw in enumerate(w.layers):
            for f, _ in _LayerWeights._fields_:
                setattr(layers[i], f, _ptr(getattr(lw, f)))
        s = _NarWeights(w.latent_dim, w.max_latent_frames, w.timestep_shift, _ptr(w.vae2llm), _ptr(w.llm2vae),
                        _ptr(w.time_in), _ptr(w.time_out), _ptr(w.latent_pos), _ptr(w.vae2llm_bias),
                        _ptr(w.llm2vae_bias), _ptr(w.time_in_bias), _ptr(w.time_out_bias), layers)
        _check(lib().yue2_hip_nar_load(self._h, C.byref(s)))
        self._nar = w

    def velocity(self, state: np.ndarray, cache: "Cache", raw_t: float, nar_cond_end: int = 0) -> np.ndarray:
        """Model::velocity (src/model.rs:611-698): state [frames, latent] ->
        [frames, latent], on the matrix cores."""
        st = np.ascontiguousarray(state, dtype=np.float32)
        out = np.empty_like(st)
        _check(lib().yue2_hip_velocity(self._h, cache._h, _ptr(st), st.shape[0], raw_t, nar_cond_end, _ptr(out)))
        return out

    def synthesize(self, prefix: Sequence[int], codec: Sequence[int], seed: int, steps: int) -> np.ndarray:
        """Model::synthesize (src/model.rs:699-775): [len(codec), 64] latents."""
        p = np.ascontiguousarray(prefix, dtype=np.int32)
        cd = np.ascontiguousarray(codec, dtype=np.int32)
        out = np.empty((len(cd), 64), np.float32)
        _check(lib().yue2_hip_synthesize(self._h, _ptr(p), len(p), _ptr(cd), len(cd), seed, steps, _ptr(out)))
        return out

    def set_step_kernel(self, on: bool) -> bool:
        """Use the persistent token-step kernel for decode steps; returns
        whether it is in use (False when the shape has none)."""
        return bool(_check(lib().yue2_hip_model_set_step_kernel(self._h, 1 if on else 0)))

    def set_prefill_mfma(self, on: bool) -> bool:
        """generate() prefills its prompts on the matrix cores (True) or in
        decode order (False, the default, bit-exact); returns the setting."""
        return bool(_check(lib().yue2_hip_model_set_prefill(self._h, 1 if on else 0)))

    def advance_sequence(self, add: int) -> None:
        """Diagnostics: advance the launch sequence of the model's forward
        workspace by `add` (the step kernel's tagged-word epoch)."""
        _check(lib().yue2_hip_model_advance_sequence(self._h, int(add)))

    def norm_fallbacks(self) -> int:
        return int(lib().yue2_hip_norm_fallbacks(self._h))

    def trace_step(self, token: int, cache: "Cache", cache2: Optional["Cache"] = None) -> np.ndarray:
        """One decode step through the persistent step kernel with phase
        stamps: uint64 array [slot, workgroup] of the device wall clock
        (100 MHz); slot 0 = start, then 15 per layer (see yue2_hip.h).
        cache2: a batch-2 step over both caches."""
        cap = (1 + 15 * self.config.num_hidden_layers) * 1024
        out = np.zeros(cap, dtype=np.uint64)
        wgs, slots = C.c_int32(0), C.c_int32(0)
        _check(lib().yue2_hip_trace_step(self._h, cache._h, None if cache2 is None else cache2._h, int(token),
                                         _ptr(out), cap, C.byref(wgs), C.byref(slots)))
        return out[: slots.value * wgs.value].reshape(slots.value, wgs.value)


class Cache:
    """Cache::new (src/model.rs:292-305): a device BF16 KV cache."""

    def __init__(self, model: Model, capacity: int):
        self.model = model
        self._h = lib().yue2_hip_cache_new(model._h, capacity)
        if not self._h:
            raise Yue2Error(-10, lib().yue2_hip_last_error().decode())
        self.capacity = capacity

    @property
    def length(self) -> int:
        return int(lib().yue2_hip_cache_length(self._h))

    def load(self, key: np.ndarray, value: np.ndarray, length: int) -> None:
        """Fill the device context from a host K/V mirror (per layer, rows of
        kv_heads * head_dim BF16-exact f32): key/value shaped [layers, stride,
        width] with stride >= length; the cache length becomes `length`."""
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        if k.shape != v.shape or k.ndim != 3:
            raise ValueError("key and value must both be [layers, stride, width]")
        _check(lib().yue2_hip_cache_load(self._h, _ptr(k), _ptr(v), int(length), k.shape[1]))

    def export(self, start: int = 0, n: Optional[int] = None, stride: Optional[int] = None):
        """The host K/V mirror of rows [start, start + n) (default: the whole
        length): (key, value), each [layers, stride, kv_heads * head_dim] f32
        with those rows filled (the rest zero)."""
        cfg = self.model.config
        n = self.length - start if n is None else n
        stride = start + n if stride is None else stride
        shape = (cfg.num_hidden_layers, stride, cfg.num_key_value_heads * cfg.head_dim)
        k, v = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
        _check(lib().yue2_hip_cache_export(self._h, _ptr(k), _ptr(v), int(start), int(n), int(stride)))
        return k, v

    def close(self) -> None:
        if self._h:
            lib().yue2_hip_cache_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Vae:
    """The VAE decoder (src/vae.rs:611-762) on the device."""

    def __init__(self, path):
        L = lib()
        self._h = L.yue2_hip_vae_open(str(path).encode())
        if not self._h:
            raise Yue2Error(-11, L.yue2_hip_last_error().decode())
        info = np.zeros(6, np.int32)
        _check(L.yue2_hip_vae_info(self._h, _ptr(info)))
        (self.sample_rate, self.latent_dim, self.audio_channels, self.downsampling_ratio, self.core_frames,
         self.halo_frames) = (int(v) for v in info)

    def output_length(self, frames: int) -> int:
        return _check(int(lib().yue2_hip_vae_output_length(self._h, frames)))

    def required_halo(self, core: int) -> int:
        return _check(lib().yue2_hip_vae_required_halo(self._h, core))

    def decode(self, z: np.ndarray) -> np.ndarray:
        z = np.ascontiguousarray(z, dtype=np.float32)
        out = np.empty((max(self.output_length(z.shape[0]), 0), self.audio_channels), np.float32)
        _check(lib().yue2_hip_vae_decode(self._h, _ptr(z), z.shape[0], _ptr(out)))
        return out

    def decode_tiled(self, z: np.ndarray, core: int, halo: int) -> np.ndarray:
        z = np.ascontiguousarray(z, dtype=np.float32)
        out = np.empty((max(self.output_length(z.shape[0]), 0), self.audio_channels), np.float32)
        _check(lib().yue2_hip_vae_decode_tiled(self._h, _ptr(z), z.shape[0], core, halo, _ptr(out)))
        return out

    def close(self) -> None:
        if self._h:
            lib().yue2_hip_vae_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Decoder:
    """The captured token loop (one hipGraph launch per step)."""

    def __init__(self, model: Model, cond: Cache, uncond: Optional[Cache] = None,
                 sampling: Optional[Sampling] = None, seed: int = 0, phase: int = PHASE_NONE,
                 scale: float = 1.0, legacy: bool = False):
        self.model = model
        self._caches = (cond, uncond)
        s = sampling.c() if sampling is not None else None
        self._h = lib().yue2_hip_decoder_new(model._h, cond._h, uncond._h if uncond else None,
                                             C.byref(s) if s is not None else None, seed, phase,
                                             scale, int(legacy))
        if not self._h:
            raise Yue2Error(-13, lib().yue2_hip_last_error().decode())
        self.rows = 2 if scale != 1.0 else 1

    def run(self, steps: int, first_logits: Optional[np.ndarray] = None, timing: bool = False):
        """Run `steps` steps; returns (tokens, step_ms or None)."""
        fl = None
        if first_logits is not None:
            fl = np.ascontiguousarray(first_logits, dtype=np.float32)
        tokens = np.zeros(max(steps, 1), dtype=np.int32)
        ms = np.zeros(max(steps, 1), dtype=np.float32) if timing else None
        n = _check(lib().yue2_hip_decoder_run(self._h, _ptr(fl), steps, _ptr(tokens), _ptr(ms)))
        return tokens[:n], (ms[:n] if timing else None)

    def logits(self) -> np.ndarray:
        """The logits of the last forward (which the next token's choice
        read; the first logits before any forward): [rows, vocab],
        conditional row first."""
        out = np.empty((self.rows, self.model.config.vocab_size), dtype=np.float32)
        _check(lib().yue2_hip_decoder_logits(self._h, _ptr(out)))
        return out

    KERNELS = {"gate_up": 0, "down": 1, "qkv": 2, "o": 3, "lm_head": 4, "step": 5}

    def time_kernel(self, kernel: str, iters: int = 112):
        """(mean launch ms, algorithmic bytes per launch) of one of the
        decoder's kernels (a per-phase GEMV, or "step": the persistent
        step kernel), timed with HIP events on its stream."""
        ms, by = C.c_float(0), C.c_double(0)
        _check(lib().yue2_hip_decoder_time_kernel(self._h, self.KERNELS[kernel], iters, C.byref(ms),
                                                  C.byref(by)))
        return float(ms.value), float(by.value)

    def close(self) -> None:
        if self._h:
            lib().yue2_hip_decoder_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass
class Generated:
    tokens: list
    truncated: bool


def choose(logits: np.ndarray, sampling: Sampling, history: Sequence[int] = (), step: int = 0,
           phase: int = PHASE_NONE, legacy: bool = False, draws: Optional[np.ndarray] = None,
           noalloc: bool = False) -> int:
    """sampling::choose (src/sampling.rs:103-215) on the device for one row of
    logits.  draws: the 2 * vocab MT19937 outputs the call consumes (needed
    unless temperature is 0).  noalloc: through yue2_hip_choose_noalloc (no
    device allocation; vocabularies up to 262144)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(history, dtype=np.int32)
    d = None if draws is None else np.ascontiguousarray(draws, dtype=np.uint32)
    if d is not None and len(d) != 2 * len(lg):
        raise ValueError("draws must hold 2 * vocab outputs")
    out = C.c_int32(-1)
    s = sampling.c()
    fn = lib().yue2_hip_choose_noalloc if noalloc else lib().yue2_hip_choose
    _check(fn(_ptr(lg), len(lg), C.byref(s), _ptr(h) if len(h) else None, len(h), step, phase, int(legacy),
              _ptr(d), C.byref(out)))
    return out.value


def generate(model: Model, prefix: Sequence[int], sampling: Sampling, seed: int,
             phase: int = PHASE_NONE, negative: Optional[Sequence[int]] = None,
             scale: float = 1.0, legacy: bool = False) -> Generated:
    """sampling::generate (src/sampling.rs:222-294) on the device."""
    p = np.ascontiguousarray(prefix, dtype=np.int32)
    n = None if negative is None else np.ascontiguousarray(negative, dtype=np.int32)
    out = np.zeros(max(sampling.max_tokens, 1), dtype=np.int32)
    count, trunc = C.c_int32(0), C.c_int32(0)
    s = sampling.c()
    _check(lib().yue2_hip_generate(model._h, _ptr(p), len(p), C.byref(s), seed, phase, _ptr(n),
                                   0 if n is None else len(n), scale, int(legacy), _ptr(out),
                                   C.byref(count), C.byref(trunc)))
    return Generated(out[:count.value].tolist(), bool(trunc.value))
