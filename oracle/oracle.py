"""ctypes binding of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker and the CPU baseline.  The
product (yue2_rs_amd) never imports this module.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"

PHASE_NONE, PHASE_ABC, PHASE_SEMANTIC = 0, 1, 2


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


class Config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "hidden", "layers", "heads", "kv_heads", "head_dim", "intermediate", "vocab", "max_pos")] + [
        ("eps", C.c_float), ("theta", C.c_float)]


class Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "q", "k", "v", "o", "gate", "up", "down", "input_norm", "q_norm", "k_norm", "post_norm")]


class NarS(C.Structure):
    _fields_ = [("latent", C.c_int32), ("max_frames", C.c_int32), ("shift", C.c_float)] + [
        (n, C.c_void_p) for n in ("vae2llm", "llm2vae", "time_in", "time_out", "latent_pos",
                                  "vae2llm_b", "llm2vae_b", "time_in_b", "time_out_b")] + [
        ("layers", C.POINTER(Layer))]


class VaeOpS(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("kind", "cin", "cout", "kernel", "stride", "padding", "dilation")] + [
        (n, C.c_void_p) for n in ("v", "g", "b", "alpha", "beta")]


VAE_CONV, VAE_CONVT, VAE_SNAKE, VAE_ELU, VAE_TANH, VAE_RES_BEGIN, VAE_RES_END = range(7)


class ModelS(C.Structure):
    _fields_ = [("c", Config), ("embed", C.c_void_p), ("lm_head", C.c_void_p),
                ("final_norm", C.c_void_p), ("layers", C.POINTER(Layer))]


class CacheS(C.Structure):
    _fields_ = [("layers", C.c_int32), ("width", C.c_int32), ("capacity", C.c_int32),
                ("length", C.c_int32), ("key", C.POINTER(C.c_float)), ("value", C.POINTER(C.c_float))]


class SamplingS(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int32),
                ("repetition_penalty", C.c_float), ("penalty_window", C.c_int32),
                ("min_tokens", C.c_int32), ("max_tokens", C.c_int32)]


class MT(C.Structure):
    _fields_ = [("state", C.c_uint32 * 624), ("next", C.c_int32)]


_lib: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        vp, i32, f32, f64 = C.c_void_p, C.c_int32, C.c_float, C.c_double
        sig = {
            "y2o_set_threads": (None, [i32]),
            "y2o_round_bf16": (f32, [f32]),
            "y2o_round_bf16_bits": (None, [vp, vp, C.c_size_t]),
            "y2o_expf": (f32, [f32]),
            "y2o_log1p": (f64, [f64]),
            "y2o_dot_bf16": (f32, [vp, vp, i32]),
            "y2o_dot_f32": (f32, [vp, vp, i32]),
            "y2o_linear": (None, [vp, i32, i32, vp, i32, vp]),
            "y2o_gemv_raw": (None, [vp, i32, i32, vp, vp]),
            "y2o_norm_scale": (f32, [vp, i32, f32]),
            "y2o_norm_apply": (None, [vp, i32, i32, vp, f32, vp]),
            "y2o_norm_heads": (None, [vp, i32, i32, vp, f32]),
            "y2o_rotary_table": (None, [i32, i32, i32, f32, vp, vp]),
            "y2o_rotary_apply": (None, [vp, i32, i32, i32, vp, vp]),
            "y2o_attention_row": (None, [vp, vp, vp, i32, i32, i32, i32, vp]),
            "y2o_superblock": (i32, [i32]),
            "y2o_cache_new": (C.POINTER(CacheS), [vp, i32]),
            "y2o_cache_free": (None, [C.POINTER(CacheS)]),
            "y2o_hidden": (i32, [vp, C.POINTER(CacheS), vp, i32, vp]),
            "y2o_hidden_prenorm": (i32, [vp, C.POINTER(CacheS), vp, i32, vp]),
            "y2o_forward": (i32, [vp, C.POINTER(CacheS), vp, i32, vp]),
            "y2o_forward_phase": (i32, [vp, C.POINTER(CacheS), vp, i32, i32, vp]),
            "y2o_forward_rows": (i32, [vp, vp, vp, i32, i32, vp]),
            "y2o_prefill": (i32, [vp, C.POINTER(CacheS), vp, i32, vp]),
            "y2o_velocity": (i32, [vp, vp, C.POINTER(CacheS), vp, i32, f64, i32, vp]),
            "y2o_normal": (None, [C.c_uint64, i32, vp]),
            "y2o_conv": (None, [i32, i32, i32, i32, i32, i32, i32, vp, i32, vp, vp, vp]),
            "y2o_conv_length": (i32, [i32, i32, i32, i32, i32, i32]),
            "y2o_vae_run": (i32, [vp, i32, vp, i32, i32, vp, vp, vp]),
            "y2o_vae_length": (i32, [vp, i32, i32]),
            "y2o_synthesize": (i32, [vp, vp, vp, i32, vp, i32, C.c_uint64, i32, vp]),
            "y2o_mt_seed": (None, [vp, C.c_uint64]),
            "y2o_mt_next": (C.c_uint32, [vp]),
            "y2o_mt_discard": (None, [vp, C.c_uint64]),
            "y2o_mt_uniform_f64": (f64, [vp]),
            "y2o_cfg_mix": (None, [vp, vp, i32, f32, vp]),
            "y2o_choose": (i32, [vp, i32, vp, vp, i32, i32, i32, i32, vp, vp]),
            "y2o_generate": (i32, [vp, vp, i32, vp, C.c_uint64, i32, vp, i32, f32, i32, vp, vp, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def set_threads(n: int) -> None:
    lib().y2o_set_threads(n)


class Model:
    """Oracle model over the same host arrays the GPU model was opened from."""

    def __init__(self, ckpt):
        c = ckpt.config
        self.config = c
        self._ckpt = ckpt
        self._layers = (Layer * c.num_hidden_layers)()
        for i, w in enumerate(ckpt.layers):
            L = self._layers[i]
            L.q, L.k, L.v, L.o = _p(w.q_proj), _p(w.k_proj), _p(w.v_proj), _p(w.o_proj)
            L.gate, L.up, L.down = _p(w.gate_proj), _p(w.up_proj), _p(w.down_proj)
            L.input_norm, L.q_norm = _p(w.input_layernorm), _p(w.q_norm)
            L.k_norm, L.post_norm = _p(w.k_norm), _p(w.post_attention_layernorm)
        cfg = Config(c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads,
                     c.head_dim, c.intermediate_size, c.vocab_size, c.max_position_embeddings,
                     c.rms_norm_eps, c.rope_theta)
        self._m = ModelS(cfg, _p(ckpt.embed_tokens), _p(ckpt.lm_head), _p(ckpt.final_norm), self._layers)

    @property
    def ref(self):
        return C.byref(self._m)

    def cache(self, capacity: int) -> "Cache":
        return Cache(self, capacity)

    def forward_phase(self, ids: Sequence[int], cache: "Cache", phase: int = PHASE_NONE) -> np.ndarray:
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.config.vocab_size, dtype=np.float32)
        rc = lib().y2o_forward_phase(self.ref, cache.ptr, _p(arr), len(arr), phase, _p(out))
        if rc:
            raise RuntimeError(f"oracle error {rc}")
        return out

    def forward(self, ids, cache):
        return self.forward_phase(ids, cache, PHASE_NONE)

    def forward_rows(self, ids: Sequence[int], caches: Sequence["Cache"], phase: int = PHASE_NONE) -> np.ndarray:
        """forward_phase([ids[r]], caches[r]) for every r in one pass over the
        weights: [len(ids), vocab] logits, the same as separate calls."""
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        if len(arr) != len(caches) or not 1 <= len(arr) <= 8:
            raise ValueError("one id per cache, 1 to 8 rows")
        ptrs = (C.POINTER(CacheS) * len(caches))(*[c.ptr for c in caches])
        out = np.empty((len(arr), self.config.vocab_size), dtype=np.float32)
        rc = lib().y2o_forward_rows(self.ref, ptrs, _p(arr), len(arr), phase, _p(out))
        if rc:
            raise RuntimeError(f"oracle error {rc}")
        return out

    def prefill(self, ids, capacity: int, phase: int = PHASE_NONE):
        cache = Cache(self, capacity)
        arr = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(self.config.vocab_size, dtype=np.float32)
        # chunks of 256 like Model::prefill_phase (src/model.rs:516)
        rc = 0
        for s in range(0, len(arr), 256):
            chunk = np.ascontiguousarray(arr[s:s + 256])
            rc = lib().y2o_forward_phase(self.ref, cache.ptr, _p(chunk), len(chunk), phase, _p(out))
            if rc:
                raise RuntimeError(f"oracle error {rc}")
        return cache, out


class Nar:
    """Oracle NAR pathway over the same host arrays (a NarWeights) as the GPU's."""

    def __init__(self, model: Model, w):
        self.model, self.w = model, w
        n = len(w.layers)
        self._layers = (Layer * n)()
        for i, lw in enumerate(w.layers):
            L = self._layers[i]
            L.q, L.k, L.v, L.o = _p(lw.q_proj), _p(lw.k_proj), _p(lw.v_proj), _p(lw.o_proj)
            L.gate, L.up, L.down = _p(lw.gate_proj), _p(lw.up_proj), _p(lw.down_proj)
            L.input_norm, L.q_norm = _p(lw.input_layernorm), _p(lw.q_norm)
            L.k_norm, L.post_norm = _p(lw.k_norm), _p(lw.post_attention_layernorm)
        self._n = NarS(w.latent_dim, w.max_latent_frames, w.timestep_shift,
                       _p(w.vae2llm), _p(w.llm2vae), _p(w.time_in), _p(w.time_out), _p(w.latent_pos),
                       _p(w.vae2llm_bias), _p(w.llm2vae_bias), _p(w.time_in_bias), _p(w.time_out_bias),
                       self._layers)

    def velocity(self, state: np.ndarray, cache: "Cache", raw_t: float, nar_cond_end: int = 0) -> np.ndarray:
        """Model::velocity (src/model.rs:611-698): state [frames, latent]."""
        st = np.ascontiguousarray(state, dtype=np.float32)
        out = np.empty_like(st)
        rc = lib().y2o_velocity(self.model.ref, C.byref(self._n), cache.ptr, _p(st), st.shape[0], raw_t,
                                nar_cond_end, _p(out))
        if rc:
            raise RuntimeError(f"oracle error {rc}")
        return out


    def synthesize(self, prefix, codec, seed: int, steps: int) -> np.ndarray:
        """Model::synthesize (src/model.rs:699-775): [len(codec), latent]."""
        p = np.ascontiguousarray(prefix, dtype=np.int32)
        cd = np.ascontiguousarray(codec, dtype=np.int32)
        out = np.empty((len(cd), self.w.latent_dim), np.float32)
        rc = lib().y2o_synthesize(self.model.ref, C.byref(self._n), _p(p), len(p), _p(cd), len(cd), seed, steps,
                                  _p(out))
        if rc:
            raise RuntimeError(f"oracle error {rc}")
        return out


def conv(transpose, x, w, b, kernel, stride, padding, dilation):
    """Conv::apply / transposed with ready weights (src/vae.rs:165-257)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    frames, cin = x.shape
    cout = w.shape[1] if transpose else w.shape[0]
    n = lib().y2o_conv_length(int(transpose), frames, kernel, stride, padding, dilation)
    out = np.empty((n, cout), np.float32)
    bb = None if b is None else np.ascontiguousarray(b, np.float32)
    lib().y2o_conv(int(transpose), cin, cout, kernel, stride, padding, dilation, _p(x), frames, _p(w), _p(bb),
                   _p(out))
    return out


class VaeOps:
    """An operation list of the VAE decoder (y2o_vae_op) over numpy arrays:
    entries (kind, dict of ints, dict of arrays)."""

    def __init__(self, ops):
        self._keep = []
        self._ops = (VaeOpS * len(ops))()
        for k, (kind, ints, arrs) in enumerate(ops):
            o = self._ops[k]
            o.kind = kind
            for f in ("cin", "cout", "kernel", "stride", "padding", "dilation"):
                setattr(o, f, int(ints.get(f, 0)))
            for f in ("v", "g", "b", "alpha", "beta"):
                a = arrs.get(f)
                if a is not None:
                    a = np.ascontiguousarray(a, np.float32)
                    self._keep.append(a)
                    setattr(o, f, a.ctypes.data)
        self.n = len(ops)

    def length(self, frames: int) -> int:
        return lib().y2o_vae_length(self._ops, self.n, frames)

    def run(self, x) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        n = self.length(x.shape[0])
        out = np.empty(n * 4096, np.float32)  # channels of any op stay below 4096
        fr, ch = C.c_int(0), C.c_int(0)
        rc = lib().y2o_vae_run(self._ops, self.n, _p(x), x.shape[0], x.shape[1], _p(out), C.byref(fr), C.byref(ch))
        if rc:
            raise RuntimeError(f"oracle error {rc}")
        return out[:fr.value * ch.value].reshape(fr.value, ch.value)


def normal(seed: int, n: int) -> np.ndarray:
    """Generator::normal_tensor's values (src/sampling.rs:64-79)."""
    out = np.empty(n, np.float32)
    lib().y2o_normal(seed, n, _p(out))
    return out


class Cache:
    def __init__(self, model: Model, capacity: int):
        self.ptr = lib().y2o_cache_new(C.byref(model._m.c), capacity)
        if not self.ptr:
            raise MemoryError("oracle cache")
        self.capacity = capacity

    @property
    def length(self) -> int:
        return self.ptr.contents.length

    def keys(self, layer: int) -> np.ndarray:
        c = self.ptr.contents
        n = c.length * c.width
        base = layer * c.capacity * c.width
        return np.ctypeslib.as_array(c.key, shape=(c.layers * c.capacity * c.width,))[base:base + n].reshape(c.length, c.width)

    def values(self, layer: int) -> np.ndarray:
        c = self.ptr.contents
        n = c.length * c.width
        base = layer * c.capacity * c.width
        return np.ctypeslib.as_array(c.value, shape=(c.layers * c.capacity * c.width,))[base:base + n].reshape(c.length, c.width)

    def arrays(self):
        """(key, value) views of the whole mirror, each [layers, capacity, width]."""
        c = self.ptr.contents
        shape = (c.layers, c.capacity, c.width)
        n = c.layers * c.capacity * c.width
        return (np.ctypeslib.as_array(c.key, shape=(n,)).reshape(shape),
                np.ctypeslib.as_array(c.value, shape=(n,)).reshape(shape))

    def load(self, key: np.ndarray, value: np.ndarray, length: int) -> None:
        """Take rows [0, length) of a host K/V mirror ([layers, stride,
        width] each, e.g. a device cache's export) as this cache's
        context."""
        c = self.ptr.contents
        assert length <= c.capacity and key.shape == value.shape and key.shape[1] >= length
        k, v = self.arrays()
        k[:, :length, :] = key[:, :length, :]
        v[:, :length, :] = value[:, :length, :]
        c.length = length

    def fill_random(self, length: int, seed: int) -> None:
        """Give the cache `length` positions of BF16-exact N(0, 1) keys and
        values (for timing a step at a given context without a prefill)."""
        c = self.ptr.contents
        assert length <= c.capacity
        n = c.layers * c.capacity * c.width
        rng = np.random.default_rng(seed)
        for arr in (np.ctypeslib.as_array(c.key, shape=(n,)), np.ctypeslib.as_array(c.value, shape=(n,))):
            v = arr.reshape(c.layers, c.capacity, c.width)
            x = rng.standard_normal((c.layers, length, c.width), dtype=np.float32)
            v[:, :length, :] = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)
        c.length = length

    def __del__(self):
        try:
            if self.ptr:
                lib().y2o_cache_free(self.ptr)
                self.ptr = None
        except Exception:
            pass


class Generator:
    """MT19937 of src/sampling.rs:10-63."""

    def __init__(self, seed: int):
        self._s = MT()
        lib().y2o_mt_seed(C.byref(self._s), seed)

    def next_u32(self) -> int:
        return lib().y2o_mt_next(C.byref(self._s))

    def discard(self, n: int) -> None:
        lib().y2o_mt_discard(C.byref(self._s), n)

    def uniform_f64(self) -> float:
        return lib().y2o_mt_uniform_f64(C.byref(self._s))

    @property
    def ref(self):
        return C.byref(self._s)


def sampling(s) -> SamplingS:
    return SamplingS(s.temperature, s.top_p, s.top_k, s.repetition_penalty, s.penalty_window,
                     s.min_tokens, s.max_tokens)


def choose(logits: np.ndarray, s, history: Sequence[int], step: int, phase: int, legacy: bool,
           rng: Generator) -> int:
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    h = np.ascontiguousarray(history, dtype=np.int32)
    out = C.c_int32(-1)
    ss = sampling(s)
    rc = lib().y2o_choose(_p(lg), len(lg), C.byref(ss), _p(h) if len(h) else None, len(h), step, phase,
                          int(legacy), rng.ref, C.byref(out))
    if rc:
        raise RuntimeError(f"oracle choose error {rc}")
    return out.value


def cfg_mix(cond: np.ndarray, uncond: np.ndarray, scale: float) -> np.ndarray:
    out = np.empty_like(cond)
    lib().y2o_cfg_mix(_p(cond), _p(uncond), len(cond), scale, _p(out))
    return out


def generate(model: Model, prefix, s, seed: int, phase: int = PHASE_NONE, negative=None,
             scale: float = 1.0, legacy: bool = False):
    p = np.ascontiguousarray(prefix, dtype=np.int32)
    n = None if negative is None else np.ascontiguousarray(negative, dtype=np.int32)
    out = np.zeros(max(s.max_tokens, 1), dtype=np.int32)
    count, trunc = C.c_int32(0), C.c_int32(0)
    ss = sampling(s)
    rc = lib().y2o_generate(model.ref, _p(p), len(p), C.byref(ss), seed, phase, _p(n),
                            0 if n is None else len(n), scale, int(legacy), _p(out), C.byref(count),
                            C.byref(trunc))
    if rc:
        raise RuntimeError(f"oracle generate error {rc}")
    return out[:count.value].tolist(), bool(trunc.value)
