"""Microbenchmarks of the decode kernels against the MI355X HBM roofline.

GEMV (the BF16 GEMV family at the 3B-class layer shapes, FP32 accumulation,
batch 1 and 2): fused QKV 5120x3072, O 3072x3072, gate+up 16384x3072, down
3072x8192, LM head 84000x3072.  Algorithmic bytes = N K 2 + b K 2 + b N 4.
Attention (split-KV GQA decode, 24 query / 8 KV heads, head_dim 128, QK-norm,
RoPE at the position and the KV append included) at contexts 1024, 4096,
16384 and 24576, batch 1 and 2, over 28 distinct layer caches; bytes per
layer-call = b 4096 L (the K and V rows).
Copy: a plain 256 MiB device-to-device hipMemcpy, the practical HBM rate
(bytes = read + written) and the calibration workload of the FETCH_SIZE /
WRITE_SIZE counters.
GEMM (the prefill's BF16 MFMA GEMM at the 3B-class linears for a 2048-row
prompt chunk) and prefill (the whole matrix-core prefill of 2048- and
24000-token prompts through the 3B-class model, random-init weights),
against the 2.5 PFLOP/s dense BF16 matrix peak.
NAR (the velocity stack of the acoustic stage on the 3B-class model with a
random-init NAR pathway): one call for 11786 latent frames after a 1000-token
prefix, the largest chunk a 24576-position context holds (synthesize,
src/model.rs:717-722), keys = prefix + codec chunk + the frames.

VAE (the FP32 decoder at an Oobleck shape of the reference's default
downsampling ratio 1920, random-init): one decode of a 512 + 2 x 16-frame
tile, the reference's decode_tiled core and halo (src/pipeline.rs:279,415),
and decode_tiled of 4500 frames (three minutes of 48 kHz audio), against the
157.3 TFLOP/s FP32 peak.  FLOPs = 2 x the multiply-adds of every
convolution (a transposed one: kernel taps per input row).

Every timed launch reads another copy of its operands (more than 512 MB in
total), so the 256 MB Infinity Cache cannot serve repeats.  One JSON line per
case on stdout.

    python -m yue2_rs_amd.microbench [gemv|attention|copy|gemm|prefill|nar|vae|all]
"""
from __future__ import annotations

import ctypes as C
import json
import sys

import numpy as np

from .api import _check, available, lib

HBM_PEAK = 8.0e12
MFMA_BF16_PEAK = 2.5e15
FP32_PEAK = 157.3e12
GEMM_SHAPES = [("qkv", 5120, 3072, 0), ("o", 3072, 3072, 0), ("gate_up", 8192, 3072, 1), ("down", 3072, 8192, 0)]
GEMV_SHAPES = [("qkv", 5120, 3072), ("o", 3072, 3072), ("gate_up", 16384, 3072), ("down", 3072, 8192),
               ("lm_head", 84000, 3072)]
CONTEXTS = [1024, 4096, 16384, 24576]


def gemv(n: int, k: int, rows: int, iters: int = 200) -> dict:
    copies = max(2, -(-600 * 2**20 // (n * k * 2)))  # > 512 MB of distinct weights
    ms, by = C.c_float(0), C.c_double(0)
    _check(lib().yue2_hip_bench_gemv(n, k, rows, copies, iters, C.byref(ms), C.byref(by)))
    gbs = by.value / (ms.value * 1e-3) / 1e9
    return {"n": n, "k": k, "rows": rows, "copies": copies, "launch_us": round(ms.value * 1e3, 2),
            "bytes": int(by.value), "GB_s": round(gbs, 1), "frac": round(gbs * 1e9 / HBM_PEAK, 4)}


def attention(context: int, rows: int, layers: int = 28, iters: int = 112) -> dict:
    ms, by = C.c_float(0), C.c_double(0)
    _check(lib().yue2_hip_bench_attention(context, rows, layers, iters, C.byref(ms), C.byref(by)))
    gbs = by.value / (ms.value * 1e-3) / 1e9
    return {"context": context, "rows": rows, "layers": layers, "launch_us": round(ms.value * 1e3, 2),
            "bytes": int(by.value), "GB_s": round(gbs, 1), "frac": round(gbs * 1e9 / HBM_PEAK, 4)}


def copy(nbytes: int = 256 * 2**20, iters: int = 20) -> dict:
    ms = C.c_float(0)
    _check(lib().yue2_hip_bench_copy(nbytes, iters, C.byref(ms)))
    gbs = 2 * nbytes / (ms.value * 1e-3) / 1e9
    return {"bytes": nbytes, "copy_us": round(ms.value * 1e3, 2), "GB_s": round(gbs, 1),
            "frac": round(gbs * 1e9 / HBM_PEAK, 4)}


def gemm(m: int, n: int, k: int, pair: int, iters: int = 50) -> dict:
    ms, fl = C.c_float(0), C.c_double(0)
    _check(lib().yue2_hip_bench_gemm(m, n, k, pair, iters, C.byref(ms), C.byref(fl)))
    tf = fl.value / (ms.value * 1e-3) / 1e12
    return {"m": m, "n": n, "k": k, "pair": pair, "launch_us": round(ms.value * 1e3, 2), "flops": fl.value,
            "TFLOP_s": round(tf, 1), "frac": round(tf * 1e12 / MFMA_BF16_PEAK, 4)}


def prefill(tokens) -> list:
    """The matrix-core prefill of each prompt length through the 3B-class
    model (seed-0 weights and prompt), the second of two runs timed."""
    import time
    from . import synthetic
    from .api import Model, synchronize
    c = synthetic.CLASS_3B
    model = Model.open(synthetic.checkpoint(c, seed=0, threads=16))
    out = []
    for n in tokens:
        ids = synthetic.prompt(n, c.vocab_size, seed=0)
        for _ in range(2):
            synchronize()
            t = time.perf_counter()
            cache, _ = model.prefill_mfma(ids, n)
            synchronize()
            dt = time.perf_counter() - t
            cache.close()
        H, D, I, V = c.hidden_size, c.head_dim, c.intermediate_size, c.vocab_size
        q, kv = c.num_attention_heads * D, c.num_key_value_heads * D
        fl = (2.0 * n * c.num_hidden_layers * (H * (q + 2 * kv) + q * H + 3 * H * I) +
              c.num_hidden_layers * c.num_attention_heads * 4.0 * D * n * (n + 1) / 2.0 + 2.0 * V * H)
        out.append({"tokens": n, "s": round(dt, 4), "tokens_per_s": round(n / dt, 1), "flops": fl,
                    "TFLOP_s": round(fl / dt / 1e12, 1), "frac": round(fl / dt / MFMA_BF16_PEAK, 4)})
    model.close()
    return out


def nar(prefix: int = 1000, frames: int = 11786) -> dict:
    """One velocity call (the second of two timed) for `frames` latent rows
    against an AR cache of prefix + frames + 1 positions (the chunk's ids:
    prefix, codec tokens, the end token)."""
    import time
    from . import synthetic
    from .api import Model, synchronize
    c = synthetic.CLASS_3B
    model = Model.open(synthetic.checkpoint(c, seed=0, threads=16))
    model.load_nar(synthetic.nar_weights(c, seed=0, threads=16))
    length = prefix + frames + 1
    cache, _ = model.prefill_mfma(synthetic.prompt(length, c.vocab_size, seed=0), length)
    st = np.random.default_rng(0).standard_normal((frames, 64)).astype(np.float32)
    st = (st.view(np.uint32) & 0xFFFF0000).view(np.float32)
    for _ in range(2):
        synchronize()
        t = time.perf_counter()
        model.velocity(st, cache, 0.5)
        synchronize()
        dt = time.perf_counter() - t
    cache.close()
    model.close()
    H, D, I = c.hidden_size, c.head_dim, c.intermediate_size
    q, kv = c.num_attention_heads * D, c.num_key_value_heads * D
    n, keys = frames + 2, length + frames + 2
    fl = (2.0 * n * c.num_hidden_layers * (H * (q + 2 * kv) + q * H + 3 * H * I) +
          c.num_hidden_layers * c.num_attention_heads * 4.0 * D * n * keys +
          2.0 * n * 64 * H * 2 + 2.0 * (256 * H + H * H))
    return {"frames": frames, "keys": keys, "s": round(dt, 4), "flops": fl, "TFLOP_s": round(fl / dt / 1e12, 1),
            "frac": round(fl / dt / MFMA_BF16_PEAK, 4)}


def vae_flops(cfg: dict, frames: int) -> float:
    """2 x the multiply-adds of the decoder's convolutions for `frames`
    latent rows (even strides: each block multiplies the length by its
    stride)."""
    d = cfg["decoder_config"]
    ch, mults, strides = d["channels"], [1] + list(d["c_mults"]), d["strides"]
    n, f = frames, 2.0 * d["latent_dim"] * ch * mults[-1] * 7 * frames
    for i in range(len(mults) - 1, 0, -1):
        cin, cout, s = ch * mults[i], ch * mults[i - 1], strides[i - 1]
        f += 2.0 * cin * cout * 2 * s * n
        n *= s
        f += 3 * 2.0 * cout * cout * (7 + 1) * n
    return f + 2.0 * ch * d["out_channels"] * 7 * n


def vae(tile: int = 544, song: int = 4500) -> list:
    """Wall-clock seconds of Vae::decode for one tile (the second of two
    calls) and of decode_tiled over `song` frames, latents in host memory,
    audio back in host memory."""
    import tempfile
    import time
    from . import synthetic
    from .api import Vae
    cfg, t = synthetic.vae(0, **synthetic.VAE_1920)
    with tempfile.TemporaryDirectory() as d:
        v = Vae(synthetic.write_vae(d, cfg, t))
    del t
    out = []
    try:
        rng = np.random.default_rng(0)
        z = rng.standard_normal((tile, cfg["latent_dim"])).astype(np.float32)
        for _ in range(2):
            t0 = time.perf_counter()
            v.decode(z)
            dt = time.perf_counter() - t0
        fl = vae_flops(cfg, tile)
        out.append({"frames": tile, "s": round(dt, 4), "flops": fl, "TFLOP_s": round(fl / dt / 1e12, 1),
                    "frac": round(fl / dt / FP32_PEAK, 4)})
        z = rng.standard_normal((song, cfg["latent_dim"])).astype(np.float32)
        core, halo = cfg["decode_core_frames"], cfg["decode_halo_frames"]
        t0 = time.perf_counter()
        audio = v.decode_tiled(z, core, halo)
        dt = time.perf_counter() - t0
        fl = sum(vae_flops(cfg, min(song, e + halo) - max(0, s - halo))
                 for s, e in ((s, min(s + core, song)) for s in range(0, song, core)))
        out.append({"frames": song, "tiled": [core, halo], "audio_s": audio.shape[0] / cfg["sample_rate"],
                    "s": round(dt, 4), "x_realtime": round(audio.shape[0] / cfg["sample_rate"] / dt, 1),
                    "flops": fl, "TFLOP_s": round(fl / dt / 1e12, 1), "frac": round(fl / dt / FP32_PEAK, 4)})
    finally:
        v.close()
    return out


def main(argv=None) -> int:
    what = (argv or sys.argv[1:] or ["all"])[0]
    if not available():
        print("no gfx950 device available", file=sys.stderr)
        return 1
    if what in ("gemv", "all"):
        for name, n, k in GEMV_SHAPES:
            for rows in (1, 2):
                print(json.dumps({"bench": "gemv", "shape": name, **gemv(n, k, rows)}), flush=True)
    if what in ("attention", "all"):
        for L in CONTEXTS:
            for rows in (1, 2):
                print(json.dumps({"bench": "attention", **attention(L, rows)}), flush=True)
    if what in ("copy", "all"):
        print(json.dumps({"bench": "copy", **copy()}), flush=True)
    if what in ("gemm", "all"):
        for m in (2048, 4096):  # the prefill's chunk rows
            for name, n, k, pair in GEMM_SHAPES:
                print(json.dumps({"bench": "gemm", "shape": name, **gemm(m, n, k, pair)}), flush=True)
    if what in ("nar", "all"):
        print(json.dumps({"bench": "nar_velocity", **nar()}), flush=True)
    if what in ("vae", "all"):
        for r in vae():
            print(json.dumps({"bench": "vae", **r}), flush=True)
    if what in ("prefill", "all"):
        for r in prefill([2048, 24000]):
            print(json.dumps({"bench": "prefill", **r}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
