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

Every timed launch reads another copy of its operands (more than 512 MB in
total), so the 256 MB Infinity Cache cannot serve repeats.  One JSON line per
case on stdout.

    python -m yue2_rs_amd.microbench [gemv|attention|copy|all]
"""
from __future__ import annotations

import ctypes as C
import json
import sys

from .api import _check, available, lib

HBM_PEAK = 8.0e12
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
    return 0


if __name__ == "__main__":
    sys.exit(main())
