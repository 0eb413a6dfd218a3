"""Write the golden fixtures of the reduced configuration with the CPU oracle.

    python tests/golden/make_golden.py

Fixtures (little-endian .npy, plus golden.json with digests):
  reduced_prompt.npy          256 prompt ids (MT19937 seed 0, id = next_u32 % V)
  reduced_prefill_head.npy    the first 64 logits after the 256-token prefill
  reduced_greedy64.npy        64 greedy ids after the prefill (Model::forward + argmax)
  reduced_generate32.npy      sampling::generate: 32 ids, T 0.9 / top-k 50 / top-p 0.93,
                              penalty 1.2 over 50, CFG 1.5 with a 100-id negative
                              prompt (seed 1), sampler seed 7
  golden.json                 SHA-256 of the full prefill logits and of the
                              synthetic weights, and the settings above

The reference holds no vectors for these paths (its only known-answer test
is the attention check of src/tensor.rs:9-83), so these pin the oracle's
own results against change; the GPU tests compare the device with them too.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import oracle as O  # noqa: E402
from yue2_rs_amd import synthetic  # noqa: E402
import yue2_rs_amd as y2  # noqa: E402

PROMPT, GREEDY, NEG, GEN = 256, 64, 100, 32
SAMPLING = dict(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                min_tokens=0, max_tokens=GEN)
SEED, SCALE = 7, 1.5


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def compute(threads: int = 8) -> dict:
    O.set_threads(threads)
    ck = synthetic.checkpoint(synthetic.REDUCED, seed=0)
    om = O.Model(ck)
    V = ck.config.vocab_size
    prompt = np.asarray(synthetic.prompt(PROMPT, V, seed=0), np.int32)
    cache, logits = om.prefill(prompt, PROMPT + GREEDY)
    prefill = logits.copy()
    greedy = []
    for _ in range(GREEDY):
        t = int(np.argmax(logits))
        greedy.append(t)
        logits = om.forward([t], cache)
    neg = np.asarray(synthetic.prompt(NEG, V, seed=1), np.int32)
    gen, _ = O.generate(om, prompt, y2.Sampling(**SAMPLING), SEED, negative=neg, scale=SCALE)
    weights = {"embed_tokens": sha(ck.embed_tokens), "lm_head": sha(ck.lm_head),
               "layer0.q_proj": sha(ck.layers[0].q_proj), "layer1.down_proj": sha(ck.layers[1].down_proj)}
    return {
        "prompt": prompt, "prefill_head": prefill[:64].astype(np.float32),
        "prefill_sha256": sha(prefill.astype(np.float32)), "greedy": np.asarray(greedy, np.int32),
        "generate": np.asarray(gen, np.int32), "weights_sha256": weights,
    }


def main() -> None:
    r = compute()
    np.save(HERE / "reduced_prompt.npy", r["prompt"].astype("<i4"))
    np.save(HERE / "reduced_prefill_head.npy", r["prefill_head"].astype("<f4"))
    np.save(HERE / "reduced_greedy64.npy", r["greedy"].astype("<i4"))
    np.save(HERE / "reduced_generate32.npy", r["generate"].astype("<i4"))
    meta = {"config": "reduced (2 layers, H 1024, Hq 16, Hkv 4, d 64, I 2816, V 32768)",
            "weights": "synthetic seed 0, BF16 ~N(0, 0.02), norms 1",
            "prefill_sha256": r["prefill_sha256"], "weights_sha256": r["weights_sha256"],
            "sampling": SAMPLING, "sampler_seed": SEED, "cfg_scale": SCALE, "negative_prompt_seed": 1,
            "negative_prompt_len": NEG}
    (HERE / "golden.json").write_text(json.dumps(meta, indent=2) + "\n")
    print("wrote", sorted(p.name for p in HERE.glob("*.npy")))


if __name__ == "__main__":
    main()
