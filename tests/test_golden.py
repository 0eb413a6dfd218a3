"""Committed golden fixtures of the reduced configuration (tests/golden/,
written by tests/golden/make_golden.py): the oracle must keep reproducing
them on the CPU, and the device must reproduce them on the GPU."""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

GOLD = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLD / name, allow_pickle=False)


@pytest.fixture(scope="module")
def meta():
    return json.loads((GOLD / "golden.json").read_text())


def test_oracle_reproduces_fixtures(meta, oracle_threads):
    import sys
    sys.path.insert(0, str(GOLD))
    import make_golden
    r = make_golden.compute(threads=oracle_threads)
    assert r["weights_sha256"] == meta["weights_sha256"], "synthetic weights changed"
    assert np.array_equal(r["prompt"], _load("reduced_prompt.npy"))
    assert np.array_equal(r["prefill_head"].view(np.uint32), _load("reduced_prefill_head.npy").view(np.uint32))
    assert r["prefill_sha256"] == meta["prefill_sha256"]
    assert np.array_equal(r["greedy"], _load("reduced_greedy64.npy"))
    assert np.array_equal(r["generate"], _load("reduced_generate32.npy"))


@pytest.mark.gpu
@pytest.mark.parametrize("step_kernel", [False, True], ids=["phase-kernels", "step-kernel"])
def test_device_reproduces_fixtures(meta, gpu, step_kernel):
    from yue2_rs_amd import synthetic
    import yue2_rs_amd as y2
    ck = synthetic.checkpoint(synthetic.REDUCED, seed=0)
    m = y2.Model.open(ck)
    assert m.set_step_kernel(step_kernel) == step_kernel
    prompt = _load("reduced_prompt.npy")
    greedy = _load("reduced_greedy64.npy")
    cache, logits = m.prefill_phase(prompt, len(prompt) + len(greedy))
    assert hashlib.sha256(logits.astype(np.float32).tobytes()).hexdigest() == meta["prefill_sha256"]
    dec = y2.Decoder(m, cache)
    toks, _ = dec.run(len(greedy), first_logits=logits)
    dec.close()
    assert np.array_equal(np.asarray(toks, np.int32), greedy)
    neg = np.asarray(synthetic.prompt(meta["negative_prompt_len"], ck.config.vocab_size,
                                      seed=meta["negative_prompt_seed"]), np.int32)
    gen = y2.generate(m, prompt, y2.Sampling(**meta["sampling"]), seed=meta["sampler_seed"],
                      negative=neg, scale=meta["cfg_scale"])
    assert np.array_equal(np.asarray(gen.tokens, np.int32), _load("reduced_generate32.npy"))
    m.close()
