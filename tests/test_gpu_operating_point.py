"""Parity where the benchmark runs: the full 28-layer 3B-class model
decoding from 2048-position caches that the matrix-core prefill filled.

The benchmark's caches come from yue2_hip_prefill_mfma, whose GEMMs sum in
their own order (a tolerance contract against the decode-order prefill).  To
check the decode loop on exactly those caches, each device cache is
exported (yue2_hip_cache_export, the `shadow` rows of src/metal.m:846-866)
into an oracle cache, and the oracle then replays sampling::generate's loop
(src/sampling.rs:258-291) from the same K/V and the same first logits: CFG
mix (guidance 1.5), choose() with the generated ids as history and the same
MT19937 stream, then each row's Model::forward.  Every step compares the
chosen id and both rows' logits bit for bit, for 64 greedy and 64 sampled
(T 0.9, top-k 50, top-p 0.93, penalty 1.2 over 50 ids) CFG steps and 32
sampled batch-1 steps.  The prompts are the benchmark's: 2048 uniform ids
from seeds 0 (conditional) and 1 (unconditional)."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

from helpers import bits

pytestmark = pytest.mark.gpu

PROMPT = 2048
SAMPLED = dict(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50)


@pytest.fixture(scope="module")
def model_3b(gpu, oracle_threads):
    ck = synthetic.checkpoint(synthetic.CLASS_3B, seed=0, threads=16)
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(True)
    yield ck, gm, O.Model(ck)
    gm.close()


def _mfma_rows(gm, om, rows, steps):
    """(device caches, oracle caches holding their export, first logits)."""
    V = om.config.vocab_size
    gcs, ocs, first = [], [], []
    for r in range(rows):
        ids = synthetic.prompt(PROMPT, V, seed=r)
        gc, gl = gm.prefill_mfma(ids, PROMPT + steps + 1)
        k, v = gc.export()
        oc = O.Cache(om, PROMPT + steps + 1)
        oc.load(k, v, PROMPT)
        gcs.append(gc)
        ocs.append(oc)
        first.append(gl)
    return gcs, ocs, first


def _run(model_3b, rows, steps, sampling, seed=2024, scale=1.5):
    _, gm, om = model_3b
    gcs, ocs, first = _mfma_rows(gm, om, rows, steps)
    s = y2.Sampling(**(sampling or {}), min_tokens=0, max_tokens=steps) if sampling else None
    dec = y2.Decoder(gm, *gcs, sampling=s, seed=seed, scale=scale if rows == 2 else 1.0)
    gen = O.Generator(seed)
    logits = first
    history = []
    for step in range(steps):
        mixed = O.cfg_mix(logits[0], logits[1], scale) if rows == 2 else logits[0]
        if s is None:
            want = int(np.argmax(mixed))
        else:
            want = O.choose(mixed, s, history, step, y2.PHASE_NONE, False, gen)
        got, _ = dec.run(1, first_logits=np.concatenate(first) if step == 0 else None)
        print(f"rows {rows} step {step}: device {list(got)} oracle {want}", flush=True)
        assert list(got) == [want], f"id differs at step {step}"
        history.append(want)
        logits = list(om.forward_rows([want] * len(ocs), ocs))
        dev = dec.logits()
        for r in range(rows):
            assert np.array_equal(bits(dev[r]), bits(logits[r])), f"row {r} logits differ at step {step}"
    dec.close()
    for gc in gcs:
        assert gc.length == PROMPT + steps
        gc.close()


@pytest.mark.timeout(600)
def test_cfg_greedy_64_steps_from_mfma_caches(model_3b):
    _run(model_3b, 2, 64, None)


@pytest.mark.timeout(600)
def test_cfg_sampled_64_steps_from_mfma_caches(model_3b):
    _run(model_3b, 2, 64, SAMPLED)


@pytest.mark.timeout(600)
def test_batch1_sampled_32_steps_from_mfma_cache(model_3b):
    _run(model_3b, 1, 32, SAMPLED, seed=77)
