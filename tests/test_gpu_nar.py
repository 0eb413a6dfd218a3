"""The NAR velocity stack on the device (yue2_hip_velocity, Model::velocity
src/model.rs:611-698) against the oracle's restatement (y2o_velocity, pinned
in tests/test_oracle_nar.py) on the same seeded weights, AR cache and
latents.

The device runs every linear as a BF16 MFMA GEMM and the attention as a
flash attention, keeping the BF16 rounding points but not the oracle's
summation order (as the reference's GPU stack differs from its CPU path), so
the contract is a tolerance: max |difference| <= 0.08 * std(oracle output)
(two-layer models; measured about 0.02-0.04), with a correlation above 0.999.
Frame counts 1, 30 and 200 cross the flash kernel's 64-key and 128-row
tiles; the AR prefix of 300 positions is prefilled bit-exactly on both
sides.  The velocity must leave the cache as it was: a decode step after it
still matches the oracle bit for bit."""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

from helpers import bits, rb

pytestmark = pytest.mark.gpu

TOL = 0.08
THREE_B_2L = dataclasses.replace(synthetic.CLASS_3B, num_hidden_layers=2, vocab_size=32768)


@pytest.fixture(scope="module", params=["reduced", "3b-2layer"])
def nar_pair(request, gpu, oracle_threads):
    cfg = synthetic.REDUCED if request.param == "reduced" else THREE_B_2L
    ck = synthetic.checkpoint(cfg, seed=1)
    nw = synthetic.nar_weights(cfg, seed=1, max_latent_frames=160, timestep_shift=2.0)
    gm, om = y2.Model.open(ck), O.Model(ck)
    gm.load_nar(nw)
    ids = synthetic.prompt(300, cfg.vocab_size, seed=8)
    gc, gl = gm.prefill_phase(ids, 320)
    oc, ol = om.prefill(ids, 320)
    assert np.array_equal(bits(gl), bits(ol))
    yield cfg, gm, om, O.Nar(om, nw), gc, oc
    gc.close()
    gm.close()


def _state(frames, seed):
    return rb(np.random.default_rng(seed).standard_normal((frames, 64)).astype(np.float32))


def _close(got, want, what):
    d = np.abs(got - want).max()
    s = want.std()
    print(f"{what}: max |d| {d:.4g} = {d / s:.4f} std", flush=True)
    assert np.all(np.isfinite(got))
    assert d <= TOL * s, f"{what}: max |d| {d:.4g} > {TOL} * std {s:.4g}"
    assert np.corrcoef(got.ravel(), want.ravel())[0, 1] > 0.999


@pytest.mark.parametrize("frames,raw_t", [(1, 0.0), (30, 1.3), (200, -2.5)])
def test_velocity_matches_oracle(nar_pair, frames, raw_t):
    cfg, gm, om, nar, gc, oc = nar_pair
    st = _state(frames, frames)
    _close(gm.velocity(st, gc, raw_t), nar.velocity(st, oc, raw_t), f"{cfg.hidden_size} frames {frames}")


def test_condition_end(nar_pair):
    cfg, gm, om, nar, gc, oc = nar_pair
    st = _state(40, 3)
    _close(gm.velocity(st, gc, 0.4, 120), nar.velocity(st, oc, 0.4, 120), "nar_cond_end 120")


def test_cache_untouched(nar_pair):
    """A decode step after velocities still matches the oracle bit for bit
    (the rows' own keys went to scratch, not to the cache)."""
    cfg, gm, om, nar, gc, oc = nar_pair
    gm.velocity(_state(16, 5), gc, 0.2)
    assert gc.length == oc.length == 300
    # the oracle's step and the device's step on caches that are still equal
    t = 7
    got = gm.forward([t], gc)
    want = om.forward([t], oc)
    assert np.array_equal(bits(got), bits(want))


def test_errors(gpu):
    cfg = synthetic.REDUCED
    gm = y2.Model.open(synthetic.checkpoint(cfg, seed=2))
    try:
        gc, _ = gm.prefill_phase([1, 2, 3], 8)
        with pytest.raises(y2.Yue2Error):
            gm.velocity(_state(4, 1), gc, 0.0)  # no NAR weights loaded
        gm.load_nar(synthetic.nar_weights(cfg, seed=2, max_latent_frames=16))
        with pytest.raises(y2.Yue2Error):
            gm.velocity(np.full((4, 64), 0.1, np.float32), gc, 0.0)  # not BF16 values
        with pytest.raises(y2.Yue2Error):
            gm.velocity(_state(cfg.max_position_embeddings, 1), gc, 0.0)  # past the RoPE table
        assert gm.velocity(_state(4, 1), gc, 0.0).shape == (4, 64)
        gc.close()
    finally:
        gm.close()


MUSIC = dataclasses.replace(synthetic.REDUCED, hidden_size=128, num_hidden_layers=2, num_attention_heads=2,
                            num_key_value_heads=1, intermediate_size=256, vocab_size=184704,
                            max_position_embeddings=128)


@pytest.fixture(scope="module")
def music(gpu, oracle_threads):
    ck = synthetic.checkpoint(MUSIC, seed=3)
    nw = synthetic.nar_weights(MUSIC, seed=3, max_latent_frames=64, timestep_shift=3.0)
    gm = y2.Model.open(ck)
    gm.load_nar(nw)
    yield ck, nw, gm, O.Nar(O.Model(ck), nw)
    gm.close()


def test_synthesize_matches_oracle(music):
    """Model::synthesize: two chunks of (128 - 20 - 3) / 2 = 52 and 38
    frames, two midpoint steps each (four velocities); the device's noise is
    the oracle's bit for bit (same MT19937 and libm), the latents agree within
    the velocity tolerance."""
    ck, nw, gm, nar = music
    prefix, codec = synthetic.prompt(20, 151643, seed=7), synthetic.prompt(90, 32768, seed=6)
    got = gm.synthesize(prefix, codec, 42, 2)
    want = nar.synthesize(prefix, codec, 42, 2)
    _close(got, want, "synthesize")


def test_synthesize_without_velocity_returns_the_noise(music):
    ck, nw, gm, nar = music
    z = dataclasses.replace(nw, llm2vae=np.zeros_like(nw.llm2vae), llm2vae_bias=np.zeros_like(nw.llm2vae_bias))
    gz = y2.Model.open(ck)
    try:
        gz.load_nar(z)
        got = gz.synthesize(synthetic.prompt(20, 151643, seed=7), synthetic.prompt(90, 32768, seed=6), 42, 2)
        want = rb(O.normal(42, 90 * 64)).reshape(90, 64)
        assert np.array_equal(bits(got), bits(want))
    finally:
        gz.close()


def test_synthesize_rejects(music):
    ck, nw, gm, nar = music
    for prefix, codec, steps in (([1] * 20, [], 2), ([1] * 20, [32768], 2), ([1] * 20, [5], 0), ([1] * 124, [5], 2)):
        with pytest.raises(y2.Yue2Error):
            gm.synthesize(prefix, codec, 1, steps)
