"""Lifetimes at the boundary and the K/V export.

The reference lets a Cache outlive its Model (src/model.rs:286-290: each
has its own Drop), so a Rust binding may free the model first.  The library
detaches a model's caches and decoders when the model is freed: a detached
decoder's calls fail with YUE2_ERR_ARG, a detached cache can still be
exported, and every free order is legal.

yue2_hip_cache_export hands device K/V rows back in the host-mirror layout,
as the reference's fast path returns each token's rows as `shadow` for its
mirror (src/metal.m:846-866, src/model.rs:556-566): the rows a device step
appended equal, bit for bit, the rows the oracle's Model::forward appends
for the same token."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

from helpers import bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ck(gpu, oracle_threads):
    return synthetic.checkpoint(synthetic.REDUCED, seed=0)


def _oracle_greedy(om, ids, cap, steps):
    oc, ol = om.prefill(ids, cap)
    toks = []
    for _ in range(steps):
        t = int(np.argmax(ol))
        toks.append(t)
        ol = om.forward([t], oc)
    return oc, toks


def test_export_round_trip(ck):
    gm, om = y2.Model.open(ck), O.Model(ck)
    try:
        oc = O.Cache(om, 300)
        oc.fill_random(250, seed=3)
        k, v = oc.arrays()
        gc = y2.Cache(gm, 300)
        gc.load(k, v, 250)
        ek, ev = gc.export()
        assert ek.shape == (2, 250, 4 * 64)
        assert np.array_equal(bits(ek), bits(k[:, :250])) and np.array_equal(bits(ev), bits(v[:, :250]))
        # a window of rows into a mirror of the cache's own stride
        pk, pv = gc.export(start=17, n=40, stride=300)
        assert np.array_equal(bits(pk[:, 17:57]), bits(k[:, 17:57]))
        assert np.array_equal(bits(pv[:, 17:57]), bits(v[:, 17:57]))
        assert not pk[:, :17].any() and not pk[:, 57:].any()
        with pytest.raises(y2.Yue2Error) as e:
            gc.export(start=240, n=20)
        assert e.value.code == -1
        gc.close()
    finally:
        gm.close()


@pytest.mark.parametrize("step_kernel", [False, True], ids=["phase-kernels", "step-kernel"])
def test_export_gives_the_shadow_rows(ck, step_kernel):
    """The rows each device step appends, exported one token at a time (the
    `shadow` of src/metal.m:846-866), are the oracle's appended rows."""
    gm, om = y2.Model.open(ck), O.Model(ck)
    try:
        assert gm.set_step_kernel(step_kernel) == step_kernel
        ids = synthetic.prompt(96, ck.config.vocab_size, seed=4)
        gc, gl = gm.prefill_phase(ids, 100)
        oc, ol = om.prefill(ids, 100)
        k, v = gc.export()
        ok, ov = oc.arrays()
        assert np.array_equal(bits(k), bits(ok[:, :96])) and np.array_equal(bits(v), bits(ov[:, :96]))
        for s in range(3):
            t = int(np.argmax(ol))
            gm.forward([t], gc)
            ol = om.forward([t], oc)
            n = gc.length
            sk, sv = gc.export(start=n - 1, n=1)
            assert np.array_equal(bits(sk[:, n - 1]), bits(ok[:, n - 1])), f"key rows of step {s}"
            assert np.array_equal(bits(sv[:, n - 1]), bits(ov[:, n - 1])), f"value rows of step {s}"
        gc.close()
    finally:
        gm.close()


@pytest.mark.parametrize("order", ["model-cache-decoder", "model-decoder-cache", "cache-decoder-model"])
def test_any_free_order(ck, order):
    """Free in an order the reference allows (model first among them); the
    detached objects fail cleanly or still export, and a model opened
    afterwards decodes as the oracle does."""
    gm, om = y2.Model.open(ck), O.Model(ck)
    ids = synthetic.prompt(64, ck.config.vocab_size, seed=1)
    gc, gl = gm.prefill_phase(ids, 80)
    dec = y2.Decoder(gm, gc)
    toks, _ = dec.run(3, first_logits=gl)
    oc, want = _oracle_greedy(om, ids, 80, 3)
    assert list(toks) == want
    # each launch forwarded the token chosen before it: the cache holds the
    # prompt and the three tokens, as the oracle's does
    ok, ov = oc.arrays()
    for name in order.split("-"):
        if name == "model":
            gm.close()
            if dec._h:
                with pytest.raises(y2.Yue2Error) as e:
                    dec.run(1)
                assert e.value.code == -13
            if gc._h:
                k, v = gc.export()
                assert k.shape[1] == 67
                assert np.array_equal(bits(k), bits(ok[:, :67])) and np.array_equal(bits(v), bits(ov[:, :67]))
        elif name == "cache":
            gc.close()
            if dec._h and gm._h:
                with pytest.raises(y2.Yue2Error):
                    dec.run(1)
        else:
            dec.close()
    # a new model on the same device after all of that
    gm2 = y2.Model.open(ck)
    try:
        gc2, gl2 = gm2.prefill_phase(ids, 80)
        assert np.array_equal(bits(gl2), bits(gl))
        dec2 = y2.Decoder(gm2, gc2)
        toks2, _ = dec2.run(5, first_logits=gl2)
        _, want5 = _oracle_greedy(om, ids, 80, 5)
        assert list(toks2) == want5
        dec2.close()
        gc2.close()
    finally:
        gm2.close()


def test_c_level_model_first(ck):
    """The same through the C ABI alone: model_free, then cache_free and
    decoder_free on the detached handles (what a Rust Drop order does)."""
    L = y2.lib()
    gm = y2.Model.open(ck)
    ids = np.asarray(synthetic.prompt(32, ck.config.vocab_size, seed=2), np.int32)
    gc, gl = gm.prefill_phase(ids, 48)
    gc2, gl2 = gm.prefill_phase(ids[:20], 48)
    dec = y2.Decoder(gm, gc, gc2, scale=1.5)
    dec.run(2, first_logits=np.concatenate([gl, gl2]))
    h_model, h_cache, h_cache2, h_dec = gm._h, gc._h, gc2._h, dec._h
    gm._h = gc._h = gc2._h = dec._h = None  # the Python mirror frees nothing more
    L.yue2_hip_model_free(h_model)
    assert L.yue2_hip_cache_length(h_cache) == 34
    L.yue2_hip_cache_free(h_cache)
    L.yue2_hip_decoder_free(h_dec)
    L.yue2_hip_cache_free(h_cache2)
    assert L.yue2_hip_synchronize() == 0
