"""The generic step kernels: shapes that have no kernel of their own.

The reference's Metal fast path runs any Config (yue2_metal_ar_stack,
src/metal.m:718-874).  Here a shape with head_dim 64 or 128, at most eight
query heads per KV head, hidden and heads * head_dim up to 4608 and
intermediate up to 14336 runs on a generic step kernel of its head_dim:
every GEMV input masked to its length, the group size taken at run time
(past four query heads per KV head, the scores and PV take them four at a
time).
(The reduced config of the other tests, hidden 1024 / intermediate 2816 /
4 query heads per KV head at head_dim 64, runs on it as well.)  Each shape
below is checked against the oracle bit for bit: a decode-order prefill and
greedy batch-1 steps, CFG batch-2 steps through the captured decoder at
2048 and 8192 positions (both rows' logits), and a sampled CFG generate."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
from yue2_rs_amd.api import Config
import yue2_rs_amd as y2

from helpers import bits

pytestmark = pytest.mark.gpu


def _config(hidden, heads, kv_heads, head_dim, inter):
    return Config(hidden_size=hidden, num_hidden_layers=2, num_attention_heads=heads, num_key_value_heads=kv_heads,
                  head_dim=head_dim, intermediate_size=inter, vocab_size=32768, max_position_embeddings=24576,
                  rms_norm_eps=1e-6, rope_theta=10000.0)


SHAPES = {
    # 4 query heads per KV head at head_dim 128, heads * head_dim != hidden
    "d128-g4": _config(1536, 16, 4, 128, 4608),
    # 2 per KV head; hidden and intermediate not multiples of 512
    "d128-g2": _config(1280, 10, 5, 128, 3456),
    # one per KV head (no grouping) at head_dim 64
    "d64-g1": _config(768, 12, 12, 64, 2048),
    # 3 per KV head at head_dim 64
    "d64-g3": _config(1152, 18, 6, 64, 3072),
    # 8B-class layers (two of them): hidden 4096, 32 x 128 query heads, 4 per
    # KV head, intermediate 14336 (the down projection's input in two
    # gather passes)
    "d128-g4-h4096": _config(4096, 32, 8, 128, 14336),
    # 7B-class layers without grouping, intermediate 11008
    "d128-g1-h4096": _config(4096, 32, 32, 128, 11008),
    # 6, 7 and 8 query heads per KV head (two head passes)
    "d128-g6": _config(1536, 12, 2, 128, 8960),
    "d64-g7": _config(896, 14, 2, 64, 4864),
    "d128-g8": _config(2048, 16, 2, 128, 11008),
}


@pytest.fixture(scope="module", params=list(SHAPES), ids=list(SHAPES))
def shape(request, gpu, oracle_threads):
    ck = synthetic.checkpoint(SHAPES[request.param], seed=3)
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(True), f"{request.param} has a step kernel"
    yield ck, gm, O.Model(ck)
    gm.close()


def test_prefill_and_greedy_batch1(shape):
    ck, gm, om = shape
    ids = synthetic.prompt(96, ck.config.vocab_size, seed=5)
    gcache, glog = gm.prefill_phase(ids, 96 + 24)
    ocache, olog = om.prefill(ids, 96 + 24)
    assert np.array_equal(bits(glog), bits(olog)), "prefill logits differ"
    for step in range(24):
        t = int(np.argmax(olog))
        glog, olog = gm.forward([t], gcache), om.forward([t], ocache)
        assert np.array_equal(bits(glog), bits(olog)), f"logits differ at step {step}"
    gcache.close()


def _caches(gm, om, length, cap, seed):
    oc = O.Cache(om, cap)
    oc.fill_random(length, seed)
    gc = y2.Cache(gm, cap)
    k, v = oc.arrays()
    gc.load(k, v, length)
    return gc, oc


@pytest.mark.parametrize("length", [2048, 8192])
def test_cfg_batch2_both_rows(shape, length):
    ck, gm, om = shape
    V, steps, scale = ck.config.vocab_size, 3, 1.5
    lengths = (length, length - 37)
    (g0, o0), (g1, o1) = (_caches(gm, om, n, n + steps, 11 + i) for i, n in enumerate(lengths))
    dec = y2.Decoder(gm, g0, g1, scale=scale)
    t = 101
    first = np.zeros(2 * V, np.float32)
    first[t] = first[V + t] = 1.0  # the CFG mix of two equal rows: argmax t
    for s in range(steps):
        print(f"contexts {lengths[0] + s}/{lengths[1] + s}, token {t}", flush=True)
        toks, _ = dec.run(1, first_logits=first if s == 0 else None)
        assert list(toks) == [t]
        got = dec.logits()
        w0, w1 = om.forward_rows([t, t], [o0, o1])
        assert np.array_equal(bits(got[0]), bits(w0)), f"conditional row differs at step {s}"
        assert np.array_equal(bits(got[1]), bits(w1)), f"unconditional row differs at step {s}"
        t = int(np.argmax(O.cfg_mix(w0, w1, scale)))
    dec.close()
    for c in (g0, g1):
        c.close()


def test_phase_kernels_cfg_batch2(shape):
    """The same shape on the per-phase kernels (their attention: the step
    kernel's attention body in a launch of its own, the group size at run
    time past two and three query heads per KV head): CFG batch-2 steps
    from 4096-position caches, both rows' logits bit for bit."""
    ck, gm, om = shape
    assert not gm.set_step_kernel(False)
    try:
        V, steps, scale = ck.config.vocab_size, 2, 1.5
        (g0, o0), (g1, o1) = (_caches(gm, om, n, n + steps, 41 + i) for i, n in enumerate((4096, 4059)))
        dec = y2.Decoder(gm, g0, g1, scale=scale)
        t = 123
        first = np.zeros(2 * V, np.float32)
        first[t] = first[V + t] = 1.0
        for s in range(steps):
            toks, _ = dec.run(1, first_logits=first if s == 0 else None)
            assert list(toks) == [t]
            got = dec.logits()
            w0, w1 = om.forward_rows([t, t], [o0, o1])
            assert np.array_equal(bits(got[0]), bits(w0)), f"conditional row differs at step {s}"
            assert np.array_equal(bits(got[1]), bits(w1)), f"unconditional row differs at step {s}"
            t = int(np.argmax(O.cfg_mix(w0, w1, scale)))
        dec.close()
        for c in (g0, g1):
            c.close()
    finally:
        assert gm.set_step_kernel(True)


def test_sampled_cfg_generate(shape):
    """sampling::generate with T 0.9, top-k 50, top-p 0.93, penalty 1.2/50, CFG 1.5."""
    ck, gm, om = shape
    V = ck.config.vocab_size
    s = y2.Sampling(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=0, max_tokens=24)
    pos = synthetic.prompt(80, V, seed=6)
    neg = synthetic.prompt(64, V, seed=7)
    got = y2.generate(gm, pos, s, seed=77, negative=neg, scale=1.5)
    want, trunc = O.generate(om, pos, s, 77, negative=neg, scale=1.5)
    assert got.tokens == want
    assert got.truncated == trunc


def test_shapes_past_the_limits_use_the_phase_kernels(gpu):
    """Hidden 5120, or intermediate 16384, have no step kernel: the model
    decodes on the per-phase kernels."""
    for c in (_config(5120, 40, 8, 128, 4096), _config(2048, 16, 8, 128, 16384)):
        gm = y2.Model.open(synthetic.checkpoint(c, seed=0))
        assert not gm.set_step_kernel(True)
        gm.close()


def test_8b_class_layers_on_the_phase_kernels(gpu, oracle_threads):
    """The per-phase kernels take the same 8B-class layers (intermediate
    14336: the down projection's two staged input rows, 115 KB, in one
    workgroup's LDS): CFG batch-2 logits of both rows bit for bit."""
    ck = synthetic.checkpoint(SHAPES["d128-g4-h4096"], seed=3)
    gm, om = y2.Model.open(ck), O.Model(ck)
    assert not gm.set_step_kernel(False)
    V, steps, scale = ck.config.vocab_size, 2, 1.5
    (g0, o0), (g1, o1) = (_caches(gm, om, n, n + steps, 21 + i) for i, n in enumerate((2048, 2011)))
    dec = y2.Decoder(gm, g0, g1, scale=scale)
    t = 55
    first = np.zeros(2 * V, np.float32)
    first[t] = first[V + t] = 1.0
    for s in range(steps):
        toks, _ = dec.run(1, first_logits=first if s == 0 else None)
        assert list(toks) == [t]
        got = dec.logits()
        w0, w1 = om.forward_rows([t, t], [o0, o1])
        assert np.array_equal(bits(got[0]), bits(w0)), f"conditional row differs at step {s}"
        assert np.array_equal(bits(got[1]), bits(w1)), f"unconditional row differs at step {s}"
        t = int(np.argmax(O.cfg_mix(w0, w1, scale)))
    dec.close()
    for c in (g0, g1):
        c.close()
    gm.close()


# Shapes the per-phase attention hands to its counter-sync body (dev_attn.h)
# instead of the tagged-word one: head_dim 256, and 40 KV heads of 64 at CFG
# batch 2 over caches of 24576 positions (80 (KV head, row) groups leave the
# tagged-word body three workgroups each, and their staged p of 128 blocks
# would outgrow its K region).
PHASE_ONLY = {
    "d256-g2": _config(1024, 4, 2, 256, 2048),
    "d64-kv40": _config(2560, 40, 40, 64, 4096),
}


@pytest.mark.parametrize("name", list(PHASE_ONLY))
def test_counter_sync_attention_shapes(name, gpu, oracle_threads):
    """Batch-1 greedy steps after a decode-order prefill, then CFG batch-2
    steps from 2048-position caches of capacity 24576 through the captured
    decoder: every logit bit for bit against the oracle."""
    ck = synthetic.checkpoint(PHASE_ONLY[name], seed=4)
    gm, om = y2.Model.open(ck), O.Model(ck)
    gm.set_step_kernel(False)
    ids = synthetic.prompt(40, ck.config.vocab_size, seed=5)
    gcache, glog = gm.prefill_phase(ids, 40 + 6)
    ocache, olog = om.prefill(ids, 40 + 6)
    assert np.array_equal(bits(glog), bits(olog)), "prefill logits differ"
    for step in range(6):
        t = int(np.argmax(olog))
        glog, olog = gm.forward([t], gcache), om.forward([t], ocache)
        assert np.array_equal(bits(glog), bits(olog)), f"logits differ at step {step}"
    gcache.close()
    V, steps, scale = ck.config.vocab_size, 2, 1.5
    (g0, o0), (g1, o1) = (_caches(gm, om, n, 24576, 31 + i) for i, n in enumerate((2048, 2011)))
    dec = y2.Decoder(gm, g0, g1, scale=scale)
    t = 77
    first = np.zeros(2 * V, np.float32)
    first[t] = first[V + t] = 1.0
    for s in range(steps):
        print(f"{name}: CFG step {s}, token {t}", flush=True)
        toks, _ = dec.run(1, first_logits=first if s == 0 else None)
        assert list(toks) == [t]
        got = dec.logits()
        w0, w1 = om.forward_rows([t, t], [o0, o1])
        assert np.array_equal(bits(got[0]), bits(w0)), f"conditional row differs at step {s}"
        assert np.array_equal(bits(got[1]), bits(w1)), f"unconditional row differs at step {s}"
        t = int(np.argmax(O.cfg_mix(w0, w1, scale)))
    dec.close()
    for c in (g0, g1):
        c.close()
    gm.close()
