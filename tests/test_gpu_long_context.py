"""The persistent step kernel where the benchmark runs it: long contexts.

Each workgroup of an attention group takes bpw = ceil(blocks / workgroups)
64-key blocks; past kAttnChunk = 3 blocks it restages K/V chunks through LDS.
The reduced config (4 KV heads) reaches bpw 1..6 at batch 1 and 2..12 at
batch 2 between 2048 and 24575 positions; the 3B config (8 KV heads) at
~3100 positions has bpw 2 at batch 1 and 4 at batch 2.  Caches are filled
with BF16-exact N(0, 1) keys and values through the host-mirror load (the
Metal bridge's contextEntry, src/metal.m:633-666) instead of an O(L^2)
prefill; the oracle holds the same mirror.  Logits of every row are compared
bit for bit with the oracle's Model::forward (src/model.rs:465-468,
:313-397 for the attention), batch 2 through the CFG decoder's captured
graph (both rows' logits, not only the chosen ids)."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

from helpers import bits

pytestmark = pytest.mark.gpu

CONTEXTS = [2048, 3100, 8192, 24575]


@pytest.fixture(scope="module")
def reduced(gpu, oracle_threads):
    ck = synthetic.checkpoint(synthetic.REDUCED, seed=0)
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(True)
    yield ck, gm, O.Model(ck)
    gm.close()


def _caches(gm, om, length, cap, seed):
    oc = O.Cache(om, cap)
    oc.fill_random(length, seed)
    gc = y2.Cache(gm, cap)
    k, v = oc.arrays()
    gc.load(k, v, length)
    assert gc.length == length
    return gc, oc


def _one_hot(vocab, t, rows):
    x = np.zeros(vocab, np.float32)
    x[t] = 1.0
    return np.concatenate([x] * rows)


def _check_batch1(gm, om, length, steps, seed):
    gc, oc = _caches(gm, om, length, length + steps, seed)
    t = 17 + seed
    for s in range(steps):
        print(f"batch 1: context {length + s}, token {t}", flush=True)
        got = gm.forward([t], gc)
        want = om.forward([t], oc)
        assert np.array_equal(bits(got), bits(want)), f"logits differ at context {length + s}"
        t = int(np.argmax(want))
    assert gc.length == length + steps


def _check_batch2(gm, om, lengths, steps, seed, scale=1.5):
    V = om.config.vocab_size
    (g0, o0), (g1, o1) = (_caches(gm, om, n, n + steps, seed + i) for i, n in enumerate(lengths))
    dec = y2.Decoder(gm, g0, g1, scale=scale)
    t = 29 + seed
    first = _one_hot(V, t, 2)  # the CFG mix of two equal rows: argmax t
    ids = []
    for s in range(steps):
        print(f"batch 2: contexts {lengths[0] + s}/{lengths[1] + s}, token {t}", flush=True)
        toks, _ = dec.run(1, first_logits=first if s == 0 else None)
        assert list(toks) == [t]
        ids.append(t)
        got = dec.logits()
        w0, w1 = om.forward_rows([t, t], [o0, o1])
        assert np.array_equal(bits(got[0]), bits(w0)), f"conditional row differs at step {s}"
        assert np.array_equal(bits(got[1]), bits(w1)), f"unconditional row differs at step {s}"
        t = int(np.argmax(O.cfg_mix(w0, w1, scale)))
    dec.close()
    assert g0.length == lengths[0] + steps and g1.length == lengths[1] + steps


@pytest.mark.parametrize("length", CONTEXTS)
def test_reduced_batch1_long_context(reduced, length):
    _, gm, om = reduced
    _check_batch1(gm, om, length, 2 if length + 2 <= 24576 else 1, seed=length % 7)


@pytest.mark.parametrize("length", CONTEXTS)
def test_reduced_cfg_batch2_long_context(reduced, length):
    """Both rows at different positions (37 apart), so their groups differ in
    blocks and in which workgroup owns the new key."""
    _, gm, om = reduced
    _check_batch2(gm, om, (length, length - 37), 2 if length + 2 <= 24576 else 1, seed=length % 5)


@pytest.fixture(scope="module")
def model_3b(gpu, oracle_threads):
    ck = synthetic.checkpoint(synthetic.CLASS_3B, seed=0, threads=16)
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(True)
    yield ck, gm, O.Model(ck)
    gm.close()


def test_3b_batch1_context_3100(model_3b):
    _, gm, om = model_3b
    _check_batch1(gm, om, 3100, 2, seed=3)


def test_3b_cfg_batch2_context_3100(model_3b):
    """The benchmark's shape at bpw 4 (the chunk-restage path) for both rows."""
    _, gm, om = model_3b
    _check_batch2(gm, om, (3100, 3063), 2, seed=4)


def test_3b_cfg_sampled_context_2048(model_3b):
    """Config 4's loop at its own context: CFG batch 2 (guidance 1.5) with T
    0.9, top-k 50, top-p 0.93 and penalty 1.2 over 50 tokens, from caches of
    2048 positions, against sampling::generate's loop (src/sampling.rs:
    258-291) replayed on the oracle: the mix, choose() with the generated
    tokens as history and the same MT19937 stream, then each row's forward."""
    _, gm, om = model_3b
    V, steps, seed, scale = om.config.vocab_size, 6, 1234, 1.5
    s = y2.Sampling(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=0, max_tokens=steps)
    (g0, o0), (g1, o1) = (_caches(gm, om, 2048, 2048 + steps, 11 + i) for i in range(2))
    rng = np.random.default_rng(5)
    first = [(3.0 * rng.standard_normal(V)).astype(np.float32) for _ in range(2)]
    dec = y2.Decoder(gm, g0, g1, sampling=s, seed=seed, scale=scale)
    got, _ = dec.run(steps, first_logits=np.concatenate(first))
    dec.close()
    gen = O.Generator(seed)
    cond, uncond = first
    want = []
    for step in range(steps):
        t = O.choose(O.cfg_mix(cond, uncond, scale), s, want, step, y2.PHASE_NONE, False, gen)
        want.append(t)
        print(f"sampled CFG step {step}: oracle {t}, device {int(got[step]) if step < len(got) else None}", flush=True)
        if step + 1 < steps:
            cond, uncond = om.forward_rows([t, t], [o0, o1])
    assert list(got) == want


def test_3b_cfg_batch2_max_context(model_3b):
    """Config 5's end point: the new tokens at positions 24575 and 24000, so
    the attention of each row spans 384 / 376 blocks, 24 per workgroup."""
    _, gm, om = model_3b
    _check_batch2(gm, om, (24575, 24000), 1, seed=5)


@pytest.fixture(scope="module")
def model_yue2(gpu, oracle_threads):
    import dataclasses
    c = dataclasses.replace(synthetic.YUE2, num_hidden_layers=2)
    ck = synthetic.checkpoint(c, seed=1, threads=16)
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(True)
    yield ck, gm, O.Model(ck)
    gm.close()


def test_yue2_batch1_context_8192(model_yue2):
    _, gm, om = model_yue2
    _check_batch1(gm, om, 8192, 2, seed=6)


def test_yue2_cfg_batch2_context_8192(model_yue2):
    """The YuE2 shape's step kernel (two query heads per KV head) on the
    chunk-restage path for both rows."""
    _, gm, om = model_yue2
    _check_batch2(gm, om, (8192, 8150), 2, seed=7)


def test_yue2_cfg_batch2_max_context(model_yue2):
    _, gm, om = model_yue2
    _check_batch2(gm, om, (24575, 24100), 1, seed=8)


@pytest.fixture(scope="module")
def phase_3b(gpu, oracle_threads):
    """Two layers of the 3B shape (24 query / 8 KV heads, head_dim 128) on
    the per-phase kernels: the split-KV attention kernel of the decode
    attention microbenchmark."""
    import dataclasses
    c = dataclasses.replace(synthetic.CLASS_3B, num_hidden_layers=2, vocab_size=32768)
    ck = synthetic.checkpoint(c, seed=2, threads=16)
    gm = y2.Model.open(ck)
    assert not gm.set_step_kernel(False)
    yield ck, gm, O.Model(ck)
    gm.close()


@pytest.mark.parametrize("length", [1024, 4096, 16384, 24575])
def test_phase_kernels_cfg_batch2_attention_lengths(phase_3b, length):
    """The attention microbenchmark's KV lengths at CFG batch 2 through the
    per-phase split-KV attention: both rows' logits bit for bit."""
    _, gm, om = phase_3b
    _check_batch2(gm, om, (length, length - 21), 1, seed=length % 11)


def test_epoch_repeat_keeps_parity(reduced):
    """The step kernel's tagged words carry a 20-bit epoch of the launch
    sequence.  The second forward below is placed exactly 2^20 launches after
    the first, so without a clear of the words every word the first launch
    left (x, q/k/v, the block statistics of all 129 blocks) would already
    carry the second launch's tags; the library clears them first."""
    _, gm, om = reduced
    gc, oc = _caches(gm, om, 8192, 8196, seed=2)
    t = 11
    for s in range(3):
        if s == 1:
            # the forward's state reset adds 2: the next launch's sequence is
            # the previous launch's + 2^20
            gm.advance_sequence((1 << 20) - 3)
        print(f"forward {s} at context {8192 + s}", flush=True)
        got = gm.forward([t], gc)
        want = om.forward([t], oc)
        assert np.array_equal(bits(got), bits(want)), f"logits differ at forward {s}"
        t = int(np.argmax(want))
