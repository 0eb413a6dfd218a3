"""The captured decode loop (one hipGraph per token) against the oracle:
greedy batch 1, CFG batch 2 greedy, and full sampling::generate with
temperature / top-k / top-p / repetition penalty / CFG on the device, token
ids bit-exact over the horizon."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

from helpers import bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", params=[False, True], ids=["phase-kernels", "step-kernel"])
def reduced(request, gpu, oracle_threads):
    ck = synthetic.checkpoint(synthetic.REDUCED, seed=0)
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(request.param) == request.param
    return ck, gm, O.Model(ck)


def test_greedy_decoder_matches_forward_loop(reduced):
    ck, gm, om = reduced
    ids = synthetic.prompt(300, ck.config.vocab_size, seed=0)
    cache, first = gm.prefill_phase(ids, 300 + 40)
    dec = y2.Decoder(gm, cache)
    toks, _ = dec.run(40, first_logits=first)
    dec.close()
    ocache, olog = om.prefill(ids, 300 + 40)
    want = []
    for _ in range(40):
        t = int(np.argmax(olog))
        want.append(t)
        olog = om.forward([t], ocache)
    assert list(toks) == want
    assert cache.length == 340


def test_cfg_greedy_decoder_matches_oracle(reduced):
    ck, gm, om = reduced
    V = ck.config.vocab_size
    pos = synthetic.prompt(260, V, seed=0)
    neg = synthetic.prompt(200, V, seed=1)
    steps, scale = 24, 1.5
    c1, l1 = gm.prefill_phase(pos, 260 + steps)
    c2, l2 = gm.prefill_phase(neg, 200 + steps)
    dec = y2.Decoder(gm, c1, c2, scale=scale)
    toks, _ = dec.run(steps, first_logits=np.concatenate([l1, l2]))
    o1, ol1 = om.prefill(pos, 260 + steps)
    o2, ol2 = om.prefill(neg, 200 + steps)
    assert np.array_equal(bits(l1), bits(ol1)) and np.array_equal(bits(l2), bits(ol2))
    want = []
    for _ in range(steps):
        t = int(np.argmax(O.cfg_mix(ol1, ol2, scale)))
        want.append(t)
        ol1, ol2 = om.forward([t], o1), om.forward([t], o2)
    assert list(toks) == want


@pytest.mark.parametrize("scale", [1.0, 1.5])
def test_generate_sampling_matches_oracle(reduced, scale):
    """sampling::generate with T 0.9, top-k 50, top-p 0.93, penalty 1.2/50."""
    ck, gm, om = reduced
    V = ck.config.vocab_size
    s = y2.Sampling(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=0, max_tokens=32)
    pos = synthetic.prompt(256, V, seed=0)
    neg = synthetic.prompt(256, V, seed=1) if scale != 1.0 else None
    got = y2.generate(gm, pos, s, seed=1234, negative=neg, scale=scale)
    want, trunc = O.generate(om, pos, s, 1234, negative=neg, scale=scale)
    assert got.tokens == want
    assert got.truncated == trunc


def test_generate_greedy_with_penalty_matches_oracle(reduced):
    ck, gm, om = reduced
    s = y2.Sampling(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=0, max_tokens=20)
    pos = synthetic.prompt(256, ck.config.vocab_size, seed=3)
    got = y2.generate(gm, pos, s, seed=0)
    want, _ = O.generate(om, pos, s, 0)
    assert got.tokens == want


def test_generate_rejects_bad_requests(reduced):
    ck, gm, _ = reduced
    s = y2.Sampling(max_tokens=10, min_tokens=0)
    with pytest.raises(y2.Yue2Error) as e:
        y2.generate(gm, [1, 2, 3], s, seed=0, scale=1.5)
    assert e.value.code == -8
    with pytest.raises(y2.Yue2Error) as e:
        y2.generate(gm, [1, 2, 3], y2.Sampling(top_k=0, max_tokens=4, min_tokens=0), seed=0)
    assert e.value.code == -6
    with pytest.raises(y2.Yue2Error) as e:
        y2.generate(gm, [1] * 24570, y2.Sampling(max_tokens=10, min_tokens=0), seed=0)
    assert e.value.code == -7
    with pytest.raises(y2.Yue2Error) as e:
        y2.generate(gm, [1, 2, 3], s, seed=0, phase=y2.PHASE_SEMANTIC)
    assert e.value.code == -3


def test_3b_cfg_greedy_step_kernel_matches_oracle(gpu, oracle_threads):
    """Batch-2 CFG through the 3B-shape step kernel (head_dim 128, GQA 3)."""
    ck = synthetic.checkpoint(synthetic.CLASS_3B, seed=0)
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(True)
    om = O.Model(ck)
    V = ck.config.vocab_size
    pos = synthetic.prompt(9, V, seed=0)
    neg = synthetic.prompt(6, V, seed=1)
    steps, scale = 3, 1.5
    c1, l1 = gm.prefill_phase(pos, 16)
    c2, l2 = gm.prefill_phase(neg, 16)
    dec = y2.Decoder(gm, c1, c2, scale=scale)
    toks, _ = dec.run(steps, first_logits=np.concatenate([l1, l2]))
    dec.close()
    o1, ol1 = om.prefill(pos, 16)
    o2, ol2 = om.prefill(neg, 16)
    assert np.array_equal(bits(l1), bits(ol1)) and np.array_equal(bits(l2), bits(ol2))
    want = []
    for _ in range(steps):
        t = int(np.argmax(O.cfg_mix(ol1, ol2, scale)))
        want.append(t)
        ol1, ol2 = om.forward([t], o1), om.forward([t], o2)
    assert list(toks) == want
    gm.close()
