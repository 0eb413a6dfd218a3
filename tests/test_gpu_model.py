"""Full token step on the GPU against the oracle: logits bit-exact at every
step, greedy ids equal, for the reduced config (256-token prompt, 64 greedy
steps), a short run of the 3B-class config, and 256 greedy tokens of the
full 3B-class model through the device decode loop, batch 1 and CFG."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def reduced(gpu, oracle_threads):
    ck = synthetic.checkpoint(synthetic.REDUCED, seed=0)
    return ck, y2.Model.open(ck), O.Model(ck)


@pytest.mark.parametrize("step_kernel", [False, True], ids=["phase-kernels", "step-kernel"])
def test_reduced_prefill_and_64_greedy_steps(reduced, step_kernel):
    ck, gm, om = reduced
    assert gm.set_step_kernel(step_kernel) == step_kernel
    ids = synthetic.prompt(256, ck.config.vocab_size, seed=0)
    gcache, glog = gm.prefill_phase(ids, 256 + 64)
    ocache, olog = om.prefill(ids, 256 + 64)
    assert np.array_equal(_bits(glog), _bits(olog)), "prefill logits differ"
    for step in range(64):
        gt, ot = int(np.argmax(glog)), int(np.argmax(olog))
        assert gt == ot, f"greedy id differs at step {step}"
        glog = gm.forward([gt], gcache)
        olog = om.forward([ot], ocache)
        assert np.array_equal(_bits(glog), _bits(olog)), f"logits differ at step {step}"
    assert gcache.length == ocache.length == 256 + 64


@pytest.mark.parametrize("step_kernel", [False, True], ids=["phase-kernels", "step-kernel"])
def test_3b_short_run_bit_exact(gpu, oracle_threads, step_kernel):
    ck = synthetic.checkpoint(synthetic.CLASS_3B, seed=0)
    gm, om = y2.Model.open(ck), O.Model(ck)
    assert gm.set_step_kernel(step_kernel) == step_kernel
    ids = synthetic.prompt(20, ck.config.vocab_size, seed=0)
    gcache, glog = gm.prefill_phase(ids, 32)
    ocache, olog = om.prefill(ids, 32)
    assert np.array_equal(_bits(glog), _bits(olog))
    for step in range(4):
        t = int(np.argmax(olog))
        glog, olog = gm.forward([t], gcache), om.forward([t], ocache)
        assert np.array_equal(_bits(glog), _bits(olog)), f"3B logits differ at step {step}"
    gm.close()


@pytest.fixture(scope="module")
def full_3b(gpu, oracle_threads):
    ck = synthetic.checkpoint(synthetic.CLASS_3B, seed=0)
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(True)
    yield ck, gm, O.Model(ck)
    gm.close()


def _first_difference(got, want):
    return next((i for i, (a, b) in enumerate(zip(got, want)) if int(a) != b), None)


def test_3b_256_greedy_tokens_through_the_decode_loop(full_3b):
    """The horizon the bit-exactness claim is made for: 256 greedy tokens of
    the full 28-layer 3B-class model through the device decode loop (the
    step kernel with its fused sampler, one launch per token; greedy choice
    as sampling::generate makes it at temperature 0, src/sampling.rs:258-291)
    against the oracle's loop: argmax of each step's logits, fed back.  The
    ids must be equal at every step, and the prefill's logits bit for bit."""
    ck, gm, om = full_3b
    V, steps = ck.config.vocab_size, 256
    ids = synthetic.prompt(16, V, seed=4)
    gcache, glog = gm.prefill_phase(ids, 16 + steps)
    dec = y2.Decoder(gm, gcache)
    toks, _ = dec.run(steps, first_logits=glog)
    dec.close()
    ocache, olog = om.prefill(ids, 16 + steps)
    assert np.array_equal(_bits(glog), _bits(olog))
    want = []
    for step in range(steps):
        t = int(np.argmax(olog))
        want.append(t)
        if step < len(toks) and int(toks[step]) != t:
            break
        if step + 1 < steps:
            olog = om.forward([t], ocache)
    print(f"256 greedy 3B tokens: first difference at {_first_difference(toks, want)}", flush=True)
    assert list(toks) == want


def test_3b_256_cfg_greedy_tokens_through_the_decode_loop(full_3b):
    """The same for CFG batch 2 (guidance 1.5): each step the device mixes
    the two rows' logits (CfgMix) and takes the greedy id, which both rows
    then consume; the oracle replays the mix and the argmax."""
    ck, gm, om = full_3b
    V, steps, scale = ck.config.vocab_size, 256, 1.5
    pos, neg = synthetic.prompt(12, V, seed=5), synthetic.prompt(9, V, seed=6)
    c1, l1 = gm.prefill_phase(pos, 12 + steps)
    c2, l2 = gm.prefill_phase(neg, 9 + steps)
    dec = y2.Decoder(gm, c1, c2, scale=scale)
    toks, _ = dec.run(steps, first_logits=np.concatenate([l1, l2]))
    dec.close()
    o1, ol1 = om.prefill(pos, 12 + steps)
    o2, ol2 = om.prefill(neg, 9 + steps)
    assert np.array_equal(_bits(l1), _bits(ol1)) and np.array_equal(_bits(l2), _bits(ol2))
    want = []
    for step in range(steps):
        t = int(np.argmax(O.cfg_mix(ol1, ol2, scale)))
        want.append(t)
        if step < len(toks) and int(toks[step]) != t:
            break
        if step + 1 < steps:
            ol1, ol2 = om.forward_rows([t, t], [o1, o2])
    print(f"256 CFG greedy 3B tokens: first difference at {_first_difference(toks, want)}", flush=True)
    assert list(toks) == want
