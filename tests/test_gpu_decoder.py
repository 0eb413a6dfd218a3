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
        ol1, ol2 = om.forward_rows([t, t], [o1, o2])
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


_LEGACY_WANT = {}


@pytest.mark.parametrize("scale,temperature,top_k,seed,steps,sensitive", [
    (1.0, 0.9, 50, 1234, 24, True), (1.0, 0.9, 65, 1234, 24, True),
    (1.5, 1.5, 50, 1, 16, True), (1.5, 1.5, 65, 1, 16, False)])
def test_generate_legacy_matches_oracle(reduced, scale, temperature, top_k, seed, steps, sensitive):
    """Legacy rounding (cast, src/sampling.rs:100-102: the penalty factors,
    the tempered scores, the nucleus probabilities and cumulative sums, the
    race noise and scores rounded to BF16, three ids protected) on the
    device loop: top-k 50 runs the step kernel's fused sampler, top-k 65 the
    sampler kernels (after the step kernel or the per-phase kernels).  Where
    `sensitive`, the oracle's legacy ids differ from its plain ids over the
    horizon, so a device loop that ignored the flag would fail."""
    ck, gm, om = reduced
    V = ck.config.vocab_size
    s = y2.Sampling(temperature=temperature, top_p=0.93, top_k=top_k, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=0, max_tokens=steps)
    pos = synthetic.prompt(256, V, seed=0)
    neg = synthetic.prompt(256, V, seed=1) if scale != 1.0 else None
    key = (scale, temperature, top_k, seed, steps)
    if key not in _LEGACY_WANT:
        want, trunc = O.generate(om, pos, s, seed, negative=neg, scale=scale, legacy=True)
        plain, _ = O.generate(om, pos, s, seed, negative=neg, scale=scale, legacy=False)
        _LEGACY_WANT[key] = (want, trunc, plain)
    want, trunc, plain = _LEGACY_WANT[key]
    assert (want != plain) == sensitive
    got = y2.generate(gm, pos, s, seed=seed, negative=neg, scale=scale, legacy=True)
    assert got.tokens == want
    assert got.truncated == trunc


@pytest.mark.parametrize("scale", [1.0, 1.5])
def test_generate_with_matrix_core_prefill(reduced, scale):
    """generate() with the matrix-core prefill (yue2_hip_model_set_prefill):
    the prompts' caches and first logits follow the MFMA tolerance contract,
    and the loop after them is exact on those caches.  So the same prompts
    prefilled through prefill_mfma (deterministic), exported into oracle
    caches and replayed by the oracle from the MFMA first logits give the
    generated ids."""
    ck, gm, om = reduced
    V = ck.config.vocab_size
    s = y2.Sampling(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=0, max_tokens=24)
    prompts = [synthetic.prompt(300, V, seed=0)] + ([synthetic.prompt(280, V, seed=1)] if scale != 1.0 else [])
    assert gm.set_prefill_mfma(True)
    try:
        got = y2.generate(gm, prompts[0], s, seed=321, negative=prompts[1] if scale != 1.0 else None, scale=scale)
    finally:
        assert not gm.set_prefill_mfma(False)
    ocs, logits = [], []
    for ids in prompts:
        gc, gl = gm.prefill_mfma(ids, len(ids) + 24)
        k, v = gc.export()
        oc = O.Cache(om, len(ids) + 24)
        oc.load(k, v, len(ids))
        gc.close()
        _, ol = om.prefill(ids, len(ids) + 1)
        d = np.abs(gl - ol).max()
        assert d <= 0.08 * ol.std(), f"MFMA prefill logits {d} from the oracle's"
        ocs.append(oc)
        logits.append(gl)
    gen = O.Generator(321)
    want = []
    for step in range(s.max_tokens):
        mixed = O.cfg_mix(logits[0], logits[1], scale) if scale != 1.0 else logits[0]
        t = O.choose(mixed, s, want, step, y2.PHASE_NONE, False, gen)
        want.append(t)
        if step + 1 < s.max_tokens:
            logits = list(om.forward_rows([t] * len(ocs), ocs))
    assert got.tokens == want and got.truncated


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
        ol1, ol2 = om.forward_rows([t, t], [o1, o2])
    assert list(toks) == want
    gm.close()


@pytest.fixture(scope="module")
def tied(gpu, oracle_threads):
    """The reduced model with exact ties at the top of every step's logits:
    every embedding carries 4.0 in dimension 0, which stays the largest
    entry of the final hidden state, and LM-head rows [0, 3000) weigh that
    dimension alone (1.0), so those 3000 logits are all rb(y[0])."""
    ck = synthetic.checkpoint(synthetic.REDUCED, seed=2)
    ck.embed_tokens[:, 0] = 0x4080  # BF16 4.0
    ck.lm_head[:3000] = 0
    ck.lm_head[:3000, 0] = 0x3F80   # BF16 1.0
    gm = y2.Model.open(ck)
    assert gm.set_step_kernel(True)
    yield ck, gm, O.Model(ck)
    gm.close()


@pytest.mark.parametrize("ties", [100, 3000])
@pytest.mark.parametrize("top_k,top_p,scale", [(50, 0.93, 1.0), (64, 1.0, 1.5), (50, 0.93, 1.5), (65, 0.93, 1.0)])
def test_sampler_with_ties_at_the_top(tied, ties, top_k, top_p, scale):
    """choose() where the top-k threshold is tied across and within the step
    kernel's per-workgroup candidate lists: 100 ties (one list cut at the
    threshold, its rows rescanned) and 3000 (more survivors than the LDS
    arrays hold).  top_k 65 exceeds the fused lists and runs the separate
    sampler kernels."""
    ck, gm, om = tied
    if ties != 3000:
        # rows [ties, 3000) back to random rows of their own
        ck = synthetic.checkpoint(synthetic.REDUCED, seed=2)
        ck.embed_tokens[:, 0] = 0x4080
        ck.lm_head[:ties] = 0
        ck.lm_head[:ties, 0] = 0x3F80
        gm = y2.Model.open(ck)
        om = O.Model(ck)
    V = ck.config.vocab_size
    s = y2.Sampling(temperature=0.9, top_p=top_p, top_k=top_k, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=0, max_tokens=8)
    pos = synthetic.prompt(40, V, seed=5)
    neg = synthetic.prompt(30, V, seed=6) if scale != 1.0 else None
    got = y2.generate(gm, pos, s, seed=99, negative=neg, scale=scale)
    want, trunc = O.generate(om, pos, s, 99, negative=neg, scale=scale)
    assert got.tokens == want and got.truncated == trunc
    assert all(t < ties for t in want), "the tied rows carry all the probability"
