"""CPU: the oracle's MT19937 and `choose` (src/sampling.rs:10-63, 103-215)
against known answers, an independent MT19937 (numpy's RandomState) and
the statistics the exponential race must produce (no GPU)."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

EOD, ABC_END, MUSIC_END, CODEC_OFFSET, CODEC_SIZE = 151643, 151848, 151852, 151853, 32768


def test_mt19937_known_answer():
    g = O.Generator(5489)
    for _ in range(9999):
        g.next_u32()
    assert g.next_u32() == 4123659995  # C++ [rand.predef]: mt19937's 10000th output


@pytest.mark.parametrize("seed", [0, 1, 5489, 2 ** 32 - 1, 2 ** 40 + 7])
def test_mt19937_matches_numpy(seed):
    g = O.Generator(seed)
    ours = np.array([g.next_u32() for _ in range(2000)], dtype=np.uint64)
    # the reference seeds with `seed as u32` (src/sampling.rs:17)
    rs = np.random.RandomState(seed & 0xFFFFFFFF)
    theirs = rs.randint(0, 2 ** 32, size=2000, dtype=np.uint64)
    assert np.array_equal(ours, theirs)


def test_uniform_f64_and_discard():
    a, b = O.Generator(7), O.Generator(7)
    for _ in range(700):
        hi, lo = b.next_u32(), b.next_u32()
        assert a.uniform_f64() == float((hi << 32 | lo) & ((1 << 53) - 1)) / 2.0 ** 53
    for n in [0, 1, 623, 624, 625, 2000, 168000]:
        a, b = O.Generator(11), O.Generator(11)
        a.next_u32()
        b.next_u32()
        a.discard(n)
        for _ in range(n):
            b.next_u32()
        assert a.next_u32() == b.next_u32(), n


def test_prompt_generator_matches_oracle_mt():
    mt, g = synthetic.MT19937(3), O.Generator(3)
    assert [mt.next_u32() for _ in range(1500)] == [g.next_u32() for _ in range(1500)]


def S(**kw):
    base = dict(temperature=1.0, top_p=1.0, top_k=1000000, repetition_penalty=1.0, penalty_window=50,
                min_tokens=0, max_tokens=100)
    base.update(kw)
    return y2.Sampling(**base)


def choose(logits, s, history=(), step=0, phase=O.PHASE_NONE, legacy=False, rng=None):
    rng = rng or O.Generator(0)
    return O.choose(np.asarray(logits, np.float32), s, list(history), step, phase, legacy, rng)


def test_greedy_lowest_index_tie_and_no_rng_use():
    lg = np.array([0.5, 2.0, -np.inf, 2.0, 1.0], np.float32)
    g, ref = O.Generator(9), O.Generator(9)
    assert choose(lg, S(temperature=0.0), rng=g) == 1
    assert g.next_u32() == ref.next_u32()  # T = 0 returns before any draw
    assert choose(lg, S(temperature=0.9, top_k=1)) == 1


@pytest.mark.parametrize("V", [5, 624, 1000, 4097])
def test_sampling_consumes_exactly_2v_draws(V):
    lg = np.random.default_rng(V).standard_normal(V).astype(np.float32)
    g, ref = O.Generator(21), O.Generator(21)
    choose(lg, S(temperature=0.9, top_k=50, top_p=0.93), rng=g)
    ref.discard(2 * V)
    assert g.next_u32() == ref.next_u32()


def _freq(lg, s, n, seed=1, **kw):
    g = O.Generator(seed)
    counts = np.zeros(len(lg), np.int64)
    for _ in range(n):
        counts[choose(lg, s, rng=g, **kw)] += 1
    return counts / n


def test_race_samples_the_softmax():
    lg = np.array([0.3, -1.2, 1.1, 0.0, 0.7, -0.4], np.float32)
    T, n = 0.8, 30000
    p = np.exp(lg / T - np.max(lg / T))
    p /= p.sum()
    f = _freq(lg, S(temperature=T), n)
    sigma = np.sqrt(p * (1 - p) / n)
    assert np.all(np.abs(f - p) <= 5 * sigma), (f, p)


def test_top_p_keeps_the_crossing_token():
    # sorted p = [0.5, 0.3, 0.15, 0.05]; with top_p 0.7 the prior cumulative
    # mass is 0, 0.5, 0.8, 0.95, so ids 0 and 1 survive (src/sampling.rs:175-190)
    p = np.array([0.5, 0.3, 0.15, 0.05])
    lg = np.log(p).astype(np.float32)
    f = _freq(lg, S(top_p=0.7), 20000)
    assert f[2] == 0 and f[3] == 0
    assert abs(f[0] - 0.625) < 5 * np.sqrt(0.625 * 0.375 / 20000)
    # protected tokens: non-legacy keeps only the top one for a tiny top_p,
    # legacy keeps three
    assert np.count_nonzero(_freq(lg, S(top_p=0.01), 3000)) == 1
    assert np.count_nonzero(_freq(lg, S(top_p=0.01), 3000, legacy=True)) == 3


def test_top_k_keeps_ties_at_the_threshold():
    lg = np.array([3.0, 2.0, 2.0, 2.0, 1.0, 0.0], np.float32)
    f = _freq(lg, S(top_k=2), 20000)
    assert f[4] == 0 and f[5] == 0
    assert np.all(f[1:4] > 0)
    assert abs(f[1] - f[3]) < 0.03


def test_repetition_penalty():
    s = S(temperature=0.0, repetition_penalty=1.2)
    assert choose([1.0, 1.1], s, history=[1]) == 0  # 1.1 / 1.2 < 1.0
    assert choose([-1.0, -1.1], s, history=[0]) == 1  # -1.0 * 1.2 < -1.1
    assert choose([1.0, 1.3], s, history=[1]) == 1  # 1.3 / 1.2 > 1.0
    assert choose([1.0, 1.3], s, history=[1, 1]) == 0  # 1.3 / 1.44 < 1.0 (powi of the count)
    # only the last `penalty_window` ids count
    s2 = S(temperature=0.0, repetition_penalty=1.2, penalty_window=2)
    assert choose([1.0, 1.1], s2, history=[1, 0, 0]) == 1


def test_invalid_logits_are_rejected():
    for bad in (np.nan, np.inf):
        with pytest.raises(RuntimeError):
            choose([0.0, bad, 1.0], S(temperature=0.0))
    assert choose([0.0, -np.inf, 1.0], S(temperature=0.0)) == 2


def test_phase_masks():
    V = CODEC_OFFSET + CODEC_SIZE
    lg = np.zeros(V, np.float32)
    lg[EOD + 10] = 9.0  # outside the ABC range
    lg[ABC_END] = 8.0
    lg[500] = 5.0
    s = S(temperature=0.0, min_tokens=4)
    assert choose(lg, s, step=0, phase=O.PHASE_ABC) == 500  # end token gated by min_tokens
    assert choose(lg, s, step=4, phase=O.PHASE_ABC) == ABC_END
    lg[CODEC_OFFSET + 77] = 7.0
    lg[MUSIC_END] = 7.5
    assert choose(lg, s, step=0, phase=O.PHASE_SEMANTIC) == CODEC_OFFSET + 77
    assert choose(lg, s, step=9, phase=O.PHASE_SEMANTIC) == MUSIC_END
    with pytest.raises(RuntimeError):
        choose(np.zeros(CODEC_OFFSET + 5, np.float32), s, phase=O.PHASE_SEMANTIC)
    with pytest.raises(RuntimeError):
        choose(np.zeros(1000, np.float32), s, phase=O.PHASE_ABC)


# ---------------------------------------------------------------------------
# sampling::generate's loop (src/sampling.rs:222-294), restated in Python over
# the oracle's separately pinned parts (prefill / forward_phase, the CFG mix,
# choose, MT19937), against the oracle's own y2o_generate.

def _generate_loop(om, prefix, s, seed, phase, negative, scale, legacy):
    cache, cond = om.prefill(prefix, len(prefix) + s.max_tokens, phase)
    ncache = unc = None
    if scale != 1.0:
        ncache, unc = om.prefill(negative, len(negative) + s.max_tokens, phase)
    end = {O.PHASE_ABC: ABC_END, O.PHASE_SEMANTIC: MUSIC_END}.get(phase, -1)
    gen = O.Generator(seed)
    tokens, truncated = [], True
    for step in range(s.max_tokens):
        logits = O.cfg_mix(cond, unc, scale) if unc is not None else cond
        t = O.choose(logits, s, tokens, step, phase, legacy, gen)
        if t == end:
            truncated = False
            break
        tokens.append(t)
        if step + 1 < s.max_tokens:
            cond = om.forward_phase([t], cache, phase)
            if ncache is not None:
                unc = om.forward_phase([t], ncache, phase)
    return tokens, truncated


LOOP = y2.Config(hidden_size=128, num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1, head_dim=64,
                 intermediate_size=256, vocab_size=184704, max_position_embeddings=256, rms_norm_eps=1e-6,
                 rope_theta=1e6)


@pytest.fixture(scope="module")
def loop_models():
    """Two models with the protocol's vocabulary: `plain` (random), and
    `ending` whose ABC_END / MUSIC_END rows win once min_tokens lets them
    (every embedding carries 4.0 in dimension 0, which only those two LM-head
    rows weigh)."""
    plain = synthetic.checkpoint(LOOP, seed=21)
    ending = synthetic.checkpoint(LOOP, seed=22)
    ending.embed_tokens[:, 0] = 0x4080
    ending.lm_head[:, 0] = 0
    ending.lm_head[ABC_END, 0] = 0x3F80
    ending.lm_head[MUSIC_END, 0] = 0x3F80
    return {"plain": O.Model(plain), "ending": O.Model(ending)}


@pytest.mark.parametrize("model,phase,temperature,scale,legacy,min_tokens", [
    ("ending", O.PHASE_SEMANTIC, 0.9, 1.5, False, 4),   # end stop after min_tokens, CFG
    ("ending", O.PHASE_ABC, 0.0, 1.0, True, 3),         # greedy, end stop, legacy
    ("plain", O.PHASE_SEMANTIC, 0.9, 1.5, True, 0),     # truncated at max_tokens, CFG, legacy
    ("plain", O.PHASE_ABC, 1.3, 1.0, False, 0),         # sampled batch 1
])
def test_generate_matches_its_loop(loop_models, model, phase, temperature, scale, legacy, min_tokens):
    om = loop_models[model]
    s = y2.Sampling(temperature=temperature, top_p=0.9, top_k=40, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=min_tokens, max_tokens=12)
    prefix = synthetic.prompt(30, EOD, seed=1)
    negative = synthetic.prompt(17, EOD, seed=2) if scale != 1.0 else None  # a different length
    want = _generate_loop(om, prefix, s, 99, phase, negative, scale, legacy)
    got = O.generate(om, prefix, s, 99, phase=phase, negative=negative, scale=scale, legacy=legacy)
    assert got == want
    if model == "ending":
        assert want[1] is False and len(want[0]) == min_tokens, "the construction must stop at min_tokens"
    else:
        assert want[1] is True and len(want[0]) == s.max_tokens
