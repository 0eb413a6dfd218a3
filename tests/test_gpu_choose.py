"""sampling::choose (src/sampling.rs:103-215) on the device against the
oracle, one call at a time through yue2_hip_choose.

The device selects through per-chunk candidate lists (top_k up to the list
bound) or a single workgroup over the whole vocabulary (larger top_k); both
must return the oracle's id for the same logits, history, step and MT19937
draws.  The cases aim at what the chunked selection could get wrong: ties at
the top-k threshold inside and across chunks, lists cut short in the middle
of a run of ties, -0.0 / +0.0 at the threshold, ragged last chunks, the
phase masks, the penalty window, and the error rules."""
import numpy as np
import pytest

from oracle import oracle as O
import yue2_rs_amd as y2

pytestmark = pytest.mark.gpu

V3B = 84000  # vocabulary of the 3B-class configuration
EOD, ABC_END, MUSIC_END, CODEC_OFFSET, CODEC_SIZE = 151643, 151848, 151852, 151853, 32768
V_PHASE = CODEC_OFFSET + CODEC_SIZE + 11


def draws(seed, v):
    # numpy's RandomState is MT19937 with the same seeding; the CPU tests pin
    # it against the oracle's generator output by output.
    return np.random.RandomState(seed & 0xFFFFFFFF).randint(0, 2 ** 32, size=2 * v,
                                                            dtype=np.uint64).astype(np.uint32)


def S(**kw):
    base = dict(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                min_tokens=0, max_tokens=100)
    base.update(kw)
    return y2.Sampling(**base)


def both(logits, s, history=(), step=0, phase=O.PHASE_NONE, legacy=False, seed=0):
    lg = np.ascontiguousarray(logits, np.float32)
    d = draws(seed, len(lg))
    dev = y2.choose(lg, s, list(history), step, phase, legacy, d)
    ref = O.choose(lg, s, list(history), step, phase, legacy, O.Generator(seed))
    return dev, ref


def normal(v, seed, scale=3.0):
    return (np.random.default_rng(seed).standard_normal(v) * scale).astype(np.float32)


def top_history(lg, n, seed):
    """n ids drawn from the 200 best entries, with repeats."""
    best = np.argsort(-lg, kind="stable")[:200]
    return np.random.default_rng(seed + 99).choice(best, n).tolist()


@pytest.mark.parametrize("legacy", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_typical_settings(gpu, seed, legacy):
    lg = normal(V3B, seed)
    h = top_history(lg, 60, seed)
    dev, ref = both(lg, S(), h, len(h), legacy=legacy, seed=seed)
    assert dev == ref


@pytest.mark.parametrize("kw", [
    dict(temperature=1.0, top_p=0.95, top_k=100, repetition_penalty=1.2, penalty_window=50),
    dict(temperature=0.7, top_p=0.9, top_k=30, repetition_penalty=1.005, penalty_window=100),
    dict(temperature=1.3, top_p=1.0, top_k=1),
    dict(temperature=2.0, top_p=1.0, top_k=197),   # the most the chunked lists hold at this vocabulary
    dict(temperature=2.0, top_p=1.0, top_k=198),   # one more: the single-workgroup path
    dict(temperature=1.0, top_p=0.99, top_k=1000),
    dict(temperature=5.0, top_p=0.5, top_k=120),
], ids=["default", "legacy-preset", "k1", "k197", "k198", "k1000", "hot"])
@pytest.mark.parametrize("seed", [4, 5])
def test_settings_and_both_paths(gpu, kw, seed):
    lg = normal(V3B, seed, scale=1.5)
    h = top_history(lg, 40, seed)
    dev, ref = both(lg, S(**kw), h, 40, seed=seed)
    assert dev == ref


@pytest.mark.parametrize("top_p", [1.0, 0.93])
@pytest.mark.parametrize("seed", range(6))
def test_ties_everywhere(gpu, seed, top_p):
    # scores on a grid of 0.5: long runs of exact ties, the threshold inside one
    lg = (np.round(normal(V3B, seed, scale=2.0) * 2) / 2).astype(np.float32)
    dev, ref = both(lg, S(top_p=top_p, top_k=50, temperature=1.0, repetition_penalty=1.0), seed=seed)
    assert dev == ref


@pytest.mark.parametrize("seed", range(8))
def test_ties_cut_inside_chunk_lists(gpu, seed):
    # 10 entries at 6.0, then 80 ties at 5.0 in chunk 0 and 60 in chunk 5:
    # top-50's threshold is 5.0 and both chunks' lists stop inside their runs
    # of ties, so all 150 tied entries must be recovered from the scores.
    lg = np.full(V3B, -1.0, np.float32)
    rng = np.random.default_rng(seed)
    lg[rng.choice(np.arange(20000, 30000), 10, replace=False)] = 6.0
    lg[100:180] = 5.0
    lg[5 * 1024 + 7:5 * 1024 + 67] = 5.0
    lg[40000:41000] = 4.5
    s = S(top_p=1.0, top_k=50, temperature=1.0, repetition_penalty=1.0)
    dev, ref = both(lg, s, seed=seed)
    assert dev == ref


@pytest.mark.parametrize("seed", range(6))
def test_signed_zero_threshold(gpu, seed):
    # 20 entries at 1.0; 100 entries of -0.0 in chunk 0 and 100 of +0.0 in
    # chunk 1; the rest -1.  The threshold is +0.0 and -0.0 >= +0.0, so all
    # 200 zeros survive, half of them beyond chunk 0's list.
    lg = np.full(V3B, -1.0, np.float32)
    rng = np.random.default_rng(seed)
    lg[rng.choice(np.arange(50000, 80000), 20, replace=False)] = 1.0
    lg[10:110] = -0.0
    lg[1024 + 3:1024 + 103] = 0.0
    for t in (1.0, 0.8):
        dev, ref = both(lg, S(top_p=1.0, top_k=50, temperature=t, repetition_penalty=1.0), seed=seed)
        assert dev == ref


@pytest.mark.parametrize("v", [1, 5, 1000, 1024, 1025, 3 * 1024 + 1])
@pytest.mark.parametrize("seed", [0, 1])
def test_ragged_vocabularies(gpu, v, seed):
    lg = normal(v, seed)
    h = [int(x) for x in np.random.default_rng(seed).integers(0, v, 30)]
    for kw in (dict(), dict(top_k=3, top_p=0.5), dict(top_k=2000, top_p=1.0)):
        dev, ref = both(lg, S(**kw), h, 30, seed=seed)
        assert dev == ref


def test_greedy_ties_and_penalty(gpu):
    lg = normal(V3B, 7)
    top = float(lg.max()) + 1.0
    lg[[70000, 2000, 5000]] = top
    s = S(temperature=0.0, top_k=1, top_p=1.0)
    assert both(lg, s)[0] == 2000  # smallest id among equal maxima
    dev, ref = both(lg, s, history=[2000, 5000, 2000], step=3)
    assert dev == ref == 70000  # the penalty demotes the other two
    dev, ref = both(lg, S(temperature=0.0, top_k=50, repetition_penalty=1.0))
    assert dev == ref == 2000


def test_history_window_and_length(gpu):
    lg = normal(V3B, 8)
    best = np.argsort(-lg, kind="stable")[:5].tolist()
    h = best * 30  # 150 ids: only the last penalty_window count
    for w in (1, 7, 50, 100):
        for step in (0, 3, 150, 400):
            dev, ref = both(lg, S(temperature=0.0, penalty_window=w, repetition_penalty=1.7), h, step)
            assert dev == ref
    dev, ref = both(lg, S(penalty_window=100), h[:10], 500, seed=3)
    assert dev == ref


@pytest.mark.parametrize("phase", [O.PHASE_ABC, O.PHASE_SEMANTIC])
@pytest.mark.parametrize("step", [0, 9, 10])
def test_phase_masks(gpu, phase, step):
    lg = normal(V_PHASE, 11)
    end = ABC_END if phase == O.PHASE_ABC else MUSIC_END
    lg[end] = 40.0  # the end token wins once min_tokens allows it
    h = [EOD + 2, CODEC_OFFSET + 5, 17, CODEC_OFFSET + 5]  # masked and unmasked ids
    for kw in (dict(temperature=0.0), dict(top_k=80), dict(top_k=2000, top_p=0.9)):
        dev, ref = both(lg, S(min_tokens=10, **kw), h, step, phase=phase, seed=step)
        assert dev == ref
        assert (dev == end) == (step >= 10)


@pytest.mark.parametrize("top_k", [50, 1000])
def test_error_rules(gpu, top_k):
    s = S(top_k=top_k)
    for bad in (np.nan, np.inf):
        lg = normal(V3B, 12)
        lg[777] = bad
        with pytest.raises(y2.Yue2Error) as e:
            y2.choose(lg, s, draws=draws(0, V3B))
        assert e.value.code == -4
        with pytest.raises(RuntimeError):
            O.choose(lg, s, [], 0, O.PHASE_NONE, False, O.Generator(0))
        with pytest.raises(y2.Yue2Error) as e:
            y2.choose(lg, S(temperature=0.0, top_k=top_k), draws=None)
        assert e.value.code == -4
    lg = np.full(V3B, -np.inf, np.float32)
    for t in (0.0, 0.9):
        with pytest.raises(y2.Yue2Error) as e:
            y2.choose(lg, S(temperature=t, top_k=top_k), draws=draws(0, V3B))
        assert e.value.code == -5
    # -inf at one entry is masked, not invalid
    lg = normal(V3B, 13)
    lg[5] = -np.inf
    dev, ref = both(lg, s, seed=2)
    assert dev == ref


@pytest.mark.parametrize("top_k,ties,seed", [(5000, 0, 0), (50, 3000, 1), (1000, 3000, 2), (50, V3B, 3),
                                              (V3B, 0, 4)])
def test_many_survivors(gpu, top_k, ties, seed):
    """More survivors than the LDS survivor arrays hold (2048): top_k 5000,
    3000 entries tied at the top-k threshold, the whole vocabulary tied, and
    top_k = vocabulary (src/sampling.rs:162-174 keeps every tie); with and
    without top-p."""
    lg = normal(V3B, seed)
    if ties:
        rng = np.random.default_rng(seed)
        at = rng.choice(V3B, ties, replace=False)
        lg[at] = np.max(lg) + 1.0  # the best entries, all equal
    for top_p in (0.93, 1.0):
        dev, ref = both(lg, S(top_k=top_k, top_p=top_p, temperature=1.3), seed=seed)
        assert dev == ref
