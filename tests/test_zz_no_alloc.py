"""yue2_hip_choose_noalloc (choose() in a file-scope device scratch array,
no allocation) against yue2_hip_choose on the same inputs: the same id, on
calls in a row that reuse the scratch with shrinking inputs, and its size
limit."""
import numpy as np
import pytest

from oracle import oracle as O
import yue2_rs_amd as y2

pytestmark = pytest.mark.gpu


def _draws(seed, v):
    return np.random.RandomState(seed).randint(0, 2 ** 32, size=2 * v, dtype=np.uint64).astype(np.uint32)


def _case(v, seed, **kw):
    rng = np.random.default_rng(seed)
    lg = (rng.standard_normal(v) * 3.0).astype(np.float32)
    base = dict(temperature=0.9, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50, min_tokens=0,
                max_tokens=100)
    base.update(kw)
    s = y2.Sampling(**base)
    hist = rng.choice(np.argsort(-lg)[:200], 60).tolist()
    return lg, s, hist, _draws(seed, v)


@pytest.mark.parametrize("order", [(184704, 84000, 32768, 1000), (84000, 5000)])
def test_noalloc_matches_choose_on_calls_in_a_row(gpu, order):
    for i, v in enumerate(order):
        for kw in ({}, {"top_k": 5000, "top_p": 1.0}, {"temperature": 0.0}):
            lg, s, hist, d = _case(v, 10 * i + v % 7, **kw)
            if v <= 5000:
                lg[::2] = np.max(lg)  # ties at the top: 2500 survivors for 5000 entries
            want = y2.choose(lg, s, hist, 3, draws=d)
            got = y2.choose(lg, s, hist, 3, draws=d, noalloc=True)
            assert got == want, f"vocab {v}, settings {kw}"
            assert want == O.choose(lg, s, hist, 3, O.PHASE_NONE, False, O.Generator(10 * i + v % 7))


def test_noalloc_rejects_vocabularies_beyond_its_scratch(gpu):
    v = 262145
    lg, s, hist, d = _case(v, 1)
    with pytest.raises(y2.Yue2Error) as e:
        y2.choose(lg, s, hist, 0, draws=d, noalloc=True)
    assert e.value.code == -13
    # the limit itself is accepted
    lg, s, hist, d = _case(262144, 2)
    assert y2.choose(lg, s, hist, 0, draws=d, noalloc=True) == y2.choose(lg, s, hist, 0, draws=d)
