"""The phase-restricted LM head and the end-token stop on the device.

A tiny model with the protocol's vocabulary (184704 ids, so ABC_END 151848,
MUSIC_END 151852 and the codec range [151853, 184621) exist) runs
project_phase (src/model.rs:478-507) and the generate loop's stop at the
phase's end token (src/sampling.rs:267-271).  Every embedding carries a
large constant in dimension 0 and the two stop rows of the LM head weigh
that dimension, while the phase ranges ignore it: once min_tokens allows
the end token, it wins.  Results are compared with the oracle bit for bit
(logits) and id for id (tokens, count, truncated)."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
from yue2_rs_amd.api import Config
import yue2_rs_amd as y2

from helpers import bits

pytestmark = pytest.mark.gpu

EOD, ABC_END, MUSIC_END, CODEC_OFFSET = 151643, 151848, 151852, 151853
TINY = Config(hidden_size=128, num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1, head_dim=64,
              intermediate_size=256, vocab_size=184704, max_position_embeddings=512, rms_norm_eps=1e-6,
              rope_theta=1e6)
ONE, FOUR = 0x3F80, 0x4080  # BF16 1.0 and 4.0


@pytest.fixture(scope="module")
def tiny(gpu, oracle_threads):
    ck = synthetic.checkpoint(TINY, seed=11)
    ck.embed_tokens[:, 0] = FOUR
    ck.lm_head[:EOD, 0] = 0
    ck.lm_head[CODEC_OFFSET:, 0] = 0
    ck.lm_head[ABC_END, 0] = ONE
    ck.lm_head[MUSIC_END, 0] = ONE
    gm = y2.Model.open(ck)
    yield ck, gm, O.Model(ck)
    gm.close()


@pytest.mark.parametrize("phase", [y2.PHASE_ABC, y2.PHASE_SEMANTIC])
def test_forward_phase_matches_oracle(tiny, phase):
    ck, gm, om = tiny
    ids = synthetic.prompt(24, TINY.vocab_size, seed=phase)
    gc, gl = gm.prefill_phase(ids, 32, phase)
    oc, ol = om.prefill(ids, 32, phase)
    assert np.array_equal(bits(gl), bits(ol))
    lo, hi, stop = (0, EOD, ABC_END) if phase == y2.PHASE_ABC else (CODEC_OFFSET, TINY.vocab_size - 83, MUSIC_END)
    keep = np.zeros(TINY.vocab_size, bool)
    keep[lo:hi] = True
    keep[stop] = True
    assert np.all(gl[~keep] == -np.inf) and np.all(np.isfinite(gl[keep]))
    for t in (5, CODEC_OFFSET + 3, 100):
        assert np.array_equal(bits(gm.forward_phase([t], gc, phase)), bits(om.forward_phase([t], oc, phase)))


@pytest.mark.parametrize("phase", [y2.PHASE_ABC, y2.PHASE_SEMANTIC])
@pytest.mark.parametrize("temperature,scale", [(0.0, 1.0), (0.9, 1.0), (0.9, 1.5)])
def test_generate_stops_at_end_token(tiny, phase, temperature, scale):
    ck, gm, om = tiny
    s = y2.Sampling(temperature=temperature, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=5, max_tokens=16)
    pos = synthetic.prompt(20, TINY.vocab_size, seed=3)
    neg = synthetic.prompt(12, TINY.vocab_size, seed=4) if scale != 1.0 else None
    got = y2.generate(gm, pos, s, seed=77, phase=phase, negative=neg, scale=scale)
    want, trunc = O.generate(om, pos, s, 77, phase=phase, negative=neg, scale=scale)
    assert not trunc and len(want) == 5, "the construction must end at min_tokens"
    assert got.tokens == want
    assert got.truncated == trunc


def test_decoder_run_ends_without_the_end_tokens_forward(tiny):
    """decoder_run returns the end id as its last token, grows the cache by
    one position less, and the cache then continues exactly as the
    reference's (whose loop never ran the end token's forward)."""
    ck, gm, om = tiny
    phase = y2.PHASE_SEMANTIC
    s = y2.Sampling(temperature=0.0, top_p=1.0, top_k=1, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=4, max_tokens=64)
    ids = synthetic.prompt(16, TINY.vocab_size, seed=9)
    gc, gl = gm.prefill_phase(ids, 40, phase)
    dec = y2.Decoder(gm, gc, sampling=s, phase=phase)
    toks, _ = dec.run(10, first_logits=gl)
    assert len(toks) == 5 and toks[-1] == MUSIC_END
    assert gc.length == 16 + 4
    assert len(dec.run(3)[0]) == 0
    dec.close()
    want, trunc = O.generate(om, ids, s, 0, phase=phase)
    assert list(toks[:-1]) == want and not trunc
    oc, _ = om.prefill(ids, 40, phase)
    for t in want:
        om.forward_phase([t], oc, phase)
    assert np.array_equal(bits(gm.forward_phase([want[0]], gc, phase)), bits(om.forward_phase([want[0]], oc, phase)))
