"""Models opened from checkpoint directories (yue2_hip_model_open_dir:
config.json + safetensors, src/model.rs:418-451, src/checkpoint.rs:310-386)
against the same weights opened from memory and against the oracle, bit for
bit; and the real YuE2 layer shape (src/model.rs:35-48: hidden 2048, 16/8
heads, head_dim 128, SwiGLU 6144, vocabulary 184704, theta 1e6; two layers)
through the persistent step kernel, with the ABC and semantic LM heads
(project_phase, src/model.rs:478-507) and the sampler inside the step
kernel."""
import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
from yue2_rs_amd.api import Checkpoint, Config, LayerWeights
import yue2_rs_amd as y2

from ckpt_files import write_checkpoint
from helpers import bits, rb

pytestmark = pytest.mark.gpu

YUE2 = Config(hidden_size=2048, num_hidden_layers=2, num_attention_heads=16, num_key_value_heads=8, head_dim=128,
              intermediate_size=6144, vocab_size=184704, max_position_embeddings=24576, rms_norm_eps=1e-6,
              rope_theta=1e6)


def _f16_rounded(ck):
    """The BF16 weights the loader makes of F16 copies of ck's matrices."""
    def r(a):
        f = (a.astype(np.uint32) << 16).view(np.float32).astype(np.float16).astype(np.float32)
        return (rb(f).view(np.uint32) >> 16).astype(np.uint16)
    layers = [LayerWeights(**{k: (r(v) if v.dtype == np.uint16 else v) for k, v in vars(w).items()})
              for w in ck.layers]
    return Checkpoint(ck.config, r(ck.embed_tokens), r(ck.lm_head), ck.final_norm, layers)


@pytest.mark.parametrize("dtype,shards", [("BF16", 4), ("F32", 1), ("F16", 2)])
def test_open_dir_matches_memory_and_oracle(gpu, oracle_threads, tmp_path, dtype, shards):
    ck = synthetic.checkpoint(synthetic.REDUCED, seed=4)
    d = write_checkpoint(tmp_path / "m", ck, dtype=dtype, shards=shards)
    want_ck = _f16_rounded(ck) if dtype == "F16" else ck
    gd = y2.Model.open_dir(d)
    gm = y2.Model.open(want_ck)
    om = O.Model(want_ck)
    ids = synthetic.prompt(40, ck.config.vocab_size, seed=2)
    c1, l1 = gd.prefill_phase(ids, 48)
    c2, l2 = gm.prefill_phase(ids, 48)
    _, l3 = om.prefill(ids, 48)
    assert np.array_equal(bits(l1), bits(l2)) and np.array_equal(bits(l1), bits(l3))
    gd.close()
    gm.close()


@pytest.fixture(scope="module")
def yue2(gpu, oracle_threads, tmp_path_factory):
    ck = synthetic.checkpoint(YUE2, seed=6, threads=16)
    d = write_checkpoint(tmp_path_factory.mktemp("yue2"), ck, shards=3)
    gm = y2.Model.open_dir(d)
    assert gm.set_step_kernel(True), "the YuE2 shape has a step kernel"
    yield ck, gm, O.Model(ck)
    gm.close()


@pytest.mark.parametrize("phase", [y2.PHASE_NONE, y2.PHASE_ABC, y2.PHASE_SEMANTIC])
def test_yue2_shape_forward_phase(yue2, phase):
    ck, gm, om = yue2
    ids = synthetic.prompt(20, YUE2.vocab_size, seed=3 + phase)
    gc, gl = gm.prefill_phase(ids, 32, phase)
    oc, ol = om.prefill(ids, 32, phase)
    assert np.array_equal(bits(gl), bits(ol))
    for t in (7, 151900, 184000):
        assert np.array_equal(bits(gm.forward_phase([t], gc, phase)), bits(om.forward_phase([t], oc, phase)))


@pytest.mark.parametrize("phase,temperature,scale", [(y2.PHASE_SEMANTIC, 0.9, 1.5), (y2.PHASE_ABC, 0.9, 1.0),
                                                     (y2.PHASE_SEMANTIC, 0.0, 1.5), (y2.PHASE_NONE, 0.9, 1.5)])
def test_yue2_shape_generate(yue2, phase, temperature, scale):
    """sampling::generate with the sampler inside the step kernel over the
    phase's LM-head rows (the semantic head: 32768 codec rows + MUSIC_END)."""
    ck, gm, om = yue2
    s = y2.Sampling(temperature=temperature, top_p=0.93, top_k=50, repetition_penalty=1.2, penalty_window=50,
                    min_tokens=0, max_tokens=12)
    pos = synthetic.prompt(24, YUE2.vocab_size, seed=8)
    neg = synthetic.prompt(16, YUE2.vocab_size, seed=9) if scale != 1.0 else None
    got = y2.generate(gm, pos, s, seed=5, phase=phase, negative=neg, scale=scale)
    want, trunc = O.generate(om, pos, s, 5, phase=phase, negative=neg, scale=scale)
    assert got.tokens == want and got.truncated == trunc
