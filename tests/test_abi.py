"""CPU: the C-ABI library (no GPU compute): it loads, exports every function
include/yue2_hip.h declares, its host-only logic (Config::read and
Sampling::validate) matches the reference's rules, the synthetic weight
generator is deterministic, and the product refuses to run without a
device or without its native library instead of falling back."""
import math
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import yue2_rs_amd as y2
from yue2_rs_amd import api, synthetic

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "yue2_hip.h"


def declared() -> set:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(yue2_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    names = declared()
    assert len(names) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", str(api.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert names <= exported, sorted(names - exported)


def test_python_binding_covers_the_header():
    api.lib()
    import inspect
    src = inspect.getsource(api.lib)
    bound = set(re.findall(r'"(yue2_\w+)"', src))
    assert declared() == bound, (sorted(declared() - bound), sorted(bound - declared()))


def test_config_validate_follows_config_read():
    y2.Config().validate()
    synthetic.CLASS_3B.validate()
    bad = [dict(hidden_size=0), dict(num_hidden_layers=0), dict(num_key_value_heads=3),
           dict(head_dim=127), dict(rope_theta=0.0), dict(rope_theta=math.inf), dict(rms_norm_eps=0.0),
           dict(rms_norm_eps=math.nan), dict(vocab_size=0), dict(intermediate_size=0)]
    for kw in bad:
        with pytest.raises(y2.Yue2Error) as e:
            y2.Config(**kw).validate()
        assert e.value.code == -11, kw


def test_sampling_validate_follows_protocol():
    y2.Sampling().validate()
    y2.Sampling(temperature=0.0).validate()
    y2.Sampling(temperature=5.0, top_p=1.0, penalty_window=100).validate()
    bad = [dict(temperature=-0.1), dict(temperature=5.01), dict(temperature=math.nan), dict(top_p=0.0),
           dict(top_p=1.01), dict(top_p=math.inf), dict(top_k=0), dict(repetition_penalty=0.0),
           dict(repetition_penalty=math.inf), dict(penalty_window=0), dict(penalty_window=101),
           dict(min_tokens=10, max_tokens=5), dict(min_tokens=0, max_tokens=0)]
    for kw in bad:
        with pytest.raises(y2.Yue2Error) as e:
            y2.Sampling(**kw).validate()
        assert e.value.code == -6, kw


def test_synthetic_weights_are_deterministic_and_normal():
    a = synthetic.bf16_normal((512, 1024), seed=3, tensor=17, threads=1)
    b = synthetic.bf16_normal((512, 1024), seed=3, tensor=17, threads=8)
    c = synthetic.bf16_normal((512, 1024), seed=3, tensor=18, threads=8)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)
    f = (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert abs(f.mean()) < 2e-4
    assert abs(f.std() - 0.02) < 2e-4
    # BF16 rounding of 0.02 * N(0, 1): about 68% within one standard deviation
    assert abs(np.mean(np.abs(f) < 0.02) - 0.6827) < 0.01


def test_prompt_ids_follow_mt19937():
    mt = synthetic.MT19937(0)
    want = [mt.next_u32() % 1000 for _ in range(50)]
    assert list(synthetic.prompt(50, 1000, seed=0)) == want


def test_model_open_refuses_without_device():
    if y2.available():
        pytest.skip("a device is present")
    ck = synthetic.checkpoint(y2.Config(hidden_size=64, num_hidden_layers=1, num_attention_heads=2,
                                        num_key_value_heads=1, head_dim=64, intermediate_size=128,
                                        vocab_size=256), seed=0)
    with pytest.raises(y2.Yue2Error) as e:
        y2.Model.open(ck)
    assert e.value.code == -12


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(api, "_lib", None)
    monkeypatch.setattr(api, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(FileNotFoundError):
        api.lib()


def test_model_close_frees_only_the_model():
    """Model.close() frees the model once and nothing else: the library
    detaches the model's caches and decoders itself, so each may be closed
    before or after it (the reference's Cache may outlive its Model,
    src/model.rs:286-290).  Host logic only: a stand-in library."""
    from yue2_rs_amd import api

    freed = []

    class FakeLib:
        @staticmethod
        def yue2_hip_model_free(h):
            freed.append(h)

    m = api.Model.__new__(api.Model)
    m._h = 7
    real_lib = api.lib
    api.lib = lambda: FakeLib
    try:
        m.close()
        m.close()  # a second close frees nothing
    finally:
        api.lib = real_lib
    assert freed == [7]
