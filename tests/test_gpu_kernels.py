"""GEMV and decode attention through the reference-twin entry points
(yue2_hip_vector, yue2_hip_cached_attention) against the oracle, bit-exact,
at the microbenchmark shapes; plus the reference's own attention
known-answer test (src/tensor.rs:9-83) with its tolerance."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

from helpers import bits, fresh_mapping, rb

pytestmark = pytest.mark.gpu

GEMV_SHAPES = [(5120, 3072), (3072, 3072), (16384, 3072), (3072, 8192), (84000, 3072), (1024, 1024),
               (2816, 1024), (1024, 2816), (8, 8)]


def _bf16_exact(x):
    return rb(np.asarray(x, dtype=np.float32))


@pytest.mark.parametrize("shape", GEMV_SHAPES)
def test_vector_matches_oracle(gpu, oracle_threads, shape):
    n, k = shape
    w = synthetic.bf16_normal((n, k), seed=7, tensor=n * 131 + k)
    x = _bf16_exact(np.random.default_rng(n + k).normal(0, 1, k))
    got = np.empty(n, np.float32)
    ok = y2.lib().yue2_hip_vector(x.ctypes.data, w.ctypes.data, fresh_mapping(), 0, 1, 1, got.ctypes.data, n, k)
    assert ok == 1, y2.lib().yue2_hip_last_error()
    want = np.empty(n, np.float32)
    O.lib().y2o_gemv_raw(w.ctypes.data, n, k, x.ctypes.data, want.ctypes.data)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_vector_one_hot_reproduces_columns(gpu):
    n, k = 256, 1024
    w = synthetic.bf16_normal((n, k), seed=3, tensor=99)
    wf = (w.astype(np.uint32) << 16).view(np.float32)
    mapping = fresh_mapping()
    for col in (0, 7, 8, 511, 512, 1023):
        x = np.zeros(k, np.float32)
        x[col] = 1.0
        got = np.empty(n, np.float32)
        assert y2.lib().yue2_hip_vector(x.ctypes.data, w.ctypes.data, mapping, 0, 1, 1, got.ctypes.data, n, k) == 1
        assert np.array_equal(got, wf[:, col])


def _attention_f64(q, key, value, heads, kv, dim):
    out = np.empty(heads * dim)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dim)))
    for h in range(heads):
        g = h // (heads // kv)
        qh = q[h * dim:(h + 1) * dim].astype(np.float64)
        kh = key[:, g * dim:(g + 1) * dim].astype(np.float64)
        vh = value[:, g * dim:(g + 1) * dim].astype(np.float64)
        s = kh @ qh * scale
        e = np.exp(s - s.max())
        out[h * dim:(h + 1) * dim] = (e @ vh) / e.sum()
    return out


def _oracle_attention(q, key, value, heads, kv, dim):
    out = np.empty(heads * dim, np.float32)
    O.lib().y2o_attention_row(q.ctypes.data, key.ctypes.data, value.ctypes.data, key.shape[0], heads, kv,
                              dim, out.ctypes.data)
    return out


def _device_attention(q, key, value, heads, kv, dim, cache, layer=0):
    out = np.empty(heads * dim, np.float32)
    ok = y2.lib().yue2_hip_cached_attention(q.ctypes.data, key.ctypes.data, value.ctypes.data,
                                            out.ctypes.data, key.shape[0], heads, kv, dim, cache, layer)
    assert ok == 1, y2.lib().yue2_hip_last_error()
    return out


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("keys", [4096, 4097, 7169, 24576])
def test_reference_attention_known_answer(gpu, oracle_threads, dim, keys):
    """src/tensor.rs:9-83: integer-hash K/V/q, one appended row, f64 softmax
    reference, tolerance 5e-5 + 0.008|expected|; also bit-exact vs the oracle."""
    heads, kv = 4, 2
    i = np.arange(keys * kv * dim, dtype=np.int64)
    key = rb(((i * 17 % 101) - 50).astype(np.float32) * np.float32(0.06)).reshape(keys, kv * dim)
    value = rb(((i * 31 % 137) - 68).astype(np.float32) * np.float32(0.007)).reshape(keys, kv * dim)
    j = np.arange(heads * dim, dtype=np.int64)
    q = rb(((j * 23 % 97) - 48).astype(np.float32) * np.float32(0.04))
    cache = 9000 + keys + dim
    for append in range(2 if keys < 24576 else 1):
        if append:
            r = np.arange(kv * dim).astype(np.float32)
            key = np.vstack([key, rb(r * np.float32(0.002) - np.float32(0.3))[None]])
            value = np.vstack([value, rb(np.float32(0.4) - r * np.float32(0.001))[None]])
        key = np.ascontiguousarray(key, np.float32)
        value = np.ascontiguousarray(value, np.float32)
        got = _device_attention(q, key, value, heads, kv, dim, cache)
        expected = rb(_attention_f64(q, key, value, heads, kv, dim).astype(np.float32))
        assert np.all(np.abs(got - expected) <= 5e-5 + np.abs(expected) * 0.008)
        assert np.array_equal(bits(got), bits(_oracle_attention(q, key, value, heads, kv, dim)))
    y2.lib().yue2_hip_release_cache(cache)


@pytest.mark.parametrize("keys", [1, 63, 64, 65, 1024, 4096, 16384, 24576])
def test_gqa_attention_bit_exact(gpu, oracle_threads, keys):
    """Decode attention microbenchmark shape (Hq 24, Hkv 8, d 128) with
    N(0,1) BF16 inputs: bit-exact against the oracle."""
    heads, kv, dim = 24, 8, 128
    rng = np.random.default_rng(keys)
    q = _bf16_exact(rng.normal(0, 1, heads * dim))
    key = _bf16_exact(rng.normal(0, 1, (keys, kv * dim)))
    value = _bf16_exact(rng.normal(0, 1, (keys, kv * dim)))
    got = _device_attention(q, key, value, heads, kv, dim, cache=77000 + keys)
    want = _oracle_attention(q, key, value, heads, kv, dim)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    y2.lib().yue2_hip_release_cache(77000 + keys)


def test_single_key_returns_value_row(gpu):
    heads, kv, dim = 8, 2, 128
    rng = np.random.default_rng(5)
    q = _bf16_exact(rng.normal(0, 1, heads * dim))
    key = _bf16_exact(rng.normal(0, 1, (1, kv * dim)))
    value = _bf16_exact(rng.normal(0, 1, (1, kv * dim)))
    got = _device_attention(q, key, value, heads, kv, dim, cache=5)
    for h in range(heads):
        g = h // (heads // kv)
        assert np.array_equal(got[h * dim:(h + 1) * dim], value[0, g * dim:(g + 1) * dim])
    y2.lib().yue2_hip_release_cache(5)
