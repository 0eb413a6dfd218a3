"""Drop-in twins of the reference's Metal bridge against the oracle:
yue2_hip_ar_stack (hidden before the final norm and the shadow K/V rows,
src/metal.m:718-874 / src/model.rs:533-568) and yue2_hip_vector with F32 and
F16 weights (rounded to BF16 as Linear does, src/tensor.rs:436-438)."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
from yue2_rs_amd.api import _GpuLayer
import yue2_rs_amd as y2

from helpers import bits, fresh_mapping, rb

pytestmark = pytest.mark.gpu

PROJ = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


def _layers(ck, cache, mapping):
    layers = (_GpuLayer * ck.config.num_hidden_layers)()
    keep = []
    for i, w in enumerate(ck.layers):
        L = layers[i]
        for j, name in enumerate(PROJ):
            arr = getattr(w, name)
            L.weights[j].raw = arr.ctypes.data
            L.weights[j].mapping = mapping
            L.weights[j].rows, L.weights[j].cols = arr.shape
            L.weights[j].dtype = 0
            L.weights[j].rounded = 1
        norms = [rb(w.input_layernorm), rb(w.q_norm), rb(w.k_norm), rb(w.post_attention_layernorm)]
        keep += norms
        for j, n in enumerate(norms):
            L.norms[j] = n.ctypes.data
        k, v = np.ascontiguousarray(cache.keys(i)), np.ascontiguousarray(cache.values(i))
        keep += [k, v]
        L.key, L.value = k.ctypes.data, v.ctypes.data
    return layers, keep


@pytest.mark.parametrize("prefix", [255, 300])
def test_ar_stack_matches_oracle(gpu, oracle_threads, prefix):
    c = synthetic.REDUCED
    ck = synthetic.checkpoint(c, seed=0)
    om = O.Model(ck)
    ids = synthetic.prompt(prefix + 2, c.vocab_size, seed=4)
    ocache, _ = om.prefill(ids[:prefix], prefix + 4)
    H, D, kv = c.hidden_size, c.head_dim, c.num_key_value_heads
    cache_id = 4242 + prefix
    mapping = fresh_mapping()
    y2.lib().yue2_hip_clear_weights()
    for step in range(2):
        pos = prefix + step
        layers, keep = _layers(ck, ocache, mapping)
        tok = int(ids[pos])
        x = (ck.embed_tokens[tok].astype(np.uint32) << 16).view(np.float32).copy()
        cs, sn = np.empty(D // 2, np.float32), np.empty(D // 2, np.float32)
        O.lib().y2o_rotary_table(pos, 1, D, c.rope_theta, cs.ctypes.data, sn.ctypes.data)
        out = np.empty(H, np.float32)
        shadow = np.empty(c.num_hidden_layers * 2 * kv * D, np.float32)
        ok = y2.lib().yue2_hip_ar_stack(x.ctypes.data, out.ctypes.data, shadow.ctypes.data, layers,
                                        c.num_hidden_layers, H, c.num_attention_heads, kv, D,
                                        c.intermediate_size, pos, prefix + 4, cache_id, c.rms_norm_eps,
                                        cs.ctypes.data, sn.ctypes.data)
        assert ok == 1, y2.lib().yue2_hip_last_error()
        want = np.empty(H, np.float32)
        tid = np.array([tok], np.int32)
        assert O.lib().y2o_hidden_prenorm(om.ref, ocache.ptr, tid.ctypes.data, 1, want.ctypes.data) == 0
        assert np.array_equal(bits(out), bits(want)), f"hidden differs at position {pos}"
        for l in range(c.num_hidden_layers):
            sk = shadow[l * 2 * kv * D:(l * 2 + 1) * kv * D]
            sv = shadow[(l * 2 + 1) * kv * D:(l * 2 + 2) * kv * D]
            assert np.array_equal(bits(sk), bits(ocache.keys(l)[pos]))
            assert np.array_equal(bits(sv), bits(ocache.values(l)[pos]))
    y2.lib().yue2_hip_release_cache(cache_id)


@pytest.mark.parametrize("dtype", [1, 2])
def test_vector_rounds_f32_and_f16_weights(gpu, dtype):
    n, k = 512, 1024
    rng = np.random.default_rng(dtype)
    w = rng.normal(0, 0.05, (n, k)).astype(np.float32 if dtype == 1 else np.float16)
    x = rb(rng.normal(0, 1, k).astype(np.float32))
    got = np.empty(n, np.float32)
    ok = y2.lib().yue2_hip_vector(x.ctypes.data, w.ctypes.data, fresh_mapping(), dtype, 1, 1, got.ctypes.data, n, k)
    assert ok == 1, y2.lib().yue2_hip_last_error()
    wb = (rb(w.astype(np.float32)).view(np.uint32) >> 16).astype(np.uint16)
    want = np.empty(n, np.float32)
    O.lib().y2o_gemv_raw(wb.ctypes.data, n, k, x.ctypes.data, want.ctypes.data)
    assert np.array_equal(bits(got), bits(want))
    # unrounded F32 weights are not handled on the device: the caller falls back
    assert y2.lib().yue2_hip_vector(x.ctypes.data, w.ctypes.data, fresh_mapping(), dtype, 0, 1, got.ctypes.data, n, k) == 0


def test_lifetime_calls_and_names(gpu):
    L = y2.lib()
    assert L.yue2_hip_available() == 1
    assert L.yue2_hip_vector_default() == 1
    assert len(L.yue2_hip_name()) > 0
    assert L.yue2_physical_memory() > 0
    L.yue2_hip_release_cache(123456)
    L.yue2_hip_clear_weights()
    L.yue2_hip_release_model()


# ---- the prefill / NAR bridge: yue2_metal_gemm, linear, attention ----------

def _p(a):
    return a.ctypes.data


def _gemm_bound(a, bt):
    """|error| bound of an f32 dot product of length k: gamma_k sum |a||b|."""
    k = a.shape[1]
    g = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    return g * (np.abs(a).astype(np.float64) @ np.abs(bt).astype(np.float64).T) + 1e-30


@pytest.mark.parametrize("transpose_b,beta", [(0, 0.0), (1, 0.0), (1, 0.5), (0, -1.25)])
def test_gemm_twin(gpu, transpose_b, beta):
    """src/tensor.rs:207-219 (MPS, src/metal.m:164-182): row-major operands
    with padded row strides, C = A op(B) + beta C; within the f32 dot bound of
    a float64 product, and exact on small integers (every partial sum exact,
    so any order gives the same bits)."""
    rng = np.random.default_rng(7 + transpose_b)
    m, n, k = 70, 300, 513
    lda, ldb, ldc = k + 3, (k if transpose_b else n) + 5, n + 2
    for ints in (False, True):
        draw = (lambda *s: rng.integers(-4, 5, size=s).astype(np.float32)) if ints else \
            (lambda *s: rng.standard_normal(s).astype(np.float32))
        A = np.zeros((m, lda), np.float32)
        A[:, :k] = draw(m, k)
        B = np.zeros(((n if transpose_b else k), ldb), np.float32)
        B[:, :(k if transpose_b else n)] = draw(n, k) if transpose_b else draw(k, n)
        Cin = np.zeros((m, ldc), np.float32)
        Cin[:, :n] = draw(m, n)
        c = Cin.copy()
        ok = y2.lib().yue2_hip_gemm(_p(A), _p(B), _p(c), m, n, k, transpose_b, lda, ldb, ldc, beta)
        assert ok == 1
        Bt = B[:, :k] if transpose_b else B[:, :n].T  # [n, k]
        want = A[:, :k].astype(np.float64) @ Bt.astype(np.float64).T + np.float64(beta) * Cin[:, :n]
        if ints:
            assert np.array_equal(c[:, :n], want.astype(np.float32))
        else:
            bound = _gemm_bound(A[:, :k], Bt) + abs(beta) * np.abs(Cin[:, :n]) * 2.0 ** -23
            assert np.all(np.abs(c[:, :n] - want) <= 2 * bound)
        assert np.array_equal(c[:, n:], Cin[:, n:]), "padding columns written"


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_linear_twin(gpu, dtype):
    """src/tensor.rs:135-145 (src/metal.m:216-237): c = a W^T for BF16, F32
    and F16 host weights; rounded F32/F16 weights are rounded to BF16 first
    (convert_weight, src/attention.metal:161-176).  Checked against float64
    on the converted weights within the f32 dot bound, the unrounded F32
    weights against their own values, and the weight cache keyed by mapping."""
    rng = np.random.default_rng(30 + dtype)
    m, n, k = 48, 400, 768
    a = rng.standard_normal((m, k)).astype(np.float32)
    w32 = (0.05 * rng.standard_normal((n, k))).astype(np.float32)
    if dtype == 0:
        raw = (rb(w32).view(np.uint32) >> 16).astype(np.uint16)
        conv = rb(w32)
    elif dtype == 1:
        raw = w32
        conv = w32
    else:
        raw = w32.astype(np.float16)
        conv = raw.astype(np.float32)
    mapping = fresh_mapping()
    for rounded in (1, 0):
        want_w = rb(conv) if (rounded and dtype != 0) else conv
        c = np.empty((m, n), np.float32)
        assert y2.lib().yue2_hip_linear(_p(a), _p(raw), mapping, dtype, rounded, _p(c), m, n, k) == 1
        want = a.astype(np.float64) @ want_w.astype(np.float64).T
        assert np.all(np.abs(c - want) <= 2 * _gemm_bound(a, want_w))
        if rounded and dtype != 0:
            # the rounding is applied: the unrounded weights' product differs
            assert not np.all(np.abs(c - a.astype(np.float64) @ conv.astype(np.float64).T) <= _gemm_bound(a, conv))


def _attention_f64(q, k, v, rows, keys, heads, kv, dim, causal, scale):
    out = np.empty((rows, heads * dim), np.float64)
    G = heads // kv
    for r in range(rows):
        vis = keys if causal < 0 else min(keys, causal + r + 1)
        for h in range(heads):
            g = h // G
            s = (k[:vis, g * dim:(g + 1) * dim].astype(np.float64) @ q[r, h * dim:(h + 1) * dim].astype(np.float64))
            e = np.exp(s * scale - (s * scale).max())
            out[r, h * dim:(h + 1) * dim] = (e @ v[:vis, g * dim:(g + 1) * dim].astype(np.float64)) / e.sum()
    return out


@pytest.mark.parametrize("dim,causal,rows,keys", [(128, 40, 90, 130), (64, 0, 200, 200), (128, -1, 33, 300),
                                                   (64, -1, 128, 128)])
def test_attention_twin(gpu, dim, causal, rows, keys):
    """src/tensor.rs:194-206 (src/metal.m:330-361): multi-row attention, row r
    over keys [0, causal + r] or all keys, BF16-rounded output; within the
    reference's own tolerance for its GPU attention against float64
    (5e-5 + 0.008 |x|, src/tensor.rs:73)."""
    rng = np.random.default_rng(dim + rows)
    heads, kv = 6, 2
    q = rb(rng.standard_normal((rows, heads * dim)).astype(np.float32))
    k = rb(rng.standard_normal((keys, kv * dim)).astype(np.float32))
    v = rb(rng.standard_normal((keys, kv * dim)).astype(np.float32))
    scale = np.float32(1.0) / np.sqrt(np.float32(dim))
    out = np.empty((rows, heads * dim), np.float32)
    assert y2.lib().yue2_hip_attention(_p(q), _p(k), _p(v), _p(out), rows, keys, heads, kv, dim, causal,
                                       float(scale)) == 1
    assert np.array_equal(out, rb(out)), "output not BF16-rounded"
    want = _attention_f64(q, k, v, rows, keys, heads, kv, dim, causal, float(scale))
    assert np.all(np.abs(out - want) <= 5e-5 + 0.008 * np.abs(want))
    # inputs that are not BF16-exact fall back to the CPU
    q2 = q.copy()
    q2[0, 0] += np.float32(1e-3)
    assert y2.lib().yue2_hip_attention(_p(q2), _p(k), _p(v), _p(out), rows, keys, heads, kv, dim, causal,
                                       float(scale)) == 0
