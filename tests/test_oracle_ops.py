"""CPU: the oracle's token-step operators against what the mathematics fixes
(no GPU).  Each check is chosen so that a plausible slip (a dropped term, a
transposed operand, a wrong index, a sum in the wrong order) fails it:

- Linear (src/tensor.rs:946-1118): one-hot inputs reproduce W's columns;
  small-integer operands make every partial sum exact, so the result equals
  an integer matrix product; random operands stay within the worst-case
  f32 dot-product bound of an f64 product.
- RMSNorm (src/tensor.rs:1140-1172): constant vectors in closed form, and the
  sequential f32 sum of squares shown on an input where pairwise summation
  would give a different scale.
- RoPE (src/model.rs:132-169): position 0 is the identity; the table equals
  BF16-rounded cos/sin of p * theta^(-2i/d).
- Attention (src/model.rs:313-397): the reference's own known-answer
  generator and tolerance (src/tensor.rs:9-83) against an f64 softmax; one
  key gives rb(V0); equal keys give the mean of V.
- CFG mix (src/sampling.rs:261-266): scale 1 gives the conditional row and
  scale 0 the unconditional one when the difference is exact.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O

from helpers import rb

f32 = np.float32


def _p(a):
    return a.ctypes.data


def _bf16(x) -> np.ndarray:
    return (rb(x).view(np.uint32) >> 16).astype(np.uint16)


def _as_f32(w16: np.ndarray) -> np.ndarray:
    return (w16.astype(np.uint32) << 16).view(np.float32)


def linear(w16, x):
    n, k = w16.shape
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    y = np.empty((x.shape[0], n), np.float32)
    O.lib().y2o_linear(_p(w16), n, k, _p(x), x.shape[0], _p(y))
    return y


def gemv_raw(w16, x):
    n, k = w16.shape
    y = np.empty(n, np.float32)
    x = np.ascontiguousarray(x, np.float32)  # kept alive across the call
    O.lib().y2o_gemv_raw(_p(w16), n, k, _p(x), _p(y))
    return y


@pytest.mark.parametrize("k", [1024, 3072, 2816, 520])
def test_linear_one_hot_reproduces_columns(k, oracle_threads):
    rng = np.random.default_rng(k)
    w16 = _bf16(rng.standard_normal((96, k)).astype(np.float32) * 0.02)
    w = _as_f32(w16)
    for j in [0, 7, 8, 63, 64, 511, 512, k - 1]:
        x = np.zeros(k, np.float32)
        x[j] = 1.0
        assert np.array_equal(linear(w16, x)[0], w[:, j])
        x[j] = -0.375
        assert np.array_equal(linear(w16, x)[0], rb(w[:, j] * f32(-0.375)))


@pytest.mark.parametrize("k", [1024, 3072, 8192])
def test_linear_small_integers_is_exact(k, oracle_threads):
    rng = np.random.default_rng(10 + k)
    wi = rng.integers(-8, 9, size=(64, k))
    xi = rng.integers(-8, 9, size=(2, k))
    y = linear(_bf16(wi.astype(np.float32)), xi.astype(np.float32))
    exact = (xi @ wi.T).astype(np.float64)  # |sum| < 2^24: every partial sum is exact in f32
    assert np.array_equal(y, rb(exact.astype(np.float32)))


@pytest.mark.parametrize("k", [8, 24, 64, 72, 504, 512, 520, 1000, 3072, 4104])
def test_linear_lanes_equal_the_scalar_dot(k, oracle_threads):
    """The linears run the DOT eight lanes at a time (vector fmas, the same
    chain per lane); every output equals the scalar y2o_dot_bf16 bit for bit,
    signed zeros included, for row lengths with partial 64- and 8-lane
    groups."""
    rng = np.random.default_rng(100 + k)
    n = 40
    w = rng.standard_normal((n, k)).astype(np.float32) * 0.05
    w[rng.random((n, k)) < 0.2] = 0.0
    w[3, :] = -0.0  # a row of negative zeros: -0 products
    w[5, :] = 0.0
    x = rng.standard_normal((2, k)).astype(np.float32)
    x[0, rng.random(k) < 0.3] = -0.0
    x[1, ::7] = 1e-30  # tiny products (flushed or subnormal: as the scalar chain)
    w16 = _bf16(w)
    got = linear(w16, x)
    dot = O.lib().y2o_dot_bf16
    dot.restype = C.c_float
    raw_want = np.empty_like(got)
    for r in range(2):
        xr = np.ascontiguousarray(x[r])
        for i in range(n):
            raw_want[r, i] = dot(C.c_void_p(_p(w16[i])), C.c_void_p(_p(xr)), k)
    want = rb(raw_want)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    raw = gemv_raw(w16, x[0])
    assert np.array_equal(rb(raw).view(np.uint32), want[0].view(np.uint32))


def test_gemv_within_dot_product_bound(oracle_threads):
    rng = np.random.default_rng(5)
    k = 3072
    w16 = _bf16(rng.standard_normal((256, k)).astype(np.float32) * 0.02)
    x = rb(rng.standard_normal(k).astype(np.float32))
    y = gemv_raw(w16, x).astype(np.float64)
    w = _as_f32(w16).astype(np.float64)
    ref = w @ x.astype(np.float64)
    gamma = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    bound = gamma * (np.abs(w) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y - ref) <= bound)
    # rows are independent: a row computed alone equals the same row in the batch
    assert np.array_equal(gemv_raw(w16[37:38].copy(), x)[0], y[37])


def test_norm_constant_vector_closed_form():
    n, eps = 1024, f32(1e-6)
    for c in [0.5, -2.0, 0.125]:
        x = np.full(n, c, np.float32)
        # the sum of squares n*c^2 is exact in f32 for these c
        want = rb(f32(1.0) / np.sqrt(f32(c * c) + eps))
        assert O.lib().y2o_norm_scale(_p(x), n, eps) == want
        g = np.full(n, 1.0, np.float32)
        out = np.empty(n, np.float32)
        O.lib().y2o_norm_apply(_p(x), 1, n, _p(g), eps, _p(out))
        assert np.array_equal(out, np.full(n, rb(rb(f32(c) * want)), np.float32))


def _scale(S, n, eps):
    return rb(f32(1.0) / np.sqrt(f32(S) / f32(n) + eps))[()]


def test_norm_sum_is_sequential():
    """x = [a, t, t, ...] with t^2 below half an ulp of a^2: the sequential
    f32 sum of squares stays fl(a*a) while the exact sum is larger.  a is
    chosen so that the BF16 scale of the two sums differs, so only the
    sequential order (src/tensor.rs:1144) passes."""
    n, eps = 4096, f32(1e-6)
    found = None
    for a in np.linspace(63.70, 63.80, 20001).astype(np.float32):
        t = f32(float(a) * 2.0 ** -13)
        x = np.full(n, t, np.float32)
        x[0] = a
        seq = np.cumsum(x * x, dtype=np.float32)[-1]  # sequential f32 sum
        exact = float(np.sum(x.astype(np.float64) ** 2))
        if _scale(seq, n, eps) != _scale(f32(exact), n, eps):
            found = x, _scale(seq, n, eps)
            break
    assert found is not None, "no separating input"
    x, want = found
    assert O.lib().y2o_norm_scale(_p(x), n, eps) == want


def test_rotary_position_zero_is_identity_and_table_matches_libm():
    d, theta, rows = 128, 10000.0, 64
    cos = np.empty(rows * d // 2, np.float32)
    sin = np.empty_like(cos)
    O.lib().y2o_rotary_table(0, rows, d, theta, _p(cos), _p(sin))
    cos, sin = cos.reshape(rows, d // 2), sin.reshape(rows, d // 2)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    x = rb(np.random.default_rng(0).standard_normal((1, 4 * d)).astype(np.float32))
    y = x.copy()
    c0, s0 = cos[0].copy(), sin[0].copy()
    O.lib().y2o_rotary_apply(_p(y), 1, 4 * d, d // 2, _p(c0), _p(s0))
    assert np.array_equal(x, y)
    # cos_i = rb(cosf(p * f_i)), f_i = 1 / powf(theta, 2i/d): compare with f64 libm,
    # allowing one BF16 step where the f32 argument sits on a rounding boundary
    i = np.arange(d // 2)
    f = (1.0 / np.power(np.float32(theta), (2 * i / d).astype(np.float32))).astype(np.float32)
    p = np.arange(rows, dtype=np.float32)[:, None]
    arg = (p * f[None, :]).astype(np.float32).astype(np.float64)
    for got, want in ((cos, rb(np.cos(arg).astype(np.float32))), (sin, rb(np.sin(arg).astype(np.float32)))):
        step = np.abs(want) * 2.0 ** -7 + 1e-30
        assert np.all(np.abs(got - want) <= step)
        assert np.mean(got == want) > 0.98


def _attention(q, K, V, heads, kv, dim):
    out = np.empty(heads * dim, np.float32)
    O.lib().y2o_attention_row(_p(q), _p(K), _p(V), K.shape[0], heads, kv, dim, _p(out))
    return out


def _kat_inputs(keys, heads, kv, dim, append):
    """The generator of src/tensor.rs:15-36."""
    i = np.arange(keys * kv * dim)
    K = rb(((i * 17 % 101).astype(np.float32) - f32(50.0)) * f32(0.06)).reshape(keys, kv * dim)
    V = rb(((i * 31 % 137).astype(np.float32) - f32(68.0)) * f32(0.007)).reshape(keys, kv * dim)
    j = np.arange(heads * dim)
    q = rb(((j * 23 % 97).astype(np.float32) - f32(48.0)) * f32(0.04))
    if append:
        a = np.arange(kv * dim).astype(np.float32)
        K = np.vstack([K, rb(a * f32(0.002) - f32(0.3))[None]])
        V = np.vstack([V, rb(f32(0.4) - a * f32(0.001))[None]])
    return q, np.ascontiguousarray(K), np.ascontiguousarray(V)


def _f64_attention(q, K, V, heads, kv, dim):
    """f64 softmax reference of src/tensor.rs:42-70."""
    out = np.empty(heads * dim, np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dim)))
    for h in range(heads):
        kh = h // (heads // kv)
        Kh = K[:, kh * dim:(kh + 1) * dim].astype(np.float64)
        Vh = V[:, kh * dim:(kh + 1) * dim].astype(np.float64)
        s = (Kh @ q[h * dim:(h + 1) * dim].astype(np.float64)) * scale
        e = np.exp(s - s.max())
        out[h * dim:(h + 1) * dim] = rb(((e @ Vh) / e.sum()).astype(np.float32))
    return out


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("keys", [4096, 4097, 7169, 8192, 16385, 24576])
def test_attention_reference_known_answer(dim, keys):
    heads, kv = 4, 2
    for append in ([0, 1] if keys < 24576 else [0]):
        q, K, V = _kat_inputs(keys, heads, kv, dim, append)
        got = _attention(q, K, V, heads, kv, dim)
        want = _f64_attention(q, K, V, heads, kv, dim)
        assert np.all(np.abs(got - want) <= 5e-5 + np.abs(want) * 0.008)


def test_attention_one_key_and_equal_keys():
    heads, kv, dim = 8, 2, 64
    rng = np.random.default_rng(4)
    q = rb(rng.standard_normal(heads * dim).astype(np.float32))
    K1 = rb(rng.standard_normal((1, kv * dim)).astype(np.float32))
    V1 = rb(rng.standard_normal((1, kv * dim)).astype(np.float32))
    out = _attention(q, K1, V1, heads, kv, dim)
    for h in range(heads):
        kh = h // (heads // kv)
        assert np.array_equal(out[h * dim:(h + 1) * dim], V1[0, kh * dim:(kh + 1) * dim])
    # 64 equal keys: p_j = 1/64 exactly; V = small integers / 8, so every
    # product and partial sum is exact and the output is rb(mean V)
    L = 64
    K = np.repeat(K1, L, axis=0)
    V = (rng.integers(-16, 17, size=(L, kv * dim)) / 8.0).astype(np.float32)
    out = _attention(q, K, np.ascontiguousarray(V), heads, kv, dim)
    mean = V.astype(np.float64).mean(axis=0).astype(np.float32)
    for h in range(heads):
        kh = h // (heads // kv)
        assert np.array_equal(out[h * dim:(h + 1) * dim], rb(mean[kh * dim:(kh + 1) * dim]))


@pytest.mark.parametrize("L", [8192, 16384, 16448, 24576])
def test_attention_equal_keys_over_super_blocks(L):
    """Equal keys at 128 blocks (no super-blocks), 256 / 257 blocks
    (super-blocks of 2, the last one short at 16448 keys) and 384 blocks:
    p_j = 1/L, and
    with V = small integers / 8 over a power-of-two L every product and
    partial sum is exact, so any association gives rb(mean V); a
    super-block dropped, counted twice or cut at the wrong block does not.
    (16448 keys: p = 1/16448 rounds, so the check there is the f64 mean
    within the known-answer tolerance.)"""
    heads, kv, dim = 4, 2, 64
    rng = np.random.default_rng(L)
    q = rb(rng.standard_normal(heads * dim).astype(np.float32))
    K = np.repeat(rb(rng.standard_normal((1, kv * dim)).astype(np.float32)), L, axis=0)
    V = (rng.integers(-8, 9, size=(L, kv * dim)) / 8.0).astype(np.float32)
    out = _attention(q, np.ascontiguousarray(K), V, heads, kv, dim)
    mean = V.astype(np.float64).mean(axis=0)
    for h in range(heads):
        kh = h // (heads // kv)
        want = mean[kh * dim:(kh + 1) * dim]
        if L & (L - 1) == 0:
            assert np.array_equal(out[h * dim:(h + 1) * dim], rb(want.astype(np.float32)))
        else:
            assert np.all(np.abs(out[h * dim:(h + 1) * dim] - want) <= 5e-5 + np.abs(want) * 0.008)
    assert [O.lib().y2o_superblock(n) for n in (1, 127, 128, 255, 256, 384)] == [1, 1, 1, 1, 2, 2]


def test_cfg_mix_closed_forms():
    rng = np.random.default_rng(6)
    # same binade, so c - u is exact in f32 and a BF16 value
    u = rb(rng.uniform(1.0, 2.0, 4096).astype(np.float32))
    c = rb(rng.uniform(1.0, 2.0, 4096).astype(np.float32))
    assert np.array_equal(O.cfg_mix(c, u, 1.0), c)
    assert np.array_equal(O.cfg_mix(c, u, 0.0), u)
    # scale 2 doubles the exact difference: u + 2(c - u) = 2c - u
    want = rb(u + rb(f32(2.0) * (c - u)))
    assert np.array_equal(O.cfg_mix(c, u, 2.0), want)
