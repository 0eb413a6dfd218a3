"""Device math routines equal the oracle's bit for bit (exp, log1p,
round_bf16 on every f32 bit pattern, SiLU, the ALU lane exchanges, and the
RMSNorm scale decisions next to BF16 rounding boundaries)."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
import yue2_rs_amd as y2

pytestmark = pytest.mark.gpu


def _device(which, x):
    out = np.empty_like(x)
    rc = y2.lib().yue2_hip_selftest_math(which, x.ctypes.data, out.ctypes.data, x.size)
    assert rc == 0, y2.lib().yue2_hip_last_error()
    return out


SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 88.72, 88.73, 89.0, -87.33, -103.0, -103.97, -104.0,
                    -150.0, 1e-30, -1e-30, np.inf, -np.inf, np.nan, 0.5, -0.5, 10.0], dtype=np.float32)


def test_expf_matches_oracle(gpu):
    rng = np.random.default_rng(1)
    x = np.concatenate([SPECIAL, rng.uniform(-110, 92, 300000).astype(np.float32),
                        rng.normal(0, 3, 300000).astype(np.float32)])
    got = _device(0, x)
    L = O.lib()
    want = np.array([L.y2o_expf(float(v)) for v in x], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_log1p_matches_oracle(gpu):
    rng = np.random.default_rng(2)
    u = (rng.integers(0, 2**53, 200000, dtype=np.uint64).astype(np.float64) / 2.0**53)
    x = np.concatenate([-u, [0.0, -0.0, -0.5, -1.0 + 2**-53, 1e-300, -1e-17]])
    got = _device(1, x)
    L = O.lib()
    want = np.array([L.y2o_log1p(float(v)) for v in x], dtype=np.float64)
    assert np.array_equal(got.view(np.uint64), want.view(np.uint64))


def test_round_and_silu_match_oracle(gpu):
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    # signalling NaNs change payload when ctypes passes them through a double,
    # so random patterns exclude NaNs; SPECIAL holds a quiet NaN.
    bits = bits[(bits & 0x7FFFFFFF) <= 0x7F800000]
    x = np.concatenate([SPECIAL, bits.view(np.float32)])
    got = _device(2, x)
    L = O.lib()
    want = np.array([L.y2o_round_bf16(float(v)) for v in x], dtype=np.float32)
    # NaNs: compare bit patterns too (quiet NaN with the top bits kept)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    g = (rng.normal(0, 4, 100000).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
    got = _device(3, g)
    # SiLU in f32 with the oracle's exp: rb(g / (1 + exp(-g)))
    e = np.array([L.y2o_expf(float(-v)) for v in g], dtype=np.float32)
    ref = (g / (np.float32(1.0) + e)).astype(np.float32)
    want = np.array([L.y2o_round_bf16(float(v)) for v in ref], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_round_matches_oracle_on_every_bit_pattern(gpu):
    """The device rounding (the gfx950 BF16 conversion instruction) equals the
    oracle's round_bf16 on all 2^32 f32 bit patterns: ties, denormals,
    infinities, quiet and signalling NaNs of both signs."""
    L = O.lib()
    chunk = 1 << 28
    for c in range(1 << 32 >> 28):
        bits = np.arange(c * chunk, (c + 1) * chunk, dtype=np.uint64).astype(np.uint32)
        got = _device(2, bits.view(np.float32)).view(np.uint32)
        want = np.empty_like(bits)
        L.y2o_round_bf16_bits(bits.ctypes.data, want.ctypes.data, bits.size)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, [(hex(int(bits[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:8]]


def test_lane_exchanges_are_exact(gpu):
    """The ALU lane exchanges (DPP, permlane swaps) read lane ^ m exactly, and
    the xor butterflies built on them give the same bits as __shfl_xor ones
    (the DOT order, attention score, PV stream and block sums all use them)."""
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.normal(0, 1, 64 * 1023).astype(np.float32),
                        np.tile(np.array([1e30, -1e30, 1e-30, -0.0, 0.0, 3.0, -3.0, 1.0], np.float32), 8)])
    lanes = np.arange(x.size) % 64
    base = np.arange(x.size) - lanes
    for j, m in enumerate([1, 2, 4, 8, 16, 32]):
        got = _device(4 + j, x)
        assert np.array_equal(got.view(np.uint32), x[base + (lanes ^ m)].view(np.uint32)), m
    for new, old in [(10, 11), (12, 13), (14, 15)]:
        assert np.array_equal(_device(new, x).view(np.uint32), _device(old, x).view(np.uint32)), new
    mx = _device(16, x).reshape(-1, 64)
    assert np.array_equal(mx, np.repeat(x.reshape(-1, 64).max(axis=1, keepdims=True), 64, axis=1))


def _near_boundary_rows(rng, count, n, eps):
    """Rows whose sum of squares puts the RMSNorm scale at a BF16 rounding
    midpoint (S = n (1 / m^2 - eps)), so the exact-interval test is undecided."""
    rows = []
    while len(rows) < count:
        e = rng.integers(-6, 7)
        mant = rng.integers(128, 256)
        mid = (mant * 2.0 ** (e - 7) + (mant + 1) * 2.0 ** (e - 7)) / 2.0
        S = n * (1.0 / mid ** 2 - float(eps))
        if S <= 0:
            continue
        x = np.sqrt(S / n) * (1.0 + 0.05 * rng.standard_normal(n))
        x *= np.sqrt(S / np.sum(x * x))
        rows.append(x.astype(np.float32))
    return rows


def test_block_norm_scales_match_chain_near_rounding_boundaries(gpu):
    """The block-wide two-row RMSNorm decision (every layer's norms) equals
    the oracle's sequential chain for each row: rows at BF16 rounding
    midpoints (the fallback chains, one per row, on different waves), ordinary
    rows, and pairs mixing the two."""
    rng = np.random.default_rng(12)
    n, eps = 128, np.float32(1e-6)
    near = _near_boundary_rows(rng, 1024, n, eps)
    ordinary = [(rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32) for _ in range(1024)]
    rows = []
    for i in range(1024):  # near/near, near/ordinary, ordinary/near, ordinary/ordinary
        k = i % 4
        rows += [near[i] if k in (0, 1) else ordinary[i], near[i] if k in (0, 2) else ordinary[(i + 1) % 1024]]
    x = np.concatenate(rows).astype(np.float32)
    got = _device(18, x).reshape(-1, n)
    L = O.lib()
    want = np.array([L.y2o_norm_scale(v.ctypes.data, n, float(eps)) for v in x.reshape(-1, n)], dtype=np.float32)
    assert np.all(got == got[:, :1])
    bad = np.nonzero(got[:, 0].view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, [(int(i), float(got[i, 0]), float(want[i])) for i in bad[:5]]


def test_wave_norm_scale_matches_chain_near_rounding_boundaries(gpu):
    """The wave-level RMSNorm decision (the QK head norms) equals the oracle's
    sequential chain, also for vectors whose sum of squares puts the scale
    next to a BF16 rounding boundary, where the exact-interval test cannot
    decide and the device runs the chain itself."""
    rng = np.random.default_rng(11)
    n, eps = 64, np.float32(1e-6)
    vecs = []
    # scales just around BF16 midpoints: S = n (1 / m^2 - eps)
    for _ in range(2048):
        e = rng.integers(-6, 7)
        mant = rng.integers(128, 256)
        lo = np.float32(mant * 2.0 ** (e - 7))
        hi = np.float32((mant + 1) * 2.0 ** (e - 7))
        mid = (float(lo) + float(hi)) / 2.0
        S = n * (1.0 / mid ** 2 - float(eps))
        if S <= 0:
            continue
        x = np.sqrt(S / n) * (1.0 + 0.05 * rng.standard_normal(n))
        x *= np.sqrt(S / np.sum(x * x))
        vecs.append(x.astype(np.float32))
    # ordinary vectors of assorted magnitudes
    while len(vecs) % 4 or len(vecs) < 4096:
        vecs.append((rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32))
    x = np.concatenate(vecs).astype(np.float32)
    got = _device(17, x).reshape(-1, n)
    assert np.all(got == got[:, :1]), "the scale is uniform over the wave"
    L = O.lib()
    want = np.array([L.y2o_norm_scale(v.ctypes.data, n, float(eps)) for v in x.reshape(-1, n)], dtype=np.float32)
    bad = np.nonzero(got[:, 0].view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, [(int(i), float(got[i, 0]), float(want[i])) for i in bad[:5]]
