"""CPU: the oracle's scalar math against closed forms and independent
libraries (no GPU).

- round_bf16 (src/tensor.rs:645-652): checked as "nearest BF16, ties to even
  mantissa, NaN stays a quiet NaN", computed from the two BF16 neighbours in
  f64, not from the bit trick the oracle uses.
- expf (the oracle's stand-in for Accelerate's vvexpf and Rust's f32::exp):
  correctly rounded, i.e. equal to numpy's f64 exp rounded once to f32.
- log1p (Rust's f64::ln_1p in the sampler's race, src/sampling.rs:205):
  within 2 ulp of numpy's log1p.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O


def _bf16_neighbours(v: np.float32):
    b = int(np.float32(v).view(np.uint32))
    lo = b & 0xFFFF0000
    hi = lo + 0x10000
    return lo, hi


def _expected_rne(v: np.float32) -> int:
    """Bits of the nearest BF16 to v, ties to even, from its neighbours."""
    lo, hi = _bf16_neighbours(v)
    flo = float(np.uint32(lo).view(np.float32))
    hi_exp = (hi >> 23) & 0xFF
    fhi = math.copysign(2.0 ** 128, flo) if hi_exp == 0xFF else float(np.uint32(hi).view(np.float32))
    x = float(v)
    dlo, dhi = abs(x - flo), abs(fhi - x)
    if dlo < dhi:
        return lo
    if dhi < dlo:
        return hi
    return lo if ((lo >> 16) & 1) == 0 else hi


def test_round_bf16_is_nearest_ties_to_even():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, size=60000, dtype=np.uint64).astype(np.uint32)
    # exact ties (low half 0x8000) and one-off neighbours, across exponents
    hi = rng.integers(0, 2 ** 16, size=6000, dtype=np.uint64).astype(np.uint32) << 16
    bits = np.concatenate([bits, hi | 0x8000, hi | 0x7FFF, hi | 0x8001, hi])
    f = O.lib().y2o_round_bf16
    checked = 0
    for b in bits:
        v = np.uint32(b).view(np.float32)
        got = int(np.float32(f(float(v))).view(np.uint32))
        if np.isnan(v):
            assert (got & 0xFFFF) == 0 and np.isnan(np.uint32(got).view(np.float32))
            assert got & 0x00400000, "NaN must come back quiet"
            continue
        if np.isinf(v):
            assert got == int(b)
            continue
        assert got == _expected_rne(v), hex(int(b))
        checked += 1
    assert checked > 60000


def test_expf_is_correctly_rounded():
    rng = np.random.default_rng(2)
    xs = np.concatenate([
        rng.uniform(-20, 20, 40000), rng.uniform(-104, 89, 40000), rng.uniform(-1e-3, 1e-3, 5000),
        rng.uniform(88.0, 89.5, 2000), rng.uniform(-105, -102.5, 2000),
        np.array([0.0, -0.0, 1.0, -1.0, 88.72283, 88.72284, -87.33655, -103.27893, -103.97208]),
    ]).astype(np.float32)
    f = O.lib().y2o_expf
    with np.errstate(over="ignore", under="ignore"):
        want = np.exp(xs.astype(np.float64)).astype(np.float32)
    got = np.array([f(float(x)) for x in xs], dtype=np.float32)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, [(float(xs[i]), float(got[i]), float(want[i])) for i in bad[:5]]
    assert f(float("inf")) == float("inf") and f(float("-inf")) == 0.0
    assert math.isnan(f(float("nan")))


def test_log1p_within_two_ulp():
    rng = np.random.default_rng(3)
    # the race uses log1p(-u), u uniform in [0, 1) with 53-bit resolution
    u = rng.random(50000)
    xs = np.concatenate([-u, rng.uniform(-0.999999, 50.0, 20000), -(2.0 ** -rng.uniform(1, 60, 5000)),
                         np.array([0.0, -0.5, 1e-300, -1e-17, 1.0])])
    f = O.lib().y2o_log1p
    got = np.array([f(float(x)) for x in xs])
    want = np.log1p(xs)
    ulp = np.spacing(np.abs(want))
    err = np.abs(got - want) / np.maximum(ulp, np.finfo(np.float64).tiny)
    assert err.max() <= 2.0, float(xs[int(np.argmax(err))])
    assert f(0.0) == 0.0
    assert f(-1.0) == float("-inf")


def test_round_bf16_bits_matches_scalar_and_keeps_nan_payload():
    """The array form rounds like the scalar one, and signalling NaNs come back
    quiet with their sign and top payload bits."""
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, size=20000, dtype=np.uint64).astype(np.uint32)
    bits = np.concatenate([bits, np.array([0x7F800001, 0xFF800001, 0x7FA12345, 0xFFBFFFFF, 0x7FC00000,
                                           0x7F800000, 0xFF800000, 0x00008000, 0x00018000, 0x7F7F8000],
                                          dtype=np.uint32)])
    out = np.empty_like(bits)
    L = O.lib()
    L.y2o_round_bf16_bits(bits.ctypes.data, out.ctypes.data, bits.size)
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    assert np.array_equal(out[nan], (bits[nan] & 0xFFFF0000) | 0x00400000)
    for b, o in zip(bits[~nan][:4000], out[~nan][:4000]):
        assert int(np.float32(L.y2o_round_bf16(float(np.uint32(b).view(np.float32)))).view(np.uint32)) == int(o)
    # ties to even: 0x00008000 -> 0, 0x00018000 -> 0x00020000; the largest
    # finite value's tie rounds to infinity
    assert list(out[-3:]) == [0, 0x00020000, 0x7F800000]
