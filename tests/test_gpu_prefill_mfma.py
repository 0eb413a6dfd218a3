"""The matrix-core prefill (yue2_hip_prefill_mfma): Model::prefill_phase
(src/model.rs:508-522) with BF16 MFMA GEMMs and a causal flash attention.

Its GEMM is pinned exactly where the order of summation cannot matter
(small-integer operands: every partial sum is an integer below 2^24) and
within the f64 bound gamma_K * sum |x| |w| on random BF16 operands, at tile
edges (M, N not multiples of the 128-wide tiles).

The whole prefill keeps every BF16 rounding point of the decode step but
sums in another order (as the reference's MPS prefill GEMMs differ from its
decode GEMVs, src/tensor.rs:991-993), so a rounding point now and then lands
on the other side of a BF16 tie and the difference travels down the
residual stream.  The tolerance contract, stated against the oracle's
decode-order prefill on the same seeded checkpoint and prompt:
  * two layers (reduced config and the 3B layer shape): max |logit
    difference| <= 0.08 * std(oracle logits), for the prefill's last row and
    for the decode step after it (through the MFMA-filled cache); measured
    about 0.035 * std;
  * all 28 layers of the 3B config, 2048 tokens, against the bit-exact
    decode-order GPU prefill: <= 0.30 * std (measured about 0.16 * std, the
    difference growing as the square root of the depth);
  * the argmax of every compared row is the same id (the 24000-token
    full-depth case reports it only: see its test);
  * phase-restricted heads: the same -inf pattern.
Prompts of 1 token (the attention over one key), 65 and 1100 tokens cross
the 64-key and 128-query flash tiles; 4100 tokens (against the decode-order
GPU prefill, itself bit-exact with the oracle) cross the 4096-row chunks of
the prefill; 24000 tokens at the 3B layer shape (two layers) are the long
prompt of the long-context workload: six chunks, up to 375 key tiles per
query tile."""
import dataclasses

import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
import yue2_rs_amd as y2

from helpers import bits

pytestmark = pytest.mark.gpu

TWO_LAYER_TOL = 0.08
FULL_DEPTH_TOL = 0.30


def _bf16(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def _f64(b16):
    return (b16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _gemm(x16, w16):
    (M, K), N = x16.shape, w16.shape[0]
    out = np.empty((M, N), np.float32)
    rc = y2.lib().yue2_hip_selftest_gemm(x16.ctypes.data, w16.ctypes.data, out.ctypes.data, M, N, K)
    assert rc == 0, y2.lib().yue2_hip_last_error().decode()
    return out


@pytest.mark.parametrize("M,N,K", [(1, 1, 64), (128, 128, 64), (200, 300, 192), (257, 129, 512)])
def test_gemm_small_integers_exact(gpu, M, N, K):
    rng = np.random.default_rng(M * 7 + N)
    x = _bf16(rng.integers(-4, 5, (M, K)).astype(np.float32))
    w = _bf16(rng.integers(-4, 5, (N, K)).astype(np.float32))
    want = _f64(x) @ _f64(w).T
    assert np.array_equal(_gemm(x, w), want.astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(257, 129, 512), (1000, 3072, 3072)])
def test_gemm_random_within_bound(gpu, M, N, K):
    rng = np.random.default_rng(K)
    x = _bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = _bf16(rng.standard_normal((N, K)).astype(np.float32))
    xf, wf = _f64(x), _f64(w)
    u = 2.0 ** -24
    bound = (K * u / (1 - K * u)) * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(_gemm(x, w) - xf @ wf.T) <= bound)


def test_gemm_rejects_ragged_k(gpu):
    x = np.zeros((4, 96), np.uint16)
    out = np.empty((4, 4), np.float32)
    assert y2.lib().yue2_hip_selftest_gemm(x.ctypes.data, x.ctypes.data, out.ctypes.data, 4, 4, 96) < 0


def _close(got, want, tol, what, argmax=True):
    """max |got - want| <= tol * std(want) over the finite entries, and
    (argmax) the same argmax.  Without `argmax` the argmax is only reported:
    where the oracle's two largest logits are closer than twice the measured
    difference the bound allows either one, and where they are not the bound
    implies the same argmax."""
    fin = np.isfinite(want)
    assert np.array_equal(fin, np.isfinite(got)), f"{what}: -inf pattern differs"
    d = np.abs(got[fin] - want[fin]).max()
    s = want[fin].std()
    top2 = np.sort(want[fin])[-2:]
    print(f"{what}: max |d| {d:.4g} = {d / s:.4f} std; top-two margin {top2[1] - top2[0]:.4g}, "
          f"argmax {int(np.argmax(got))} vs {int(np.argmax(want))}", flush=True)
    assert d <= tol * s, f"{what}: max |d| {d:.4g} > {tol} * std {s:.4g}"
    if argmax:
        assert int(np.argmax(got)) == int(np.argmax(want)), f"{what}: argmax differs"


THREE_B_2L = dataclasses.replace(synthetic.CLASS_3B, num_hidden_layers=2, vocab_size=32768)


@pytest.fixture(scope="module", params=["reduced", "3b-2layer"])
def two_layer(request, gpu, oracle_threads):
    cfg = synthetic.REDUCED if request.param == "reduced" else THREE_B_2L
    ck = synthetic.checkpoint(cfg, seed=0)
    gm = y2.Model.open(ck)
    yield cfg, gm, O.Model(ck)
    gm.close()


@pytest.mark.parametrize("n", [1, 65, 1100])
def test_prefill_within_tolerance(two_layer, n):
    cfg, gm, om = two_layer
    print(f"prefill_mfma {cfg.hidden_size}x{cfg.num_hidden_layers} n={n}", flush=True)
    ids = synthetic.prompt(n, cfg.vocab_size, seed=n)
    gc, gl = gm.prefill_mfma(ids, n + 2)
    oc, ol = om.prefill(ids, n + 2)
    assert gc.length == n
    _close(gl, ol, TWO_LAYER_TOL, "prefill logits")
    t = int(np.argmax(ol))
    _close(gm.forward([t], gc), om.forward([t], oc), TWO_LAYER_TOL, "next-step logits")
    gc.close()


def test_prefill_crosses_chunks(gpu):
    ck = synthetic.checkpoint(synthetic.REDUCED, seed=3)
    gm = y2.Model.open(ck)
    try:
        n = 4100
        ids = synthetic.prompt(n, synthetic.REDUCED.vocab_size, seed=5)
        c1, l1 = gm.prefill_phase(ids, n + 2)
        c2, l2 = gm.prefill_mfma(ids, n + 2)
        assert c2.length == n
        _close(l2, l1, TWO_LAYER_TOL, "prefill logits")
        t = int(np.argmax(l1))
        _close(gm.forward([t], c2), gm.forward([t], c1), TWO_LAYER_TOL, "next-step logits")
        c1.close()
        c2.close()
    finally:
        gm.close()


def test_prefill_24000_tokens_3b_shape(gpu):
    cfg = dataclasses.replace(synthetic.CLASS_3B, num_hidden_layers=2, vocab_size=32768)
    gm = y2.Model.open(synthetic.checkpoint(cfg, seed=4, threads=16))
    try:
        n = 24000
        ids = synthetic.prompt(n, cfg.vocab_size, seed=6)
        c1, l1 = gm.prefill_phase(ids, n + 2)
        c2, l2 = gm.prefill_mfma(ids, n + 2)
        assert c2.length == n
        _close(l2, l1, TWO_LAYER_TOL, "24000-token prefill logits")
        t = int(np.argmax(l1))
        _close(gm.forward([t], c2), gm.forward([t], c1), TWO_LAYER_TOL, "next-step logits")
        c1.close()
        c2.close()
    finally:
        gm.close()


def test_prefill_needs_empty_cache(two_layer):
    cfg, gm, om = two_layer
    gc, _ = gm.prefill_mfma([1, 2, 3], 8)
    out = np.empty(cfg.vocab_size, np.float32)
    ids = np.array([4], np.int32)
    assert y2.lib().yue2_hip_prefill_mfma(gm._h, gc._h, ids.ctypes.data, 1, 0, out.ctypes.data) < 0
    gc.close()


def test_phase_heads(gpu, oracle_threads):
    from test_gpu_phase import TINY, FOUR, ONE, EOD, ABC_END, MUSIC_END, CODEC_OFFSET
    ck = synthetic.checkpoint(TINY, seed=11)
    ck.embed_tokens[:, 0] = FOUR
    ck.lm_head[:EOD, 0] = 0
    ck.lm_head[CODEC_OFFSET:, 0] = 0
    ck.lm_head[ABC_END, 0] = ONE
    ck.lm_head[MUSIC_END, 0] = ONE
    gm, om = y2.Model.open(ck), O.Model(ck)
    try:
        for phase in (y2.PHASE_ABC, y2.PHASE_SEMANTIC):
            ids = synthetic.prompt(80, TINY.vocab_size, seed=phase)
            gc, gl = gm.prefill_mfma(ids, 96, phase)
            oc, ol = om.prefill(ids, 96, phase)
            _close(gl, ol, TWO_LAYER_TOL, f"phase {phase}")
            gc.close()
    finally:
        gm.close()


def test_full_depth_3b_against_decode_order_prefill(gpu):
    """28 layers, 2048 tokens: the MFMA prefill against the bit-exact
    decode-order GPU prefill (itself pinned to the oracle elsewhere)."""
    ck = synthetic.checkpoint(synthetic.CLASS_3B, seed=0, threads=16)
    gm = y2.Model.open(ck)
    try:
        ids = synthetic.prompt(2048, synthetic.CLASS_3B.vocab_size, seed=1)
        c1, l1 = gm.prefill_phase(ids, 2050)
        c2, l2 = gm.prefill_mfma(ids, 2050)
        _close(l2, l1, FULL_DEPTH_TOL, "3B prefill logits")
        c3, l3 = gm.prefill_mfma(ids, 2050)
        assert np.array_equal(bits(l2), bits(l3)), "MFMA prefill is not deterministic"
        t = int(np.argmax(l1))
        _close(gm.forward([t], c2), gm.forward([t], c1), FULL_DEPTH_TOL, "3B next-step logits")
        for c in (c1, c2, c3):
            c.close()
    finally:
        gm.close()


@pytest.mark.timeout(900)
def test_full_depth_3b_24000_tokens_against_decode_order_prefill(gpu):
    """The long-context workload's prompt at full depth: 28 layers, 24000
    tokens, the MFMA prefill against the bit-exact decode-order GPU prefill
    (24000 token steps), within the same full-depth bound; then the decode
    step after it through each cache.  At this depth and length the two
    largest logits can sit closer than the bound (measured: a 0.17 std
    difference flipped the next step's argmax), so the argmax is reported,
    not required."""
    ck = synthetic.checkpoint(synthetic.CLASS_3B, seed=0, threads=16)
    gm = y2.Model.open(ck)
    try:
        n = 24000
        ids = synthetic.prompt(n, synthetic.CLASS_3B.vocab_size, seed=0)
        c2, l2 = gm.prefill_mfma(ids, n + 2)
        print("matrix-core prefill done; decode-order prefill of 24000 tokens", flush=True)
        c1, l1 = gm.prefill_phase(ids, n + 2)
        _close(l2, l1, FULL_DEPTH_TOL, "3B 24000-token prefill logits", argmax=False)
        t = int(np.argmax(l1))
        _close(gm.forward([t], c2), gm.forward([t], c1), FULL_DEPTH_TOL, "3B next-step logits at 24001",
               argmax=False)
        c1.close()
        c2.close()
    finally:
        gm.close()
