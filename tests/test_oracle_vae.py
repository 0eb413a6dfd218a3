"""Pins of the oracle's VAE decoder (y2o_conv, y2o_vae_*; src/vae.rs).

- The reference's own convolution known-answer test
  (metal_convolutions_match_scalar_reference, src/vae.rs:812-892): its six
  (transpose, stride, padding, dilation, kernel) cases, its input generators
  and scalar formula, and its tolerance 2e-6.
- Closed forms of the activations: SnakeBeta with alpha = beta parameters 0
  (alpha = beta = 1) is x + sin(x)^2 / (1 + 1e-9); ELU; tanh.
- The weight norm: the effective weights read back through a 1-tap
  convolution of one-hot rows have row norms |g|.
- Conv::length and a tiled decode equal to the whole decode on every core
  row (each output depends only on its receptive field).
- The float64 convolution the device self-tests use, against the same
  known answers, and the oracle's convolution against it on those shapes.
- The whole decoder against an independent float64 evaluation: within the
  FP32 rounding the network's gain allows (1e-4 of the output scale on a
  small network; the wide one amplifies it, see the device test)."""
import numpy as np
import pytest

from oracle import oracle as O
from vae_files import CONV_SHAPES, conv_case, conv_f64, decode_f64, decode_tiled, oracle_ops, required_halo, synthetic_vae

KAT = [(False, 1, 3, 1, 7), (False, 1, 9, 3, 7), (False, 2, 1, 1, 4), (True, 2, 1, 1, 4), (True, 5, 3, 1, 10),
       (True, 6, 3, 1, 12)]
# beyond the reference's cases: transposed convolutions with kernel < stride,
# whose output phases without a tap hold the bias alone
SPARSE = [(True, 4, 0, 1, 2), (True, 3, 1, 1, 2)]


def kat_case(transpose, stride, padding, dilation, kernel):
    frames, ci, co = 19, 3, 4
    x = np.array([((i * 7 % 31) - 15.0) * 0.03 for i in range(frames * ci)], np.float32).reshape(frames, ci)
    w = np.array([((i * 13 % 37) - 18.0) * 0.01 for i in range(ci * co * kernel)], np.float32)
    bias = np.array([0.1, -0.2, 0.3, -0.4], np.float32)
    if transpose:
        length = (frames - 1) * stride + kernel - 2 * padding
    else:
        length = (frames + 2 * padding - dilation * (kernel - 1) - 1) // stride + 1
    expected = np.empty((length, co), np.float64)
    for t in range(length):
        for o in range(co):
            e = float(bias[o])
            for i in range(ci):
                for k in range(kernel):
                    if transpose:
                        pos = t + padding - k * dilation
                        if pos % stride:
                            continue
                        src = pos // stride
                    else:
                        src = t * stride + k * dilation - padding
                    if not 0 <= src < frames:
                        continue
                    idx = (i * co + o) * kernel + k if transpose else (o * ci + i) * kernel + k
                    e += float(x[src, i]) * float(w[idx])
            expected[t, o] = e
    wshape = (ci, co, kernel) if transpose else (co, ci, kernel)
    return x, w.reshape(wshape), bias, expected


@pytest.mark.parametrize("case", KAT + SPARSE)
def test_convolution_known_answers(case):
    transpose, stride, padding, dilation, kernel = case
    x, w, bias, expected = kat_case(*case)
    got = O.conv(transpose, x, w, bias, kernel, stride, padding, dilation)
    assert got.shape == expected.shape
    assert np.abs(got - expected).max() < 2e-6


def test_activation_closed_forms():
    x = np.linspace(-3, 3, 4 * 5, dtype=np.float32).reshape(4, 5)
    zero = np.zeros(5, np.float32)
    snake = O.VaeOps([(O.VAE_SNAKE, {}, dict(alpha=zero, beta=zero))]).run(x)
    want = x + (np.sin(x.astype(np.float64)) ** 2 / (1.0 + 1e-9)).astype(np.float32)
    assert np.abs(snake - want).max() < 2e-6
    elu = O.VaeOps([(O.VAE_ELU, {}, {})]).run(x)
    assert np.abs(elu - np.where(x < 0, np.expm1(x.astype(np.float64)), x)).max() < 2e-6
    th = O.VaeOps([(O.VAE_TANH, {}, {})]).run(x)
    assert np.abs(th - np.tanh(x.astype(np.float64))).max() < 2e-6


@pytest.mark.parametrize("transpose", [False, True])
def test_weight_norm_rows(transpose):
    rng = np.random.default_rng(3)
    cin, cout = 5, 6
    v = rng.standard_normal((cin, cout, 1) if transpose else (cout, cin, 1)).astype(np.float32)
    g = rng.uniform(0.5, 2.0, (v.shape[0], 1, 1)).astype(np.float32)
    op = (O.VAE_CONVT if transpose else O.VAE_CONV,
          dict(cin=cin, cout=cout, kernel=1, stride=1, padding=0, dilation=1), dict(v=v, g=g, b=None))
    w = O.VaeOps([op]).run(np.eye(cin, dtype=np.float32))  # row t = weights from input channel t
    rows = w if transpose else w.T  # the norm runs over v's first dimension
    assert np.allclose(np.linalg.norm(rows.astype(np.float64), axis=1), g.ravel(), rtol=1e-5)


def test_lengths_and_tiling():
    cfg, t = synthetic_vae(seed=1)
    ops = oracle_ops(cfg, t)
    ratio = cfg["downsampling_ratio"]
    for frames in (1, 5, 20):  # even strides: each transposed layer multiplies the length by its stride
        assert ops.length(frames) == frames * ratio
    odd = oracle_ops(*synthetic_vae(seed=1, strides=(2, 3)))
    # (n - 1) s + 2 s - 2 ceil(s / 2) per transposed layer, the last stride first: 3, then 2
    n1 = (5 - 1) * 3 + 6 - 2 * 2
    assert odd.length(5) == (n1 - 1) * 2 + 4 - 2 * 1
    z = np.random.default_rng(2).standard_normal((60, cfg["latent_dim"])).astype(np.float32)
    full = ops.run(z)
    assert full.shape == (60 * ratio, cfg["audio_channels"])
    assert np.all(np.abs(full) <= 1.0)  # final tanh
    halo = required_halo(cfg, 8)
    tiled = decode_tiled(ops.run, z, 8, halo, ratio, full.shape[0])
    assert np.array_equal(tiled.view(np.uint32), full.view(np.uint32))
    # one frame less of halo changes the outputs next to some tile edge
    short = decode_tiled(ops.run, z, 8, halo - 1, ratio, full.shape[0])
    assert not np.array_equal(short.view(np.uint32), full.view(np.uint32))


@pytest.mark.parametrize("kw", [dict(seed=1), dict(seed=2, snake=False), dict(seed=4, final_tanh=False)])
def test_decoder_against_float64(kw):
    cfg, t = synthetic_vae(**kw)
    z = np.random.default_rng(7).standard_normal((30, cfg["latent_dim"])).astype(np.float32)
    got = oracle_ops(cfg, t).run(z)
    want = decode_f64(cfg, t, z)
    assert np.abs(got - want).max() <= 1e-4 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("case", KAT + SPARSE)
def test_float64_convolution_known_answers(case):
    transpose, stride, padding, dilation, kernel = case
    x, w, bias, expected = kat_case(*case)
    got = conv_f64(transpose, x, w, bias, kernel, stride, padding, dilation)
    assert np.abs(got - expected).max() < 1e-12


@pytest.mark.parametrize("shape", CONV_SHAPES)
def test_oracle_convolution_shapes(shape):
    transpose, cin, cout, kernel, stride, padding, dilation, frames = shape
    x, w, b, want = conv_case(*shape)
    got = O.conv(transpose, x, w, b, kernel, stride, padding, dilation)
    assert got.shape == want.shape
    assert np.abs(got - want).max() < 1e-5
