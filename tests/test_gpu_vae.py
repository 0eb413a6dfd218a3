"""The VAE decoder on the device (yue2_hip_vae_*, src/vae.rs) against the
oracle's restatement (tests/test_oracle_vae.py pins it).

- The reference's own convolution known-answer cases through the device
  convolution kernel, at the reference's tolerance 2e-6, and two transposed
  ones with kernel < stride (output phases that see no tap get the bias).
- Shapes that reach every branch of the matrix-core (FP32 MFMA) and narrow
  convolution kernels against a float64 convolution: max |difference|
  <= 1e-5 (FP32 sums of at most 910 products of magnitude < 0.5).
- Whole decodes of synthetic checkpoints written in the reference's layout
  (SnakeBeta and ELU variants; one with 256 channels, so several input
  chunks and output tiles per convolution; one without the final tanh):
  FP32 throughout but in another summation order.  The contract: the device
  is as close to an independent float64 evaluation as the FP32 oracle is,
  max |device - f64| <= 4 * max |oracle - f64| + 1e-6 (the wide random
  network amplifies rounding: its activations reach ~200 and both FP32 paths
  sit ~1e-3 from float64; the small ones ~5e-5).
- The full Oobleck shape of the reference's default ratio (widths 128 x (1,
  2, 4, 8, 16), strides (2, 4, 4, 6, 10): 1024- and 2048-channel tiles, ten-
  and six-phase transposed convolutions) on 2 latent frames, with the
  weight-norm gains scaled by 0.3 so the activations stay O(1) and FP32
  rounding is not amplified into noise (at gain 1 the oracle itself is 0.1
  from float64 there): the same contract against float64, and against the
  oracle.
- decode_tiled with the required halo equals the whole decode bit for bit
  (every output sees the same arithmetic); a smaller halo is refused; the
  reference's configuration checks and messages."""
import json

import numpy as np
import pytest

from oracle import oracle as O
import yue2_rs_amd as y2
from yue2_rs_amd import synthetic

from test_oracle_vae import KAT, SPARSE, kat_case
from vae_files import CONV_SHAPES, conv_case, decode_f64, oracle_ops, required_halo, synthetic_vae, write_vae_dir

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", KAT + SPARSE)
def test_convolution_known_answers(gpu, case):
    transpose, stride, padding, dilation, kernel = case
    x, w, bias, expected = kat_case(*case)
    out = np.empty(expected.shape, np.float32)
    rc = y2.lib().yue2_hip_selftest_conv(int(transpose), x.shape[1], 4, kernel, stride, padding, dilation,
                                         x.ctypes.data, x.shape[0], np.ascontiguousarray(w).ctypes.data,
                                         bias.ctypes.data, out.ctypes.data)
    assert rc == 0, y2.lib().yue2_hip_last_error().decode()
    assert np.abs(out - expected).max() < 2e-6


def _selftest(transpose, cin, cout, kernel, stride, padding, dilation, x, w, bias, length):
    out = np.empty((length, cout), np.float32)
    rc = y2.lib().yue2_hip_selftest_conv(int(transpose), cin, cout, kernel, stride, padding, dilation,
                                         x.ctypes.data, x.shape[0], np.ascontiguousarray(w).ctypes.data,
                                         bias.ctypes.data, out.ctypes.data)
    assert rc == 0, y2.lib().yue2_hip_last_error().decode()
    return out


@pytest.mark.parametrize("shape", CONV_SHAPES)
def test_convolution_shapes(gpu, shape):
    transpose, cin, cout, kernel, stride, padding, dilation, frames = shape
    x, w, b, want = conv_case(*shape)
    got = _selftest(transpose, cin, cout, kernel, stride, padding, dilation, x, w, b, want.shape[0])
    assert np.abs(got - want).max() <= 1e-5


CASES = {
    "snake": dict(seed=1),
    "elu": dict(seed=2, snake=False),
    "wide": dict(seed=3, channels=32, c_mults=(2, 4, 8), strides=(2, 4, 2)),
    "no-tanh": dict(seed=4, final_tanh=False),
}


@pytest.mark.parametrize("name", list(CASES))
def test_decode_matches_oracle(gpu, tmp_path, name):
    cfg, t = synthetic_vae(**CASES[name])
    vae = y2.Vae(write_vae_dir(tmp_path / name, cfg, t))
    try:
        ops = oracle_ops(cfg, t)
        frames = 30
        z = np.random.default_rng(7).standard_normal((frames, cfg["latent_dim"])).astype(np.float32)
        assert vae.output_length(frames) == ops.length(frames)
        got, want = vae.decode(z), ops.run(z)
        assert got.shape == want.shape
        exact = decode_f64(cfg, t, z)
        d, ref = np.abs(got - exact).max(), np.abs(want - exact).max()
        print(f"{name}: device-f64 {d:.3g}, oracle-f64 {ref:.3g}, device-oracle {np.abs(got - want).max():.3g}",
              flush=True)
        assert d <= 4 * ref + 1e-6
    finally:
        vae.close()


def test_decode_1920_shape(gpu, tmp_path):
    cfg, t = synthetic.vae(0, **synthetic.VAE_1920)
    t = {k: (v * np.float32(0.3) if k.endswith("weight_g") else v) for k, v in t.items()}
    vae = y2.Vae(write_vae_dir(tmp_path / "big", cfg, t))
    try:
        z = np.random.default_rng(1).standard_normal((2, cfg["latent_dim"])).astype(np.float32)
        got = vae.decode(z)
        exact = decode_f64(cfg, t, z)
        want = oracle_ops(cfg, t).run(z)
        assert got.shape == want.shape == exact.shape == (2 * 1920, 2)
        d, ref = np.abs(got - exact).max(), np.abs(want - exact).max()
        print(f"1920 shape: device-f64 {d:.3g}, oracle-f64 {ref:.3g}, device-oracle {np.abs(got - want).max():.3g}, "
              f"output std {exact.std():.3g}", flush=True)
        assert d <= 4 * ref + 1e-6
    finally:
        vae.close()


def test_tiled_decode_is_the_whole_decode(gpu, tmp_path):
    cfg, t = synthetic_vae(seed=5)
    vae = y2.Vae(write_vae_dir(tmp_path / "v", cfg, t))
    try:
        core = 8
        halo = vae.required_halo(core)
        assert halo == required_halo(cfg, core)
        z = np.random.default_rng(3).standard_normal((45, cfg["latent_dim"])).astype(np.float32)
        full = vae.decode(z)
        tiled = vae.decode_tiled(z, core, halo)
        assert np.array_equal(tiled.view(np.uint32), full.view(np.uint32))
        with pytest.raises(y2.Yue2Error, match="VAE halo must be at least"):
            vae.decode_tiled(z, core, halo - 1)
        bad = z.copy()
        bad[40, 3] = np.inf  # the latent is validated before the halo, as validate_latent runs first
        with pytest.raises(y2.Yue2Error, match="Expected finite nonempty"):
            vae.decode_tiled(bad, core, halo - 1)
    finally:
        vae.close()


def test_configuration_checks(gpu, tmp_path):
    cfg, t = synthetic_vae(seed=6)
    bad = dict(cfg, model_type="other")
    with pytest.raises(y2.Yue2Error, match="Expected YuE2 VAE checkpoint"):
        y2.Vae(write_vae_dir(tmp_path / "a", bad, t))
    bad = json.loads(json.dumps(cfg))
    bad["downsampling_ratio"] = 9
    with pytest.raises(y2.Yue2Error, match="VAE configuration mismatch"):
        y2.Vae(write_vae_dir(tmp_path / "b", bad, t))
    missing = {k: v for k, v in t.items() if not k.endswith("layers.0.weight_g")}
    with pytest.raises(y2.Yue2Error, match="Missing checkpoint tensor"):
        y2.Vae(write_vae_dir(tmp_path / "c", cfg, missing))
    vae = y2.Vae(write_vae_dir(tmp_path / "d", cfg, t))
    try:
        with pytest.raises(y2.Yue2Error):
            vae.decode(np.full((4, cfg["latent_dim"]), np.nan, np.float32))
    finally:
        vae.close()
