"""Pins of the oracle's NAR velocity (y2o_velocity, Model::velocity
src/model.rs:611-698) without the reference.

1. Closed forms: with every NAR layer matrix zero, each layer leaves x as it
   is (o_proj and down_proj contribute +0), so the output is
   llm2vae(final_norm(x0[1 .. n-1])).  With one-hot vae2llm / time / llm2vae
   matrices every DOT is exact, and x0 = rb(rb(rb(pad + rb(b)) + time) + pe)
   reduces to the padded rows, the biases, the timestep embedding and the
   (clamped) latent position rows, stated here directly from the reference's
   lines; the norm's sum is the sequential f32 chain.
2. An independent float64 restatement of the whole velocity (every product
   and sum in f64, BF16 rounding points kept, plain softmax and matmuls) on a
   small two-layer model with a non-empty AR cache: the oracle agrees within
   a stated tolerance, so a wrong key set, RoPE offset, row slice or layer
   order (each a large difference) would fail.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from yue2_rs_amd import synthetic
from yue2_rs_amd.api import Config, LayerWeights

from helpers import rb

TINY = Config(hidden_size=128, num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1, head_dim=64,
              intermediate_size=256, vocab_size=512, max_position_embeddings=4096, rms_norm_eps=1e-6,
              rope_theta=10000.0)
LATENT = 64


def f32(x):
    return np.float32(x)


def bf16_bits(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def f_of(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def exp32(x):
    """The correctly rounded f32 exp (the oracle's substitute for f32::exp)."""
    return np.float32(np.exp(np.float64(x)))


def rbs(x):
    """round_bf16 of one f32 scalar."""
    return np.float32(rb(np.array([x], np.float32))[0])


def seq_norm(x, gamma, eps):
    s = np.float32(-0.0)
    for v in x.astype(np.float32):
        s = np.float32(s + np.float32(v * v))
    sc = rb(np.float32(1.0) / np.sqrt(np.float32(s / np.float32(len(x)) + np.float32(eps))))
    return rb(rb(x * sc) * gamma)


def one_hot(rows, cols, col_of):
    w = np.zeros((rows, cols), np.uint16)
    for i in range(rows):
        w[i, col_of(i)] = 0x3F80  # BF16 1.0
    return w


def zero_layers(c):
    sh = synthetic.shapes(c)
    return [LayerWeights(**{n: np.zeros(sh[n], np.uint16) for n in synthetic.PROJECTIONS},
                         input_layernorm=np.ones(c.hidden_size, np.float32), q_norm=np.ones(c.head_dim, np.float32),
                         k_norm=np.ones(c.head_dim, np.float32),
                         post_attention_layernorm=np.ones(c.hidden_size, np.float32)) for _ in range(c.num_hidden_layers)]


def timestep_sinus(raw_t, shift):
    raw = rbs(f32(raw_t))
    sig = rbs(f32(1.0) / (f32(1.0) + exp32(-raw)))
    top = rbs(f32(shift) * sig)
    bottom = rbs(f32(1.0) + rbs(f32(shift - 1.0) * sig))
    t = rbs(top / bottom)
    sinus = np.empty(256, np.float32)
    ln = np.float32(math.log(10000.0))
    for i in range(128):
        f = exp32(np.float32(np.float32(-ln * f32(i)) / f32(128.0)))
        sinus[i] = rbs(np.float32(math.cos(float(f32(t * f)))))
        sinus[128 + i] = rbs(np.float32(math.sin(float(f32(t * f)))))
    return sinus


def one_hot_nar(c, nw):
    """Zero NAR layers and one-hot vae2llm / time / llm2vae matrices: every
    layer leaves x unchanged and every DOT picks one value exactly."""
    H = c.hidden_size
    nw.layers = zero_layers(c)
    nw.vae2llm = one_hot(H, LATENT, lambda i: i % LATENT)
    nw.time_in = one_hot(H, 256, lambda i: i % 256)
    nw.time_out = one_hot(H, H, lambda i: i)
    nw.llm2vae = one_hot(LATENT, H, lambda j: (3 * j) % H)
    return nw


def closed_velocity(c, nw, state, raw_t):
    """The velocity of one_hot_nar's model stated directly from the
    reference's lines (src/model.rs:611-698): x0 = rb(rb(rb(pad + rb(b)) +
    time) + pe) per padded row, then llm2vae(final_norm(x0[1 .. n-1]))."""
    H, frames = c.hidden_size, state.shape[0]
    n = frames + 2
    pad = np.zeros((n, LATENT), np.float32)
    pad[1:n - 1] = state
    b = lambda v: rb(v.astype(np.float32))  # noqa: E731
    x = np.empty((n, H), np.float32)
    for i in range(H):
        x[:, i] = rb(pad[:, i % LATENT] + b(nw.vae2llm_bias)[i])
    sinus = timestep_sinus(raw_t, nw.timestep_shift)
    t0 = rb(sinus[np.arange(H) % 256] + b(nw.time_in_bias))
    t0 = rb(t0 / (f32(1.0) + np.array([exp32(-v) for v in t0], np.float32)))
    time = rb(t0 + b(nw.time_out_bias))
    pe = f_of(nw.latent_pos)
    for r in range(n):
        x[r] = rb(rb(x[r] + time) + pe[min(r, nw.max_latent_frames - 1)])
    want = np.empty((frames, LATENT), np.float32)
    for f in range(frames):
        h = seq_norm(x[f + 1], np.ones(H, np.float32), c.rms_norm_eps)
        want[f] = rb(h[(3 * np.arange(LATENT)) % H] + b(nw.llm2vae_bias))
    return want


@pytest.mark.parametrize("shift", [1.0, 3.0])
def test_closed_form_without_layers(oracle_threads, shift):
    c = TINY
    ck = synthetic.checkpoint(c, seed=4)
    nw = one_hot_nar(c, synthetic.nar_weights(c, seed=4, max_latent_frames=16, timestep_shift=shift))
    om = O.Model(ck)
    nar = O.Nar(om, nw)
    oc, _ = om.prefill(synthetic.prompt(40, c.vocab_size, seed=2), 40)
    frames, raw_t = 20, 0.7
    rng = np.random.default_rng(1)
    state = rb(rng.standard_normal((frames, LATENT)).astype(np.float32))
    got = nar.velocity(state, oc, raw_t)
    want = closed_velocity(c, nw, state, raw_t)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _velocity_f64(c, ck, nw, keys_k, keys_v, cache_len, state, raw_t):
    """Model::velocity in float64 with the BF16 rounding points."""
    H, D, L = c.hidden_size, c.head_dim, LATENT
    hq, hk = c.num_attention_heads, c.num_key_value_heads
    r64 = lambda v: rb(np.asarray(v, np.float64).astype(np.float32)).astype(np.float64)  # noqa: E731
    W = lambda a: f_of(a).astype(np.float64)  # noqa: E731

    def norm(x, g):
        s = np.sum(x * x, axis=-1, keepdims=True)
        sc = r64(1.0 / np.sqrt(s / x.shape[-1] + c.rms_norm_eps))
        return r64(r64(x * sc) * g)

    def lin(w, x, bias=None):
        y = x @ W(w).T
        return r64(y + r64(bias)) if bias is not None else r64(y)

    frames = state.shape[0]
    n = frames + 2
    pad = np.zeros((n, L))
    pad[1:n - 1] = state
    x = lin(nw.vae2llm, pad, nw.vae2llm_bias)
    sinus = timestep_sinus(raw_t, nw.timestep_shift).astype(np.float64)
    t0 = lin(nw.time_in, sinus[None], nw.time_in_bias)
    t0 = r64(t0 / (1.0 + np.exp(-t0)))
    time = lin(nw.time_out, t0, nw.time_out_bias)[0]
    pe = W(nw.latent_pos)
    rows = np.minimum(np.arange(n), nw.max_latent_frames - 1)
    x = r64(r64(x + time) + pe[rows])
    half = D // 2
    freq = np.array([np.float32(1.0) / np.float32(np.float32(c.rope_theta) ** np.float32(np.float32(2 * i) / np.float32(D)))
                     for i in range(half)], np.float32)
    ang = (np.arange(cache_len, cache_len + n, dtype=np.float32)[:, None] * freq[None]).astype(np.float32)
    cos = rb(np.cos(ang.astype(np.float64)).astype(np.float32)).astype(np.float64)
    sin = rb(np.sin(ang.astype(np.float64)).astype(np.float32)).astype(np.float64)

    def rope(v):
        a, b_ = v[..., :half], v[..., half:]
        return np.concatenate([r64(r64(a * cos[:, None]) - r64(b_ * sin[:, None])),
                               r64(r64(b_ * cos[:, None]) + r64(a * sin[:, None]))], axis=-1)

    for l, P in enumerate(nw.layers):
        h = norm(x, P.input_layernorm)
        q = norm(lin(P.q_proj, h).reshape(n, hq, D), P.q_norm)
        k = norm(lin(P.k_proj, h).reshape(n, hk, D), P.k_norm)
        v = lin(P.v_proj, h).reshape(n, hk, D)
        q, k = rope(q), rope(k)
        K = np.concatenate([keys_k[l][:cache_len].reshape(cache_len, hk, D), k])
        V = np.concatenate([keys_v[l][:cache_len].reshape(cache_len, hk, D), v])
        att = np.empty((n, hq, D))
        for hh in range(hq):
            g = hh // (hq // hk)
            s = q[:, hh] @ K[:, g].T / math.sqrt(D)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            att[:, hh] = r64(p @ V[:, g])
        x = r64(x + lin(P.o_proj, att.reshape(n, hq * D)))
        h = norm(x, P.post_attention_layernorm)
        g_ = lin(P.gate_proj, h)
        g_ = r64(g_ / (1.0 + np.exp(-g_)))
        x = r64(x + lin(P.down_proj, r64(g_ * lin(P.up_proj, h))))
    return lin(nw.llm2vae, norm(x[1:n - 1], ck.final_norm), nw.llm2vae_bias)


@pytest.mark.parametrize("frames,max_frames", [(24, 64), (40, 16)])
def test_against_float64_restatement(oracle_threads, frames, max_frames):
    c = TINY
    ck = synthetic.checkpoint(c, seed=7, std=0.05)
    nw = synthetic.nar_weights(c, seed=7, std=0.05, max_latent_frames=max_frames, timestep_shift=2.0)
    om = O.Model(ck)
    nar = O.Nar(om, nw)
    oc, _ = om.prefill(synthetic.prompt(50, c.vocab_size, seed=3), 50)
    state = rb(np.random.default_rng(frames).standard_normal((frames, LATENT)).astype(np.float32))
    got = nar.velocity(state, oc, -0.4)
    kk, vv = oc.arrays()
    want = _velocity_f64(c, ck, nw, kk, vv, oc.length, state.astype(np.float64), -0.4)
    d = np.abs(got - want)
    assert d.max() <= 0.05 * want.std(), (d.max(), want.std())
    assert np.corrcoef(got.ravel(), want.ravel())[0, 1] > 0.999


def test_condition_end_limits_the_keys(oracle_threads):
    """nar_cond_end keeps the first keys only: a velocity against a cache
    whose later positions differ is unchanged below the condition end."""
    c = TINY
    ck = synthetic.checkpoint(c, seed=9)
    nw = synthetic.nar_weights(c, seed=9, max_latent_frames=64)
    om = O.Model(ck)
    nar = O.Nar(om, nw)
    ids = synthetic.prompt(60, c.vocab_size, seed=4)
    a, _ = om.prefill(ids, 60)
    b, _ = om.prefill(np.concatenate([ids[:30], synthetic.prompt(30, c.vocab_size, seed=5)]), 60)
    state = rb(np.random.default_rng(2).standard_normal((12, LATENT)).astype(np.float32))
    va, vb = nar.velocity(state, a, 0.1, 30), nar.velocity(state, b, 0.1, 30)
    assert np.array_equal(va.view(np.uint32), vb.view(np.uint32))
    assert not np.array_equal(nar.velocity(state, a, 0.1).view(np.uint32), nar.velocity(state, b, 0.1).view(np.uint32))


def test_normal_tensor_box_muller_within_ulps():
    """Every value of Generator::normal_tensor (src/sampling.rs:64-79) is the
    Box-Muller transform of the same MT19937 uniform_f32 draws (u_i gives the
    radius sqrt(-2 ln(1 - u_i)), u_(i+8) the angle 2 pi u, cos at i and sin at
    i + 8 within each block of 16), evaluated here in float64 from the f32
    angle: the oracle's f32 chain (logf, sqrtf, cosf / sinf and the product,
    each within an ulp or a half) stays within 3 f32 ulps of it (measured
    2.08).  A cos / sin swap, a wrong pairing or a wrong angle factor is off
    by far more."""
    n = 16 * 4000
    got = O.normal(11, n).astype(np.float64)
    g = synthetic.MT19937(11)
    u = (np.array([g.next_u32() & 0xFFFFFF for _ in range(n)], np.float64) / 16777216.0).reshape(-1, 16)
    r = np.sqrt(-2.0 * np.log(1.0 - u[:, :8]))
    th = (2.0 * math.pi * u[:, 8:]).astype(np.float32).astype(np.float64)
    want = np.concatenate([r * np.cos(th), r * np.sin(th)], axis=1).reshape(-1)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    worst = float(np.max(np.abs(got - want) / ulp))
    print(f"normal_tensor: max {worst:.2f} ulp from float64 Box-Muller")
    assert worst <= 3.0


def test_normal_tensor_pairs():
    """Generator::normal_tensor (src/sampling.rs:64-79): in each block of 16
    the pair (i, i + 8) shares the radius, x^2 + y^2 = -2 ln(1 - u_i) for the
    i-th uniform_f32 draw of MT19937(seed), and the values are N(0, 1)."""
    n = 16 * 4000
    v = O.normal(11, n).astype(np.float64)
    g = synthetic.MT19937(11)
    u = np.array([(g.next_u32() & 0xFFFFFF) / 16777216.0 for _ in range(n)])
    blk = v.reshape(-1, 16)
    ub = u.reshape(-1, 16)
    r2 = blk[:, :8] ** 2 + blk[:, 8:] ** 2
    want = -2.0 * np.log(1.0 - ub[:, :8])
    assert np.allclose(r2, want, rtol=2e-5, atol=1e-6)
    assert abs(v.mean()) < 0.02 and abs(v.std() - 1.0) < 0.02


MUSIC = Config(hidden_size=128, num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1, head_dim=64,
               intermediate_size=256, vocab_size=184704, max_position_embeddings=128, rms_norm_eps=1e-6,
               rope_theta=10000.0)


def test_synthesize_without_velocity_returns_the_noise(oracle_threads):
    """With llm2vae and its bias zero the velocity is +0, every midpoint step
    keeps the state, and the result is the rounded noise in chunk order."""
    ck = synthetic.checkpoint(MUSIC, seed=3)
    nw = synthetic.nar_weights(MUSIC, seed=3, max_latent_frames=64)
    nw.llm2vae = np.zeros_like(nw.llm2vae)
    nw.llm2vae_bias = np.zeros_like(nw.llm2vae_bias)
    nar = O.Nar(O.Model(ck), nw)
    codec = synthetic.prompt(90, 32768, seed=6)
    got = nar.synthesize(synthetic.prompt(20, 151643, seed=7), codec, 42, 2)
    want = rb(O.normal(42, 90 * 64)).reshape(90, 64)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_synthesize_rejects(oracle_threads):
    ck = synthetic.checkpoint(MUSIC, seed=3)
    nar = O.Nar(O.Model(ck), synthetic.nar_weights(MUSIC, seed=3, max_latent_frames=64))
    for prefix, codec, steps in (([1] * 20, [], 2), ([1] * 20, [32768], 2), ([1] * 20, [5], 0), ([1] * 124, [5], 2)):
        with pytest.raises(RuntimeError):
            nar.synthesize(prefix, codec, 1, steps)


def _logit(t):
    """logit (src/model.rs:777-779) in float64, clamped to [-20, 20]."""
    v = math.inf if t >= 1.0 else (-math.inf if t <= 0.0 else math.log(t / (1.0 - t)))
    return min(20.0, max(-20.0, v))


@pytest.mark.parametrize("steps", [1, 3])
def test_synthesize_midpoint_schedule_closed_form(oracle_threads, steps):
    """Model::synthesize's loop (src/model.rs:699-775) on a model whose
    velocity is known in closed form and depends on both the state and the
    time (one_hot_nar: the timestep embedding enters every row), restated
    here: the song's noise sliced at the chunk cuts (size = (min(24576,
    max positions) - prefix - 3) / 2), per step t = 1 - step / steps, the
    first velocity at logit(t), the midpoint state rb(s - rb(v1 * (dt / 2))),
    the second velocity at logit(t - 0.5 / steps), then rb(s - rb(v2 * dt)).
    A wrong midpoint, dt, time schedule or chunk cut changes the bits."""
    nw = one_hot_nar(MUSIC, synthetic.nar_weights(MUSIC, seed=5, max_latent_frames=64, timestep_shift=3.0))
    nar = O.Nar(O.Model(synthetic.checkpoint(MUSIC, seed=5)), nw)
    prefix = synthetic.prompt(20, 151643, seed=7)
    codec = synthetic.prompt(90, 32768, seed=8)
    got = nar.synthesize(prefix, codec, 42, steps)
    size = (min(24576, MUSIC.max_position_embeddings) - len(prefix) - 3) // 2
    assert 0 < size < len(codec), "the construction must cut the song into chunks"
    noise = O.normal(42, len(codec) * LATENT).reshape(-1, LATENT)
    dt = f32(1.0) / f32(steps)
    want = []
    for start in range(0, len(codec), size):
        state = rb(noise[start:start + size])
        for step in range(steps):
            t = 1.0 - step / steps
            v1 = closed_velocity(MUSIC, nw, state, _logit(t))
            mid = rb(state - rb(v1 * f32(dt / f32(2.0))))
            v2 = closed_velocity(MUSIC, nw, mid, _logit(t - 0.5 / steps))
            state = rb(state - rb(v2 * dt))
        want.append(state)
    want = np.concatenate(want)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
