"""Synthetic VAE decoder checkpoints in the layout Vae::open reads
(src/vae.rs:635-669): config.json (model_type yue2_vae, decoder_config) and
model.safetensors with F32 weight-norm pairs, biases and SnakeBeta
parameters under the reference's tensor names (network, src/vae.rs:470-546;
residual, :427-466).  Also the same decoder as the oracle's operation list
(test infrastructure) and the tiling of Vae::decode_tiled (:729-762)."""
import numpy as np

from oracle import oracle as O
from yue2_rs_amd import synthetic


def synthetic_vae(seed=0, **kw):
    return synthetic.vae(seed, **kw)


def write_vae_dir(path, cfg, tensors):
    return synthetic.write_vae(path, cfg, tensors)


def oracle_ops(cfg, t):
    """The decoder of network(decoder = true) as y2o_vae operations."""
    d = cfg["decoder_config"]
    ch, mults, strides = d["channels"], [1] + d["c_mults"], d["strides"]
    snake = d.get("use_snake", False)
    ops = []

    def conv(name, cin, cout, k, s=1, p=0, dil=1, transpose=False, bias=True):
        ops.append((O.VAE_CONVT if transpose else O.VAE_CONV,
                    dict(cin=cin, cout=cout, kernel=k, stride=s, padding=p, dilation=dil),
                    dict(v=t[f"{name}.weight_v"], g=t[f"{name}.weight_g"],
                         b=t[f"{name}.bias"] if bias else None)))

    def act(name):
        if snake:
            ops.append((O.VAE_SNAKE, {}, dict(alpha=t[f"{name}.alpha"], beta=t[f"{name}.beta"])))
        else:
            ops.append((O.VAE_ELU, {}, {}))

    conv("decoder.layers.0", d["latent_dim"], ch * mults[-1], 7, p=3)
    index = 1
    for i in range(len(mults) - 1, 0, -1):
        cin, cout, s = ch * mults[i], ch * mults[i - 1], strides[i - 1]
        p = f"decoder.layers.{index}.layers"
        act(f"{p}.0")
        conv(f"{p}.1", cin, cout, 2 * s, s=s, p=(s + 1) // 2, transpose=True)
        for r, dil in ((2, 1), (3, 3), (4, 9)):
            ops.append((O.VAE_RES_BEGIN, {}, {}))
            act(f"{p}.{r}.layers.0")
            conv(f"{p}.{r}.layers.1", cout, cout, 7, p=3 * dil, dil=dil)
            act(f"{p}.{r}.layers.2")
            conv(f"{p}.{r}.layers.3", cout, cout, 1)
            ops.append((O.VAE_RES_END, {}, {}))
        index += 1
    act(f"decoder.layers.{index}")
    conv(f"decoder.layers.{index + 1}", ch, d["out_channels"], 7, p=3, bias=False)
    ops.append((O.VAE_TANH if d.get("final_tanh", True) else None, {}, {}))
    return O.VaeOps([o for o in ops if o[0] is not None])


def decode_tiled(decode, z, core, halo, ratio, length):
    """Vae::decode_tiled (src/vae.rs:729-762) over a decode function."""
    frames = z.shape[0]
    out = None
    for start in range(0, frames, core):
        end = min(start + core, frames)
        left, right = max(0, start - halo), min(frames, end + halo)
        tile = decode(z[left:right])
        if out is None:
            out = np.zeros((length, tile.shape[1]), np.float32)
        a, b = start * ratio, min(end * ratio, length)
        crop = (start - left) * ratio
        out[a:b] = tile[crop:crop + b - a]
    return out


def required_halo(cfg, core):
    """Vae::required_halo (src/vae.rs:676-681): the latent frames a tile
    needs on each side, from Op::support (:410-425) of the decoder."""
    d = cfg["decoder_config"]
    mults, strides = [1] + d["c_mults"], d["strides"]
    convs = [("c", 7, 1, 3, 1)]  # (kind, kernel, stride, padding, dilation) in network order
    for i in range(len(mults) - 1, 0, -1):
        s = strides[i - 1]
        convs.append(("t", 2 * s, s, (s + 1) // 2, 1))
        for dil in (1, 3, 9):
            convs.append(("r", dil))
    convs.append(("c", 7, 1, 3, 1))

    def div_ceil(a, b):
        return -((-a) // b)

    def conv_support(k, s, p, dil, t, low, high):
        if t:
            return div_ceil(low + p - dil * (k - 1), s), (high + p) // s
        return low * s - p, high * s - p + dil * (k - 1)

    low, high = 0, core * cfg["downsampling_ratio"] - 1
    for op in reversed(convs):
        if op[0] == "r":  # residual unit: conv k7 dilated then conv k1
            dil = op[1]
            a, b = conv_support(1, 1, 0, 1, False, low, high)
            a, b = conv_support(7, 1, 3 * dil, dil, False, a, b)
            low, high = min(a, low), max(b, high)
        else:
            _, k, s, p, dil = op
            low, high = conv_support(k, s, p, dil, op[0] == "t", low, high)
    return max(0, -low, high - core + 1)


def decode_f64(cfg, t, z):
    """The decoder in float64 (every product and sum in f64), an independent
    evaluation to measure FP32 paths against."""
    d = cfg["decoder_config"]
    ch, mults, strides = d["channels"], [1] + d["c_mults"], d["strides"]
    snake = d.get("use_snake", False)

    def conv(x, name, k, s=1, p=0, dil=1, tr=False, bias=True):
        v = t[f"{name}.weight_v"].astype(np.float64)
        g = t[f"{name}.weight_g"].astype(np.float64).reshape(-1, 1)
        r = v.reshape(v.shape[0], -1)
        w = (r * (g / np.sqrt((r * r).sum(1, keepdims=True)))).reshape(v.shape)
        n = x.shape[0]
        if tr:
            length = (n - 1) * s + dil * (k - 1) + 1 - 2 * p
            y = np.zeros((length, w.shape[1]))
            for j in range(k):
                rows = np.arange(n) * s + j * dil - p
                ok = (rows >= 0) & (rows < length)
                np.add.at(y, rows[ok], x[ok] @ w[:, :, j])
        else:
            length = (n + 2 * p - dil * (k - 1) - 1) // s + 1
            y = np.zeros((length, w.shape[0]))
            for j in range(k):
                src = np.arange(length) * s + j * dil - p
                ok = (src >= 0) & (src < n)
                y[ok] += x[src[ok]] @ w[:, :, j].T
        if bias:
            y += t[f"{name}.bias"].astype(np.float64)
        return y

    def act(x, name):
        if snake:
            a = np.exp(t[f"{name}.alpha"].astype(np.float64))
            b = np.exp(t[f"{name}.beta"].astype(np.float64))
            return x + 1.0 / (b + 1e-9) * np.sin(x * a) ** 2
        return np.where(x < 0, np.expm1(np.minimum(x, 0)), x)

    x = conv(np.asarray(z, np.float64), "decoder.layers.0", 7, p=3)
    index = 1
    for i in range(len(mults) - 1, 0, -1):
        s = strides[i - 1]
        p = f"decoder.layers.{index}.layers"
        x = conv(act(x, f"{p}.0"), f"{p}.1", 2 * s, s=s, p=(s + 1) // 2, tr=True)
        for r, dil in ((2, 1), (3, 3), (4, 9)):
            h = conv(act(x, f"{p}.{r}.layers.0"), f"{p}.{r}.layers.1", 7, p=3 * dil, dil=dil)
            x = conv(act(h, f"{p}.{r}.layers.2"), f"{p}.{r}.layers.3", 1) + x
        index += 1
    x = conv(act(x, f"decoder.layers.{index}"), f"decoder.layers.{index + 1}", 7, p=3, bias=False)
    return np.tanh(x) if d.get("final_tanh", True) else x


def conv_f64(transpose, x, w, bias, kernel, stride, padding, dilation):
    """One convolution in float64: x [frames, cin], w [cout, cin, k] (plain)
    or [cin, cout, k] (transposed), bias [cout] or None."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    n = x.shape[0]
    if transpose:
        length = (n - 1) * stride + dilation * (kernel - 1) + 1 - 2 * padding
        y = np.zeros((length, w.shape[1]))
        for j in range(kernel):
            rows = np.arange(n) * stride + j * dilation - padding
            ok = (rows >= 0) & (rows < length)
            np.add.at(y, rows[ok], x[ok] @ w[:, :, j])
    else:
        length = (n + 2 * padding - dilation * (kernel - 1) - 1) // stride + 1
        y = np.zeros((length, w.shape[0]))
        for j in range(kernel):
            src = np.arange(length) * stride + j * dilation - padding
            ok = (src >= 0) & (src < n)
            y[ok] += x[src[ok]] @ w[:, :, j].T
    if bias is not None:
        y += np.asarray(bias, np.float64)
    return y


# (transpose, cin, cout, kernel, stride, padding, dilation, frames): shapes
# that reach every branch of the device convolutions -- the matrix-core
# kernel with 16-byte and scalar input loads, several output-channel tiles,
# ten and twenty phases, phases without a tap and a strided plain convolution; the
# narrow kernel with several row tiles and a ragged channel chunk.
CONV_SHAPES = [
    (False, 20, 40, 7, 1, 9, 3, 300),
    (False, 6, 130, 7, 1, 3, 1, 200),
    (True, 24, 64, 20, 10, 5, 1, 40),
    (True, 16, 33, 2, 4, 0, 1, 50),
    (True, 8, 40, 40, 20, 10, 1, 12),
    (False, 8, 48, 4, 2, 1, 1, 300),
    (False, 130, 3, 7, 1, 27, 9, 600),
    (False, 64, 16, 7, 1, 3, 1, 100),
]


def conv_case(transpose, cin, cout, kernel, stride, padding, dilation, frames, seed=0):
    rng = np.random.default_rng(seed)
    x = (0.5 * rng.standard_normal((frames, cin))).astype(np.float32)
    w = (0.1 * rng.standard_normal((cin, cout, kernel) if transpose else (cout, cin, kernel))).astype(np.float32)
    b = (0.1 * rng.standard_normal(cout)).astype(np.float32)
    return x, w, b, conv_f64(transpose, x, w, b, kernel, stride, padding, dilation)
