// vae.hip -- the VAE decoder (src/vae.rs), FP32 on the device.
//
// The decoder (network, src/vae.rs:470-546) is a chain of 1-D convolutions
// over [time, channels] tensors: a 7-tap convolution from the latents, per
// upsampling block SnakeBeta, a transposed convolution (kernel 2s, stride s)
// and three residual units (SnakeBeta, 7-tap convolution with dilation 1, 3
// or 9, SnakeBeta, 1-tap convolution, plus the unit's input), then SnakeBeta,
// a 7-tap convolution to the audio channels and tanh.  Everything is FP32,
// as the reference's MPSGraph and eager paths are.
//
// One kernel computes every convolution: output rows o0 + ostride * m take
// the sum over taps q and input channels i of x[m * istride + off_q][i] *
// W_q[i][o] (+ bias, + the residual input).  A plain convolution is one
// launch (ostride 1, istride = stride, off_q = q * dilation - padding); a
// transposed one is one launch per output phase p < stride, whose rows
// p + stride * m see exactly the taps j = (p + padding) mod stride + q *
// stride at source rows m + (p + padding - j) / stride -- the polyphase form
// of the reference's per-phase packing (src/vae.rs:107-126).  Each 64 x 64
// output tile stages 16 input channels of its source rows and the taps'
// weights in LDS; each thread keeps a 4 x 4 block of outputs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "../../include/yue2_hip.h"
#include "runtime.h"
#include "vae.h"

using namespace y2;

namespace y2 {
namespace {

constexpr int kConvTile = 64, kConvChunk = 16, kConvTaps = 8, kConvSpan = 256;

struct ConvArgs {
    const float* x;
    int rows_in, cin;
    const float* w;  // tap slabs [k][cin][cout]
    const float* b;  // [cout] or null
    const float* res;  // added to the output (same layout) or null
    float* y;
    int cout, m_count, istride, ostride, o0, ntaps, off_min;
    int off[kConvTaps], slab[kConvTaps];
};

__global__ __launch_bounds__(256) void conv_kernel(const ConvArgs a) {
    __shared__ float xs[kConvSpan][kConvChunk];
    __shared__ __align__(16) float ws[kConvTaps][kConvChunk][kConvTile];
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    const int m0 = blockIdx.x * kConvTile, c0 = blockIdx.y * kConvTile;
    const int src_lo = m0 * a.istride + a.off_min;
    int off_max = a.off_min;
    for (int q = 0; q < a.ntaps; ++q) off_max = max(off_max, a.off[q]);
    const int span = (kConvTile - 1) * a.istride + off_max - a.off_min + 1;
    float acc[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] = 0.0f;
    for (int i0 = 0; i0 < a.cin; i0 += kConvChunk) {
        for (int u = tid; u < span * kConvChunk; u += 256) {
            const int r = u / kConvChunk, c = u % kConvChunk, src = src_lo + r, i = i0 + c;
            xs[r][c] = src >= 0 && src < a.rows_in && i < a.cin ? a.x[(size_t)src * a.cin + i] : 0.0f;
        }
        for (int u = tid; u < a.ntaps * kConvChunk * kConvTile; u += 256) {
            const int q = u / (kConvChunk * kConvTile), c = (u / kConvTile) % kConvChunk, o = u % kConvTile;
            const int i = i0 + c, oc = c0 + o;
            ws[q][c][o] = i < a.cin && oc < a.cout ? a.w[((size_t)a.slab[q] * a.cin + i) * a.cout + oc] : 0.0f;
        }
        __syncthreads();
        for (int q = 0; q < a.ntaps; ++q) {
            const int base = a.off[q] - a.off_min;
#pragma unroll 4
            for (int c = 0; c < kConvChunk; ++c) {
                const float4 wv = *reinterpret_cast<const float4*>(&ws[q][c][tx * 4]);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float xv = xs[(ty * 4 + r) * a.istride + base][c];
                    acc[r][0] = __builtin_fmaf(xv, wv.x, acc[r][0]);
                    acc[r][1] = __builtin_fmaf(xv, wv.y, acc[r][1]);
                    acc[r][2] = __builtin_fmaf(xv, wv.z, acc[r][2]);
                    acc[r][3] = __builtin_fmaf(xv, wv.w, acc[r][3]);
                }
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int m = m0 + ty * 4 + r;
        if (m >= a.m_count) continue;
        const size_t row = (size_t)(a.o0 + a.ostride * m) * a.cout;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int o = c0 + tx * 4 + c;
            if (o >= a.cout) continue;
            float v = acc[r][c] + (a.b ? a.b[o] : 0.0f);  // Conv::apply: the product, then the bias
            if (a.res) v = v + a.res[row + o];           // Op::Residual: h + x
            a.y[row + o] = v;
        }
    }
}

// Activation::apply (src/vae.rs:282-320), out of place.
__global__ __launch_bounds__(256) void activation_kernel(const float* x, float* y, size_t n, int c, int kind,
                                                         const float* alpha, const float* inv_beta) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float v = x[i];
        float o;
        if (kind == VAE_SNAKE) {
            const int ch = (int)(i % (size_t)c);
            const float s = sinf(v * alpha[ch]);
            o = v + inv_beta[ch] * (s * s);
        } else if (kind == VAE_ELU) {
            o = v < 0.0f ? expf(v) - 1.0f : v;
        } else {
            o = tanhf(v);
        }
        y[i] = o;
    }
}

__global__ __launch_bounds__(256) void add_kernel(float* y, const float* x, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) y[i] = y[i] + x[i];
}

int conv_length(const VaeOpHost& op, int n) {
    if (op.kind == VAE_CONVT) return (n - 1) * op.stride + op.dilation * (op.kernel - 1) + 1 - 2 * op.padding;
    return (n + 2 * op.padding - op.dilation * (op.kernel - 1) - 1) / op.stride + 1;
}

hipError_t launch_conv(hipStream_t s, ConvArgs a) {
    if (a.m_count <= 0) return hipSuccess;
    if (a.ntaps == 0) a.off[0] = 0;  // no tap: the rows get the bias (and the residual) only
    a.off_min = a.off[0];
    int off_max = a.off[0];
    for (int q = 1; q < a.ntaps; ++q) {
        a.off_min = std::min(a.off_min, a.off[q]);
        off_max = std::max(off_max, a.off[q]);
    }
    if (a.ntaps < 0 || a.ntaps > kConvTaps || (kConvTile - 1) * a.istride + off_max - a.off_min + 1 > kConvSpan)
        return hipErrorInvalidValue;
    const dim3 grid((a.m_count + kConvTile - 1) / kConvTile, (a.cout + kConvTile - 1) / kConvTile);
    conv_kernel<<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

// One convolution (plain or transposed) of x [n, cin] into y [length, cout]
// with device tap slabs w [k][cin][cout].
hipError_t run_conv(hipStream_t s, const VaeOpHost& op, const float* w, const float* b, const float* x, int n,
                    float* y, const float* res) {
    const int len = conv_length(op, n);
    if (op.kind == VAE_CONV) {
        if (op.kernel > kConvTaps) return hipErrorInvalidValue;
        ConvArgs a{x, n, op.cin, w, b, res, y, op.cout, len, op.stride, 1, 0, op.kernel};
        for (int q = 0; q < op.kernel; ++q) {
            a.off[q] = q * op.dilation - op.padding;
            a.slab[q] = q;
        }
        return launch_conv(s, a);
    }
    if (op.dilation != 1) return hipErrorInvalidValue;
    for (int ph = 0; ph < op.stride; ++ph) {
        ConvArgs a{x, n, op.cin, w, b, res, y, op.cout, (len - ph + op.stride - 1) / op.stride, 1, op.stride, ph, 0};
        for (int j = (ph + op.padding) % op.stride; j < op.kernel; j += op.stride) {
            if (a.ntaps == kConvTaps) return hipErrorInvalidValue;
            a.off[a.ntaps] = (ph + op.padding - j) / op.stride;  // exact: j = ph + padding (mod stride)
            a.slab[a.ntaps] = j;
            ++a.ntaps;
        }
        if (hipError_t e = launch_conv(s, a); e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Tap slabs [k][cin][cout] from the checkpoint layout ([out, in, k] or, for
// a transposed convolution, [in, out, k]).
std::vector<float> tap_slabs(const VaeOpHost& op) {
    std::vector<float> t((size_t)op.kernel * op.cin * op.cout);
    for (int o = 0; o < op.cout; ++o)
        for (int i = 0; i < op.cin; ++i)
            for (int j = 0; j < op.kernel; ++j) {
                const size_t src = op.kind == VAE_CONVT ? ((size_t)i * op.cout + o) * op.kernel + j
                                                        : ((size_t)o * op.cin + i) * op.kernel + j;
                t[((size_t)j * op.cin + i) * op.cout + o] = op.w[src];
            }
    return t;
}

}  // namespace
}  // namespace y2

struct Yue2Vae {
    y2::VaeHost host;
    std::vector<float*> w, b, a, ib;  // per op, device
    void* block = nullptr;
    hipStream_t stream = nullptr;
};

extern "C" void yue2_hip_vae_free(Yue2Vae* v) {
    if (!v) return;
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (v->stream) (void)hipStreamSynchronize(v->stream);
    if (v->block) (void)hipFree(v->block);
    if (v->stream) (void)hipStreamDestroy(v->stream);
    delete v;
}

extern "C" Yue2Vae* yue2_hip_vae_open(const char* dir) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!device_ready()) {
        fail(YUE2_ERR_DEVICE, "no usable gfx950 device");
        return nullptr;
    }
    auto* v = new Yue2Vae;
    if (vae_read(dir, &v->host) != YUE2_OK) {
        delete v;
        return nullptr;
    }
    // one allocation for every operation's parameters
    size_t total = 0;
    auto take = [&](size_t n) {
        const size_t o = total;
        total += (n * sizeof(float) + 255) / 256 * 256;
        return o;
    };
    const size_t nops = v->host.ops.size();
    std::vector<size_t> ow(nops), ob(nops), oa(nops), oi(nops);
    for (size_t k = 0; k < nops; ++k) {
        const VaeOpHost& op = v->host.ops[k];
        ow[k] = take(op.w.size());
        ob[k] = take(op.b.size());
        oa[k] = take(op.a.size());
        oi[k] = take(op.ib.size());
    }
    hipError_t e = hipStreamCreateWithFlags(&v->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&v->block, std::max<size_t>(total, 256));
    if (e != hipSuccess) {
        hip_fail(e, "VAE weights");
        yue2_hip_vae_free(v);
        return nullptr;
    }
    char* base = static_cast<char*>(v->block);
    v->w.assign(nops, nullptr);
    v->b.assign(nops, nullptr);
    v->a.assign(nops, nullptr);
    v->ib.assign(nops, nullptr);
    for (size_t k = 0; k < nops && e == hipSuccess; ++k) {
        const VaeOpHost& op = v->host.ops[k];
        auto up = [&](const std::vector<float>& src, size_t off, float** dst) {
            if (src.empty() || e != hipSuccess) return;
            *dst = reinterpret_cast<float*>(base + off);
            e = hipMemcpy(*dst, src.data(), src.size() * sizeof(float), hipMemcpyHostToDevice);
        };
        if (op.kind == VAE_CONV || op.kind == VAE_CONVT) up(tap_slabs(op), ow[k], &v->w[k]);
        up(op.b, ob[k], &v->b[k]);
        up(op.a, oa[k], &v->a[k]);
        up(op.ib, oi[k], &v->ib[k]);
    }
    if (e != hipSuccess) {
        hip_fail(e, "VAE weight upload");
        yue2_hip_vae_free(v);
        return nullptr;
    }
    return v;
}

extern "C" int32_t yue2_hip_vae_info(const Yue2Vae* v, int32_t* info) {
    if (!v || !info) return fail(YUE2_ERR_ARG, "null VAE or output");
    const VaeHost& h = v->host;
    const int32_t vals[6] = {h.sample_rate, h.latent_dim, h.audio_channels, h.ratio, h.core_frames, h.halo_frames};
    std::copy(vals, vals + 6, info);
    return YUE2_OK;
}

extern "C" int64_t yue2_hip_vae_output_length(const Yue2Vae* v, int32_t frames) {
    if (!v) return fail(YUE2_ERR_ARG, "null VAE");
    if (frames <= 0) return fail(YUE2_ERR_ARG, "Empty VAE latent");
    int64_t n = frames;
    for (const VaeOpHost& op : v->host.ops)
        if (op.kind == VAE_CONV || op.kind == VAE_CONVT) n = conv_length(op, (int)n);
    return n;
}

// Vae::required_halo (src/vae.rs:676-681) from Op::support (:410-425): the
// input span each output span needs, walked back through the decoder.
extern "C" int32_t yue2_hip_vae_required_halo(const Yue2Vae* v, int32_t core) {
    if (!v || core <= 0) return fail(YUE2_ERR_ARG, "null VAE or empty core");
    auto div_ceil = [](int64_t a, int64_t b) { return -((-a) >= 0 ? (-a) / b : -(((a) + b - 1) / b)); };
    auto floor_div = [](int64_t a, int64_t b) { return a >= 0 ? a / b : -((-a + b - 1) / b); };
    auto support = [&](const VaeOpHost& op, int64_t lo, int64_t hi, int64_t* l, int64_t* h) {
        const int64_t s = op.stride, p = op.padding, d = op.dilation, k = op.kernel;
        if (op.kind == VAE_CONVT) {
            *l = div_ceil(lo + p - d * (k - 1), s);
            *h = floor_div(hi + p, s);
        } else {
            *l = lo * s - p;
            *h = hi * s - p + d * (k - 1);
        }
    };
    const auto& ops = v->host.ops;
    int64_t lo = 0, hi = (int64_t)core * v->host.ratio - 1;
    // walk back; a residual unit's span is its body's widened by its own
    std::vector<std::pair<int64_t, int64_t>> outer;
    for (int k = (int)ops.size() - 1; k >= 0; --k) {
        const VaeOpHost& op = ops[k];
        if (op.kind == VAE_RES_END) {
            outer.emplace_back(lo, hi);
        } else if (op.kind == VAE_RES_BEGIN) {
            lo = std::min(lo, outer.back().first);
            hi = std::max(hi, outer.back().second);
            outer.pop_back();
        } else if (op.kind == VAE_CONV || op.kind == VAE_CONVT) {
            int64_t l, h;
            support(op, lo, hi, &l, &h);
            lo = l;
            hi = h;
        }
    }
    return (int32_t)std::max<int64_t>({0, -lo, hi - core + 1});
}

namespace {

// Vae::decode's network on the device (src/vae.rs:688-727): z [frames,
// latent] -> out [length, audio channels].
int vae_decode(Yue2Vae* v, const float* z, int frames, float* out) {
    const VaeHost& h = v->host;
    if (!z || !out || frames <= 0) return fail(YUE2_ERR_ARG, "Expected finite nonempty [frames,64] latents");
    for (size_t i = 0; i < (size_t)frames * h.latent_dim; ++i)
        if (!std::isfinite(z[i])) return fail(YUE2_ERR_ARG, "Expected finite nonempty [frames,64] latents");
    // the largest activation of the chain
    size_t most = (size_t)frames * h.latent_dim;
    int n = frames, c = h.latent_dim;
    for (const VaeOpHost& op : h.ops)
        if (op.kind == VAE_CONV || op.kind == VAE_CONVT) {
            n = conv_length(op, n);
            c = op.cout;
            if (n <= 0) return fail(YUE2_ERR_ARG, "VAE latent too short");
            most = std::max(most, (size_t)n * c);
        }
    float* buf[3] = {nullptr, nullptr, nullptr};
    void* block = nullptr;
    const size_t stride = (most * sizeof(float) + 255) / 256 * 256;
    hipError_t e = hipMalloc(&block, 3 * stride);
    if (e != hipSuccess) return hip_fail(e, "VAE activations");
    for (int i = 0; i < 3; ++i) buf[i] = reinterpret_cast<float*>(static_cast<char*>(block) + i * stride);
    hipStream_t s = v->stream;
    int cur = 0, res = -1;
    n = frames;
    c = h.latent_dim;
    auto free_buf = [&]() {
        for (int i = 0; i < 3; ++i)
            if (i != cur && i != res) return i;
        return -1;
    };
    e = hipMemcpyAsync(buf[0], z, sizeof(float) * (size_t)frames * c, hipMemcpyHostToDevice, s);
    int rc = e == hipSuccess ? YUE2_OK : hip_fail(e, "VAE input");
    const size_t nops = h.ops.size();
    for (size_t k = 0; k < nops && rc == YUE2_OK; ++k) {
        const VaeOpHost& op = h.ops[k];
        const int dst = free_buf();
        if (op.kind == VAE_CONV || op.kind == VAE_CONVT) {
            // the unit's residual joins in this convolution's epilogue when it ends the unit
            const bool join = k + 1 < nops && h.ops[k + 1].kind == VAE_RES_END && res >= 0;
            e = run_conv(s, op, v->w[k], v->b[k], buf[cur], n, buf[dst], join ? buf[res] : nullptr);
            if (e != hipSuccess) {
                rc = hip_fail(e, "VAE convolution");
                break;
            }
            n = conv_length(op, n);
            c = op.cout;
            cur = dst;
            if (join) {
                res = -1;
                ++k;  // the RES_END
            }
        } else if (op.kind == VAE_SNAKE || op.kind == VAE_ELU || op.kind == VAE_TANH) {
            const size_t cnt = (size_t)n * c;
            activation_kernel<<<(unsigned)std::min<size_t>((cnt + 255) / 256, 65536), 256, 0, s>>>(
                buf[cur], buf[dst], cnt, c, op.kind, v->a[k], v->ib[k]);
            cur = dst;
        } else if (op.kind == VAE_RES_BEGIN) {
            res = cur;
        } else if (op.kind == VAE_RES_END) {
            const size_t cnt = (size_t)n * c;
            add_kernel<<<(unsigned)std::min<size_t>((cnt + 255) / 256, 65536), 256, 0, s>>>(buf[cur], buf[res], cnt);
            res = -1;
        }
        if ((e = hipGetLastError()) != hipSuccess) rc = hip_fail(e, "VAE operation");
    }
    if (rc == YUE2_OK) {
        e = hipMemcpyAsync(out, buf[cur], sizeof(float) * (size_t)n * c, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) rc = hip_fail(e, "VAE output");
    }
    (void)hipStreamSynchronize(s);
    (void)hipFree(block);
    if (rc == YUE2_OK)
        for (size_t i = 0; i < (size_t)n * c; ++i)
            if (!std::isfinite(out[i])) return fail(YUE2_ERR_LOGITS, "VAE produced nonfinite audio");
    return rc;
}

}  // namespace

extern "C" int32_t yue2_hip_vae_decode(Yue2Vae* v, const float* z, int32_t frames, float* out) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!v) return fail(YUE2_ERR_ARG, "null VAE");
    return vae_decode(v, z, frames, out);
}

// Vae::decode_tiled (src/vae.rs:729-762).
extern "C" int32_t yue2_hip_vae_decode_tiled(Yue2Vae* v, const float* z, int32_t frames, int32_t core,
                                             int32_t halo, float* out) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!v || !z || !out || frames <= 0) return fail(YUE2_ERR_ARG, "Expected finite nonempty [frames,64] latents");
    const VaeHost& h = v->host;
    if (core <= 0 || halo < yue2_hip_vae_required_halo(v, std::max(core, 1)))
        return fail(YUE2_ERR_ARG, "VAE halo must be at least " + std::to_string(yue2_hip_vae_required_halo(v, std::max(core, 1))));
    const int64_t length = yue2_hip_vae_output_length(v, frames);
    if (length <= 0) return (int32_t)length;
    const int ch = h.audio_channels;
    std::vector<float> tile;
    for (int start = 0; start < frames; start += core) {
        const int end = std::min(start + core, frames);
        const int left = std::max(0, start - halo), right = std::min(frames, end + halo);
        const int64_t tlen = yue2_hip_vae_output_length(v, right - left);
        tile.resize((size_t)tlen * ch);
        if (int rc = vae_decode(v, z + (size_t)left * h.latent_dim, right - left, tile.data())) return rc;
        const int64_t a = (int64_t)start * h.ratio, b = std::min<int64_t>((int64_t)end * h.ratio, length);
        const int64_t crop = (int64_t)(start - left) * h.ratio;
        if (crop + b - a > tlen) return fail(YUE2_ERR_ARG, "VAE tile did not cover output core");
        std::copy(tile.begin() + crop * ch, tile.begin() + (crop + b - a) * ch, out + a * ch);
    }
    return YUE2_OK;
}

// Diagnostics: one convolution through the device kernel (the reference's
// convolution known-answer cases, src/vae.rs:812-892): x [frames, cin], w in
// the checkpoint layout (no weight norm), bias [cout] or null.
extern "C" int32_t yue2_hip_selftest_conv(int32_t transpose, int32_t cin, int32_t cout, int32_t kernel, int32_t stride,
                                          int32_t padding, int32_t dilation, const float* x, int32_t frames,
                                          const float* w, const float* bias, float* out) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!x || !w || !out || cin < 1 || cout < 1 || kernel < 1 || stride < 1 || dilation < 1 || padding < 0 || frames < 1)
        return fail(YUE2_ERR_ARG, "bad convolution selftest");
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no usable gfx950 device");
    VaeOpHost op;
    op.kind = transpose ? VAE_CONVT : VAE_CONV;
    op.cin = cin;
    op.cout = cout;
    op.kernel = kernel;
    op.stride = stride;
    op.padding = padding;
    op.dilation = dilation;
    op.w.assign(w, w + (size_t)cin * cout * kernel);
    const int len = conv_length(op, frames);
    if (len <= 0) return fail(YUE2_ERR_ARG, "bad convolution selftest");
    const std::vector<float> slabs = tap_slabs(op);
    float *dx = nullptr, *dw = nullptr, *db = nullptr, *dy = nullptr;
    hipError_t e = hipMalloc(&dx, sizeof(float) * (size_t)frames * cin);
    if (e == hipSuccess) e = hipMalloc(&dw, sizeof(float) * slabs.size());
    if (e == hipSuccess) e = hipMalloc(&db, sizeof(float) * cout);
    if (e == hipSuccess) e = hipMalloc(&dy, sizeof(float) * (size_t)len * cout);
    if (e == hipSuccess) e = hipMemcpy(dx, x, sizeof(float) * (size_t)frames * cin, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dw, slabs.data(), sizeof(float) * slabs.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && bias) e = hipMemcpy(db, bias, sizeof(float) * cout, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = run_conv(nullptr, op, dw, bias ? db : nullptr, dx, frames, dy, nullptr);
    if (e == hipSuccess) e = hipMemcpy(out, dy, sizeof(float) * (size_t)len * cout, hipMemcpyDeviceToHost);
    (void)hipFree(dx);
    (void)hipFree(dw);
    (void)hipFree(db);
    (void)hipFree(dy);
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "convolution selftest");
}
