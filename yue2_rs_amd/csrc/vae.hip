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
// Every convolution is a GEMM over output rows o0 + ostride * m: the sum
// over taps q and input channels i of x[m * istride + off_q][i] * W_q[i][o]
// (+ bias, + the residual input).  A plain convolution has one phase
// (ostride 1, istride = stride, off_q = q * dilation - padding); a
// transposed one has `stride` phases, launched together, whose rows p +
// stride * m see exactly the taps j = (p + padding) mod stride + q * stride
// at source rows m + (p + padding - j) / stride -- the polyphase form of the
// reference's per-phase packing (src/vae.rs:107-126).  The activation
// before a convolution (SnakeBeta or ELU) is applied while its input is
// staged, and a final tanh in the epilogue, so activations never make a
// round trip through HBM.
//
// conv_mfma_kernel: 128 x 128 output tiles, 4 waves of 2 x 2 FP32 MFMA
// blocks (v_mfma_f32_32x32x2_f32); per 8-channel chunk the source rows and
// every tap's weights are staged in LDS (52 KB for 7 taps: two workgroups
// per CU); step t of a chunk feeds lane half h channel 4h + t, so each lane
// reads its 4 channels with one 16-byte LDS load.  conv_narrow_kernel: outputs with at most 16 channels (the audio
// projection), one output row per thread on the vector ALUs.
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

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxTaps = 8, kMaxPhases = 32;  // ConvPlan stays under the 4 KB kernel-argument limit
constexpr int kMmaTile = 128;
constexpr int kChunk = 16, kNarrowRows = 256, kNarrowPad = 17;
constexpr size_t kMaxLds = 160 * 1024;
enum { ACT_NONE = 0, ACT_SNAKE = 1, ACT_ELU = 2 };

struct ConvPlan {
    const float* x;         // [rows_in][cin]
    const float* w;         // tap slabs in the kernel's layout
    const float* b;         // [cout] or null
    const float* res;       // [rows][cout] added to the output, or null
    float* y;               // [rows][cout]
    const float* alpha;     // SnakeBeta exp(alpha), 1 / (exp(beta) + 1e-9) per input channel
    const float* inv_beta;
    int rows_in, cin, cin_pad, cout, cout_pad, istride, ostride, tanh_out, span, ltaps;
    int m_count[kMaxPhases], o0[kMaxPhases], ntaps[kMaxPhases], off_min[kMaxPhases];
    int off[kMaxPhases][kMaxTaps], slab[kMaxPhases][kMaxTaps];
};

// Conv::apply's product, then the bias; Op::Residual's h + x; the final tanh.
__device__ __forceinline__ void conv_store(const ConvPlan& p, int m, int o, float acc) {
    const size_t at = (size_t)(p.o0[blockIdx.z] + p.ostride * m) * p.cout + o;
    float v = acc + (p.b ? p.b[o] : 0.0f);
    if (p.res) v = v + p.res[at];
    if (p.tanh_out) v = tanhf(v);
    p.y[at] = v;
}

// Rows [src_lo, src_lo + span) x channels [c0, c0 + 16) of the input,
// activated as Activation::apply does (src/vae.rs:282-320), into LDS rows
// of kNarrowPad floats; zero outside the input.  (Batching every thread's
// loads ahead of their use measured slower here: the extra registers halve
// the occupancy that hides this kernel's latency.)
template <int ACT>
__device__ __forceinline__ void stage_rows(const ConvPlan& p, float* X, int src_lo, int c0) {
    for (int u = threadIdx.x; u < p.span * 4; u += blockDim.x) {
        const int r = u >> 2, ch = c0 + 4 * (u & 3), src = src_lo + r;
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (src >= 0 && src < p.rows_in) {
            const float* row = p.x + (size_t)src * p.cin;
            if ((p.cin & 3) == 0) {
                if (ch < p.cin) {
                    const float4 t = *reinterpret_cast<const float4*>(row + ch);
                    v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (ch + e < p.cin) v[e] = row[ch + e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (ch + e < p.cin) {
                    if constexpr (ACT == ACT_SNAKE) {
                        const float t = sinf(v[e] * p.alpha[ch + e]);
                        v[e] = v[e] + p.inv_beta[ch + e] * (t * t);
                    } else if constexpr (ACT == ACT_ELU) {
                        v[e] = v[e] < 0.0f ? expf(v[e]) - 1.0f : v[e];
                    }
                }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) X[r * kNarrowPad + 4 * (u & 3) + e] = v[e];
    }
}

// Weight slabs [k][cin_pad / KC][cout_pad][KC]; x [rows][cin], y [rows][cout].
// Chunk ck + 1's rows and weights are loaded into registers while chunk
// ck's MFMAs run, then activated and written to LDS between two barriers.
// KC = 8 for up to 8 taps (52 KB of LDS for 7), KC = 32 for up to 2 (the
// 1-tap and the transposed convolutions).  NT > 0: exactly NT taps in every
// phase, so the (tap, group) steps unroll without branches; NT = 0: up to
// 8 taps, counted per phase.  VEC: cin % 4 == 0, 16-byte source loads.
template <int ACT, int NT, int KC, bool VEC>
__global__ __launch_bounds__(256, 2) void conv_mfma_kernel(const ConvPlan p) {
    constexpr int MAXT = NT > 0 ? NT : kMaxTaps;
    constexpr int PITCH = KC + 4, G = KC / 4;  // LDS row pitch (floats), float4 groups per row
    constexpr int XS = KC == 8 ? 3 : NT == 1 ? 4 : 5;  // float4 slots per thread for the source rows
    constexpr int WE = KC / 8;                 // float4 slots per thread per tap; MFMA groups per tap
    extern __shared__ __align__(16) float lds[];
    float* W = lds;                                    // [ltaps][128][PITCH]
    float* X = lds + p.ltaps * kMmaTile * PITCH;       // [span][PITCH]
    const int ph = blockIdx.z, m_count = p.m_count[ph];
    const int m0 = blockIdx.x * kMmaTile, n0 = blockIdx.y * kMmaTile;
    if (m0 >= m_count) return;
    const int ntaps = NT > 0 ? NT : p.ntaps[ph];
    const int src_lo = m0 * p.istride + p.off_min[ph], nchunks = p.cin_pad / KC;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
    const int wm = wave >> 1, wn = wave & 1;
    int offs[MAXT], slabs[MAXT];
#pragma unroll
    for (int q = 0; q < MAXT; ++q) {
        offs[q] = p.off[ph][q] - p.off_min[ph];
        slabs[q] = p.slab[ph][q];
    }
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // source-row slot s: item u = tid + 256 s (row u / G, channels 4 (u % G) ..); weight slot q WE + e:
    // item tid + 256 e of tap q (output row n0 + item / G, channels 4 (item % G) ..)
    f32x4 xr[XS], wr[MAXT * WE], ar = {}, br = {};
    for (int ck = -1; ck < nchunks; ++ck) {
        const int nx = ck + 1;
        if (nx < nchunks) {
            // unconditional loads from clamped addresses (a conditional load would make the
            // compiler wait for every load where the branches join); the store zeroes what lies
            // outside the input
            const int c0 = nx * KC, ch = c0 + 4 * (tid % G);
#pragma unroll
            for (int s = 0; s < XS; ++s) {
                const int u = tid + 256 * s, src = min(max(src_lo + u / G, 0), p.rows_in - 1);
                const float* row = p.x + (size_t)src * p.cin;
                if constexpr (VEC) {
                    xr[s] = *reinterpret_cast<const f32x4*>(row + min(ch, p.cin - 4));
                } else {
                    xr[s] = f32x4{row[min(ch, p.cin - 1)], row[min(ch + 1, p.cin - 1)], row[min(ch + 2, p.cin - 1)],
                                  row[min(ch + 3, p.cin - 1)]};
                }
            }
            if constexpr (ACT == ACT_SNAKE) {
                if constexpr (VEC) {
                    ar = *reinterpret_cast<const f32x4*>(p.alpha + min(ch, p.cin - 4));
                    br = *reinterpret_cast<const f32x4*>(p.inv_beta + min(ch, p.cin - 4));
                } else {
                    const int l = p.cin - 1;
                    ar = f32x4{p.alpha[min(ch, l)], p.alpha[min(ch + 1, l)], p.alpha[min(ch + 2, l)],
                               p.alpha[min(ch + 3, l)]};
                    br = f32x4{p.inv_beta[min(ch, l)], p.inv_beta[min(ch + 1, l)], p.inv_beta[min(ch + 2, l)],
                               p.inv_beta[min(ch + 3, l)]};
                }
            }
#pragma unroll
            for (int q = 0; q < MAXT; ++q)
                if (NT > 0 || q < ntaps)
#pragma unroll
                    for (int e = 0; e < WE; ++e) {
                        const int it = tid + 256 * e;
                        wr[q * WE + e] = *reinterpret_cast<const f32x4*>(
                            p.w + (((size_t)slabs[q] * nchunks + nx) * p.cout_pad + n0 + it / G) * KC + 4 * (it % G));
                    }
        }
        if (ck >= 0) {
            // step (q, g): lane half h supplies channels (KC / 2) h + 4 g .. + 3 of the chunk, to A and B alike
#pragma unroll
            for (int k = 0; k < MAXT * WE; ++k) {
                const int q = k / WE, g = k % WE;
                if (NT > 0 || q < ntaps) {
                    f32x4 a[2], b[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        a[i] = *reinterpret_cast<const f32x4*>(
                            X + ((wm * 64 + i * 32 + l32) * p.istride + offs[q]) * PITCH + (KC / 2) * h + 4 * g);
                        b[i] = *reinterpret_cast<const f32x4*>(W + (q * kMmaTile + wn * 64 + i * 32 + l32) * PITCH +
                                                                (KC / 2) * h + 4 * g);
                    }
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].x, b[j].x, acc[i][j], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].y, b[j].y, acc[i][j], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].z, b[j].z, acc[i][j], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].w, b[j].w, acc[i][j], 0, 0, 0);
                }
            }
        }
        __syncthreads();
        if (nx < nchunks) {
            const int c0 = nx * KC, ch = c0 + 4 * (tid % G);
#pragma unroll
            for (int s = 0; s < XS; ++s) {
                const int u = tid + 256 * s, src = src_lo + u / G;
                if (u < p.span * G) {
                    f32x4 v = xr[s];
                    if constexpr (ACT == ACT_SNAKE) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float t = sinf(v[e] * ar[e]);
                            v[e] = v[e] + br[e] * (t * t);
                        }
                    } else if constexpr (ACT == ACT_ELU) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = v[e] < 0.0f ? expf(v[e]) - 1.0f : v[e];
                    }
                    const bool row_ok = src >= 0 && src < p.rows_in;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (!row_ok || ch + e >= p.cin) v[e] = 0.0f;
                    *reinterpret_cast<f32x4*>(X + (u / G) * PITCH + 4 * (u % G)) = v;
                }
            }
#pragma unroll
            for (int q = 0; q < MAXT; ++q)
                if (NT > 0 || q < ntaps)
#pragma unroll
                    for (int e = 0; e < WE; ++e) {
                        const int it = tid + 256 * e;
                        *reinterpret_cast<f32x4*>(W + (q * kMmaTile + it / G) * PITCH + 4 * (it % G)) =
                            wr[q * WE + e];
                    }
            __syncthreads();
        }
    }
    // C layout of the 32 x 32 blocks: register r of lane l is row 8 (r / 4) +
    // 4 (l / 32) + r % 4, column l % 32.  A block's 16 residual values are
    // requested together (clamped addresses), then added and stored.
    const int ostride = p.ostride, o0 = p.o0[ph], cout = p.cout;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int o = n0 + wn * 64 + j * 32 + l32, oc = min(o, cout - 1);
            const float bias = p.b ? p.b[oc] : 0.0f;
            float rv[16];
            if (p.res) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int m = min(m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3), m_count - 1);
                    rv[r] = p.res[(size_t)(o0 + ostride * m) * cout + oc];
                }
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (m < m_count && o < cout) {
                    float v = acc[i][j][r] + bias;  // Conv::apply: the product, then the bias
                    if (p.res) v = v + rv[r];       // Op::Residual: h + x
                    if (p.tanh_out) v = tanhf(v);
                    p.y[(size_t)(o0 + ostride * m) * cout + o] = v;
                }
            }
        }
}

// Weight slabs [k][cin_pad][CO]; one output row per thread.
template <int CO, int ACT>
__global__ __launch_bounds__(256) void conv_narrow_kernel(const ConvPlan p) {
    extern __shared__ __align__(16) float lds[];
    float* W = lds;                                  // [ltaps][16][CO]
    float* X = lds + p.ltaps * kChunk * CO;          // [span][kNarrowPad]
    const int ph = blockIdx.z, m_count = p.m_count[ph], m0 = blockIdx.x * kNarrowRows;
    if (m0 >= m_count) return;
    const int ntaps = p.ntaps[ph], src_lo = m0 * p.istride + p.off_min[ph], tid = threadIdx.x;
    float acc[CO];
#pragma unroll
    for (int o = 0; o < CO; ++o) acc[o] = 0.0f;
    for (int c0 = 0; c0 < p.cin_pad; c0 += kChunk) {
        stage_rows<ACT>(p, X, src_lo, c0);
        for (int u = tid; u < ntaps * kChunk * CO; u += 256) {
            const int q = u / (kChunk * CO), rest = u % (kChunk * CO);
            W[u] = p.w[((size_t)p.slab[ph][q] * p.cin_pad + c0) * CO + rest];
        }
        __syncthreads();
        for (int q = 0; q < ntaps; ++q) {
            const float* xr = X + (tid * p.istride + p.off[ph][q] - p.off_min[ph]) * kNarrowPad;
#pragma unroll 4
            for (int c = 0; c < kChunk; ++c) {
                const float xv = xr[c];
#pragma unroll
                for (int o = 0; o < CO; ++o) acc[o] = __builtin_fmaf(xv, W[(q * kChunk + c) * CO + o], acc[o]);
            }
        }
        __syncthreads();
    }
    const int m = m0 + tid;
    if (m < m_count)
#pragma unroll
        for (int o = 0; o < CO; ++o)
            if (o < p.cout) conv_store(p, m, o, acc[o]);
}

// An activation that no convolution follows, out of place.
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

// The device form of one convolution: which kernel, its channel chunk and
// padded widths.
struct ConvShape {
    bool mfma = false;
    int chunk = kChunk, cin_pad = 0, cout_pad = 0;
};

// Source rows a 128-row output tile reads: at most 160 (32-channel chunks)
// or 384 (8-channel chunks), from the register slots of the kernel.
int mfma_span(const VaeOpHost& op) {
    if (op.kind == VAE_CONVT) return kMmaTile - 1 + (op.kernel - 1) / op.stride + 1;
    return (kMmaTile - 1) * op.stride + op.dilation * (op.kernel - 1) + 1;
}

ConvShape conv_shape(const VaeOpHost& op) {
    ConvShape c;
    c.mfma = op.cout > 16;
    const int taps = op.kind == VAE_CONVT ? (op.kernel + op.stride - 1) / op.stride : op.kernel;
    const bool uniform = op.kind == VAE_CONV || op.kernel % op.stride == 0;  // every phase has `taps` taps
    c.chunk = !c.mfma ? kChunk : taps <= 2 && uniform && op.cin % 4 == 0 && mfma_span(op) <= 160 ? 32 : 8;
    c.cin_pad = (op.cin + c.chunk - 1) / c.chunk * c.chunk;
    c.cout_pad = c.mfma ? (op.cout + kMmaTile - 1) / kMmaTile * kMmaTile : op.cout <= 2 ? 2 : op.cout <= 4 ? 4
                                                                         : op.cout <= 8 ? 8 : 16;
    return c;
}

// Tap slabs in the kernel's layout from the checkpoint layout ([out, in, k]
// or, for a transposed convolution, [in, out, k]); zero padding.
std::vector<float> conv_slabs(const VaeOpHost& op, const ConvShape& c) {
    std::vector<float> t((size_t)op.kernel * c.cin_pad * c.cout_pad, 0.0f);
    const int nchunks = c.cin_pad / c.chunk;
    for (int o = 0; o < op.cout; ++o)
        for (int i = 0; i < op.cin; ++i)
            for (int j = 0; j < op.kernel; ++j) {
                const size_t src = op.kind == VAE_CONVT ? ((size_t)i * op.cout + o) * op.kernel + j
                                                        : ((size_t)o * op.cin + i) * op.kernel + j;
                const size_t dst = c.mfma ? ((((size_t)j * nchunks + i / c.chunk) * c.cout_pad + o) * c.chunk +
                                             i % c.chunk)
                                          : (((size_t)j * c.cin_pad + i) * c.cout_pad + o);
                t[dst] = op.w[src];
            }
    return t;
}

template <typename K>
hipError_t launch(K kernel, dim3 grid, size_t lds, hipStream_t s, const ConvPlan& p) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)lds);
    kernel<<<grid, 256, lds, s>>>(p);
    return hipGetLastError();
}

// One convolution (plain or transposed) of x [n, cin] into y [length, cout]:
// act is the activation applied to x on the way in (ACT_*, SnakeBeta's
// folded parameters), res the residual added to the output, tanh_out the
// final tanh.
hipError_t run_conv(hipStream_t s, const VaeOpHost& op, const ConvShape& c, const float* w, const float* b,
                    const float* x, int n, float* y, const float* res, int act, const float* alpha,
                    const float* inv_beta, bool tanh_out) {
    const int len = conv_length(op, n);
    if (len <= 0) return hipErrorInvalidValue;
    ConvPlan p{};
    p.x = x, p.w = w, p.b = b, p.res = res, p.y = y, p.alpha = alpha, p.inv_beta = inv_beta;
    p.rows_in = n, p.cin = op.cin, p.cin_pad = c.cin_pad, p.cout = op.cout, p.cout_pad = c.cout_pad;
    p.tanh_out = tanh_out ? 1 : 0;
    int phases = 1;
    if (op.kind == VAE_CONV) {
        if (op.kernel > kMaxTaps) return hipErrorInvalidValue;
        p.istride = op.stride, p.ostride = 1, p.m_count[0] = len, p.ntaps[0] = op.kernel;
        for (int q = 0; q < op.kernel; ++q) {
            p.off[0][q] = q * op.dilation - op.padding;
            p.slab[0][q] = q;
        }
    } else {
        if (op.dilation != 1 || op.stride > kMaxPhases) return hipErrorInvalidValue;
        phases = op.stride, p.istride = 1, p.ostride = op.stride;
        for (int ph = 0; ph < phases; ++ph) {
            p.o0[ph] = ph;
            p.m_count[ph] = std::max(0, (len - ph + op.stride - 1) / op.stride);
            for (int j = (ph + op.padding) % op.stride; j < op.kernel; j += op.stride) {
                if (p.ntaps[ph] == kMaxTaps) return hipErrorInvalidValue;
                p.off[ph][p.ntaps[ph]] = (ph + op.padding - j) / op.stride;  // exact: j = ph + padding (mod stride)
                p.slab[ph][p.ntaps[ph]] = j;
                ++p.ntaps[ph];
            }
        }
    }
    const int tile = c.mfma ? kMmaTile : kNarrowRows;
    int mtiles = 0;
    for (int ph = 0; ph < phases; ++ph) {
        int lo = 0, hi = 0;
        if (p.ntaps[ph] > 0) lo = hi = p.off[ph][0];
        for (int q = 1; q < p.ntaps[ph]; ++q) {
            lo = std::min(lo, p.off[ph][q]);
            hi = std::max(hi, p.off[ph][q]);
        }
        p.off_min[ph] = lo;
        p.span = std::max(p.span, (tile - 1) * p.istride + hi - lo + 1);
        p.ltaps = std::max(p.ltaps, p.ntaps[ph]);
        mtiles = std::max(mtiles, (p.m_count[ph] + tile - 1) / tile);
    }
    if (mtiles == 0) return hipSuccess;
    const size_t pitch = c.chunk + 4;
    const size_t lds = c.mfma ? sizeof(float) * ((size_t)p.ltaps * kMmaTile * pitch + (size_t)p.span * pitch)
                              : sizeof(float) * ((size_t)p.ltaps * kChunk * c.cout_pad + (size_t)p.span * kNarrowPad);
    if (lds > kMaxLds) return hipErrorInvalidValue;
    if (c.mfma) {
        const dim3 grid(mtiles, c.cout_pad / kMmaTile, phases);
#define Y2_MFMA(T, KC, VEC)                                                                           \
    {                                                                                                 \
        if (act == ACT_SNAKE) return launch(conv_mfma_kernel<ACT_SNAKE, T, KC, VEC>, grid, lds, s, p); \
        if (act == ACT_ELU) return launch(conv_mfma_kernel<ACT_ELU, T, KC, VEC>, grid, lds, s, p);     \
        return launch(conv_mfma_kernel<ACT_NONE, T, KC, VEC>, grid, lds, s, p);                       \
    }
        // the kernels' register slots hold span * KC / 4 source floats4 over 256 threads
        bool same = true;  // every phase has ltaps taps
        for (int ph = 0; ph < phases; ++ph) same = same && p.ntaps[ph] == p.ltaps;
        const bool vec = op.cin % 4 == 0;
        if (c.chunk == 32 && vec) {
            if (same && p.ltaps == 1 && p.span * 8 <= 4 * 256) Y2_MFMA(1, 32, true)
            if (same && p.ltaps == 2 && p.span * 8 <= 5 * 256) Y2_MFMA(2, 32, true)
        }
        if (c.chunk == 8 && p.span * 2 <= 3 * 256) {
            if (same && p.ltaps == 7 && vec) Y2_MFMA(7, 8, true)
            if (p.ltaps <= kMaxTaps && vec) Y2_MFMA(0, 8, true)
            if (p.ltaps <= kMaxTaps) Y2_MFMA(0, 8, false)
        }
#undef Y2_MFMA
        return hipErrorInvalidValue;
    }
    const dim3 grid(mtiles, 1, phases);
#define Y2_NARROW(CO)                                                                       \
    if (c.cout_pad == CO) {                                                                 \
        if (act == ACT_SNAKE) return launch(conv_narrow_kernel<CO, ACT_SNAKE>, grid, lds, s, p); \
        if (act == ACT_ELU) return launch(conv_narrow_kernel<CO, ACT_ELU>, grid, lds, s, p);     \
        return launch(conv_narrow_kernel<CO, ACT_NONE>, grid, lds, s, p);                   \
    }
    Y2_NARROW(2)
    Y2_NARROW(4)
    Y2_NARROW(8)
    Y2_NARROW(16)
#undef Y2_NARROW
    return hipErrorInvalidValue;
}

}  // namespace
}  // namespace y2

struct Yue2Vae {
    y2::VaeHost host;
    std::vector<float*> w, b, a, ib;  // per op, device
    std::vector<y2::ConvShape> shape;  // per op: the convolution's kernel and padded widths
    void* block = nullptr;
    void* acts = nullptr;  // three activation buffers, kept between calls
    size_t acts_bytes = 0;
    hipStream_t stream = nullptr;
};

extern "C" void yue2_hip_vae_free(Yue2Vae* v) {
    if (!v) return;
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (v->stream) (void)hipStreamSynchronize(v->stream);
    if (v->block) (void)hipFree(v->block);
    if (v->acts) (void)hipFree(v->acts);
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
    v->shape.assign(nops, ConvShape{});
    for (size_t k = 0; k < nops; ++k) {
        const VaeOpHost& op = v->host.ops[k];
        if (op.kind == VAE_CONV || op.kind == VAE_CONVT) v->shape[k] = conv_shape(op);
        ow[k] = take((size_t)op.kernel * v->shape[k].cin_pad * v->shape[k].cout_pad);
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
        if (op.kind == VAE_CONV || op.kind == VAE_CONVT) up(conv_slabs(op, v->shape[k]), ow[k], &v->w[k]);
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
// latent] -> out [length, audio channels].  An activation that a
// convolution follows is applied inside that convolution, a residual unit's
// sum in its last convolution's epilogue, a final tanh in the last
// convolution's.
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
    const size_t stride = (most * sizeof(float) + 255) / 256 * 256;
    hipStream_t s = v->stream;
    hipError_t e = hipSuccess;
    if (3 * stride > v->acts_bytes) {
        if (v->acts) (void)hipFree(v->acts);
        v->acts = nullptr;
        v->acts_bytes = 0;
        if ((e = hipMalloc(&v->acts, 3 * stride)) != hipSuccess) return hip_fail(e, "VAE activations");
        v->acts_bytes = 3 * stride;
    }
    float* buf[3];
    for (int i = 0; i < 3; ++i) buf[i] = reinterpret_cast<float*>(static_cast<char*>(v->acts) + i * stride);
    int cur = 0, res = -1, pending = -1;  // pending: an activation waiting for the next convolution
    n = frames;
    c = h.latent_dim;
    auto free_buf = [&]() {
        for (int i = 0; i < 3; ++i)
            if (i != cur && i != res) return i;
        return -1;
    };
    auto is_conv = [&](size_t k) { return k < h.ops.size() && (h.ops[k].kind == VAE_CONV || h.ops[k].kind == VAE_CONVT); };
    e = hipMemcpyAsync(buf[0], z, sizeof(float) * (size_t)frames * c, hipMemcpyHostToDevice, s);
    int rc = e == hipSuccess ? YUE2_OK : hip_fail(e, "VAE input");
    const size_t nops = h.ops.size();
    for (size_t k = 0; k < nops && rc == YUE2_OK; ++k) {
        const VaeOpHost& op = h.ops[k];
        const int dst = free_buf();
        if (is_conv(k)) {
            const bool join = k + 1 < nops && h.ops[k + 1].kind == VAE_RES_END && res >= 0;
            const bool tanh_out = !join && k + 1 < nops && h.ops[k + 1].kind == VAE_TANH;
            int act = ACT_NONE;
            const float *alpha = nullptr, *inv_beta = nullptr;
            if (pending >= 0) {
                act = h.ops[pending].kind == VAE_SNAKE ? ACT_SNAKE : ACT_ELU;
                alpha = v->a[pending];
                inv_beta = v->ib[pending];
            }
            e = run_conv(s, op, v->shape[k], v->w[k], v->b[k], buf[cur], n, buf[dst], join ? buf[res] : nullptr, act,
                         alpha, inv_beta, tanh_out);
            if (e != hipSuccess) {
                rc = hip_fail(e, "VAE convolution");
                break;
            }
            n = conv_length(op, n);
            c = op.cout;
            cur = dst;
            pending = -1;
            if (join) res = -1;
            if (join || tanh_out) ++k;  // the RES_END or TANH it absorbed
        } else if ((op.kind == VAE_SNAKE || op.kind == VAE_ELU) && is_conv(k + 1)) {
            pending = (int)k;
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
    for (size_t i = 0; i < (size_t)frames * h.latent_dim; ++i)  // validate_latent before the halo check
        if (!std::isfinite(z[i])) return fail(YUE2_ERR_ARG, "Expected finite nonempty [frames,64] latents");
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
    const ConvShape shape = conv_shape(op);
    const std::vector<float> slabs = conv_slabs(op, shape);
    float *dx = nullptr, *dw = nullptr, *db = nullptr, *dy = nullptr;
    hipError_t e = hipMalloc(&dx, sizeof(float) * (size_t)frames * cin);
    if (e == hipSuccess) e = hipMalloc(&dw, sizeof(float) * slabs.size());
    if (e == hipSuccess) e = hipMalloc(&db, sizeof(float) * cout);
    if (e == hipSuccess) e = hipMalloc(&dy, sizeof(float) * (size_t)len * cout);
    if (e == hipSuccess) e = hipMemcpy(dx, x, sizeof(float) * (size_t)frames * cin, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(dw, slabs.data(), sizeof(float) * slabs.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess && bias) e = hipMemcpy(db, bias, sizeof(float) * cout, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = run_conv(nullptr, op, shape, dw, bias ? db : nullptr, dx, frames, dy, nullptr, ACT_NONE, nullptr, nullptr,
                     false);
    if (e == hipSuccess) e = hipMemcpy(out, dy, sizeof(float) * (size_t)len * cout, hipMemcpyDeviceToHost);
    (void)hipFree(dx);
    (void)hipFree(dw);
    (void)hipFree(db);
    (void)hipFree(dy);
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "convolution selftest");
}
