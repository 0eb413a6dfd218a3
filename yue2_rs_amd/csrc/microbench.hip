// microbench.hip -- device-resident microbenchmarks of the decode kernels
// against the HBM roofline: the BF16 GEMV family at the 3B layer shapes,
// the split-KV decode attention over growing contexts, and a plain
// device-to-device copy (the practical HBM rate and the calibration workload
// of the traffic counters).  Inputs live in HBM
// before timing; each launch reads a different copy of its operands (more
// than the 256 MB Infinity Cache in total), so repeats are not served from
// the cache.  Times are HIP events around the launches on one stream.
#include <algorithm>
#include <cmath>
#include <vector>

#include "../../include/yue2_hip.h"
#include "kernels.h"
#include "runtime.h"
#include "y2_math.h"

namespace y2 {
namespace {

// BF16 values in [-0.0345, 0.0345) (the magnitude of N(0, 0.02) weights)
// from a counter hash: the timing does not depend on the values.
__global__ void fill_bf16_kernel(uint16_t* p, size_t n, uint64_t seed, float scale) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        uint64_t z = seed + 0x9e3779b97f4a7c15ull * (i + 1);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        const float u = (float)(z >> 40) * 0x1.0p-24f - 0.5f;  // [-0.5, 0.5)
        p[i] = bf16_bits(rb(u * scale));
    }
}

void fill_bf16(hipStream_t s, uint16_t* p, size_t n, uint64_t seed, float scale) {
    fill_bf16_kernel<<<1024, 256, 0, s>>>(p, n, seed, scale);
}

// Frees every pointer it holds on scope exit.
struct DevBufs {
    std::vector<void*> p;
    void* alloc(size_t bytes) {
        void* q = nullptr;
        if (hipMalloc(&q, bytes) != hipSuccess) return nullptr;
        p.push_back(q);
        return q;
    }
    ~DevBufs() {
        for (void* q : p) (void)hipFree(q);
    }
};

struct Events {
    hipEvent_t a = nullptr, b = nullptr;
    bool ok() { return hipEventCreate(&a) == hipSuccess && hipEventCreate(&b) == hipSuccess; }
    ~Events() {
        if (a) (void)hipEventDestroy(a);
        if (b) (void)hipEventDestroy(b);
    }
};

}  // namespace
}  // namespace y2

using namespace y2;

extern "C" int32_t yue2_hip_bench_copy(int64_t bytes, int32_t iters, float* avg_ms) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!avg_ms || bytes <= 0 || bytes % 256 || iters < 1) return fail(YUE2_ERR_ARG, "bad copy benchmark request");
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no usable gfx950 device");
    DevBufs m;
    void* src = m.alloc((size_t)bytes);
    void* dst = m.alloc((size_t)bytes);
    if (!src || !dst) return fail(YUE2_ERR_ALLOC, "copy benchmark buffers");
    hipStream_t s = nullptr;
    fill_bf16(s, static_cast<uint16_t*>(src), (size_t)bytes / 2, 11, 1.0f);
    Events ev;
    if (!ev.ok()) return fail(YUE2_ERR_DEVICE, "hipEventCreate");
    hipError_t e = hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipEventRecord(ev.a, s);
    for (int i = 0; i < iters && e == hipSuccess; ++i)
        e = hipMemcpyAsync(dst, src, (size_t)bytes, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipEventRecord(ev.b, s);
    if (e == hipSuccess) e = hipEventSynchronize(ev.b);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.a, ev.b);
    if (e != hipSuccess) return hip_fail(e, "copy benchmark");
    *avg_ms = ms / (float)iters;
    return YUE2_OK;
}

extern "C" int32_t yue2_hip_bench_gemv(int32_t n, int32_t k, int32_t rows, int32_t copies, int32_t iters,
                                       float* avg_ms, double* bytes) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!avg_ms || !bytes || n <= 0 || k <= 0 || k % 8 || rows < 1 || rows > kMaxRows || copies < 1 || iters < 1)
        return fail(YUE2_ERR_ARG, "bad GEMV benchmark request");
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no usable gfx950 device");
    DevBufs m;
    std::vector<uint16_t*> w(copies);
    const size_t wn = (size_t)n * k;
    for (int c = 0; c < copies; ++c)
        if (!(w[c] = static_cast<uint16_t*>(m.alloc(wn * 2)))) return fail(YUE2_ERR_ALLOC, "GEMV benchmark weights");
    float* x = static_cast<float*>(m.alloc((size_t)rows * k * sizeof(float)));
    float* y = static_cast<float*>(m.alloc((size_t)rows * n * sizeof(float)));
    uint16_t* xb = static_cast<uint16_t*>(m.alloc((size_t)rows * k * 2));
    if (!x || !y || !xb) return fail(YUE2_ERR_ALLOC, "GEMV benchmark vectors");
    hipStream_t s = nullptr;
    for (int c = 0; c < copies; ++c) fill_bf16(s, w[c], wn, 1000 + c, 0.069f);
    // x ~ N(0, 1)-sized BF16 values held as f32
    fill_bf16(s, xb, (size_t)rows * k, 7, 3.46f);
    std::vector<uint16_t> hb((size_t)rows * k);
    std::vector<float> hx(hb.size());
    if (hipMemcpy(hb.data(), xb, hb.size() * 2, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(YUE2_ERR_DEVICE, "GEMV benchmark input");
    for (size_t i = 0; i < hb.size(); ++i) hx[i] = bf16(hb[i]);
    if (hipMemcpy(x, hx.data(), hx.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
        return fail(YUE2_ERR_DEVICE, "GEMV benchmark input");
    Events ev;
    if (!ev.ok()) return fail(YUE2_ERR_DEVICE, "hipEventCreate");
    GemvArgs a{nullptr, nullptr, x, y, k, n, n, k, rows, nullptr, 0.0f, nullptr};
    hipError_t e = hipSuccess;
    for (int i = 0; i < copies && e == hipSuccess; ++i) {
        a.w = w[i];
        e = launch_gemv(s, EPI_STORE, a);
    }
    if (e == hipSuccess) e = hipEventRecord(ev.a, s);
    for (int i = 0; i < iters && e == hipSuccess; ++i) {
        a.w = w[i % copies];
        e = launch_gemv(s, EPI_STORE, a);
    }
    if (e == hipSuccess) e = hipEventRecord(ev.b, s);
    if (e == hipSuccess) e = hipEventSynchronize(ev.b);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.a, ev.b);
    if (e != hipSuccess) return hip_fail(e, "GEMV benchmark");
    *avg_ms = ms / (float)iters;
    *bytes = (double)wn * 2.0 + (double)rows * k * 2.0 + (double)rows * n * 4.0;
    return YUE2_OK;
}

extern "C" int32_t yue2_hip_bench_attention(int32_t context, int32_t rows, int32_t layers, int32_t iters,
                                            float* avg_ms, double* bytes) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    constexpr int Hq = 24, Hkv = 8, D = 128;
    if (!avg_ms || !bytes || context < 1 || context > kContext || rows < 1 || rows > kMaxRows || layers < 1 ||
        iters < 1)
        return fail(YUE2_ERR_ARG, "bad attention benchmark request");
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no usable gfx950 device");
    const int pos = context - 1, cap = context;  // the new token attends `context` positions
    const int max_blocks = (cap + kBlockKeys - 1) / kBlockKeys;
    const size_t qkvw = (size_t)(Hq + 2 * Hkv) * D;
    const size_t per_row = (size_t)layers * 2 * Hkv * cap * D;  // BF16 K/V of one cache
    DevBufs m;
    KvView kv{};
    for (int b = 0; b < rows; ++b) {
        kv.base[b] = static_cast<uint16_t*>(m.alloc(per_row * 2));
        kv.capacity[b] = cap;
        if (!kv.base[b]) return fail(YUE2_ERR_ALLOC, "attention benchmark cache");
    }
    float* qkv = static_cast<float*>(m.alloc((size_t)rows * qkvw * sizeof(float)));
    float* out = static_cast<float*>(m.alloc((size_t)rows * Hq * D * sizeof(float)));
    const size_t blk = (size_t)rows * Hq * max_blocks;
    float* bmax = static_cast<float*>(m.alloc(blk * sizeof(float)));
    float* bsum = static_cast<float*>(m.alloc(blk * sizeof(float)));
    float* part = static_cast<float*>(m.alloc(blk * D * sizeof(float)));
    int32_t* counters = static_cast<int32_t*>(m.alloc((size_t)rows * Hkv * 4 * sizeof(int32_t)));
    // the tagged-word attention's block maxima, sums and partials
    uint64_t* tags = static_cast<uint64_t*>(m.alloc((2 + D) * blk * sizeof(uint64_t)));
    StepState* st = static_cast<StepState*>(m.alloc(sizeof(StepState)));
    float* cos_t = static_cast<float*>(m.alloc((size_t)cap * (D / 2) * sizeof(float)));
    float* sin_t = static_cast<float*>(m.alloc((size_t)cap * (D / 2) * sizeof(float)));
    float* gam = static_cast<float*>(m.alloc(D * sizeof(float)));
    uint16_t* qb = static_cast<uint16_t*>(m.alloc((size_t)rows * qkvw * 2));
    if (!qkv || !out || !bmax || !bsum || !part || !counters || !tags || !st || !cos_t || !sin_t || !gam || !qb)
        return fail(YUE2_ERR_ALLOC, "attention benchmark buffers");
    hipStream_t s = nullptr;
    // K, V and q ~ N(0, 1)-sized BF16 values; RoPE at the positions
    // (theta 1e4); QK-norm gammas 1.
    for (int b = 0; b < rows; ++b) fill_bf16(s, kv.base[b], per_row, 50 + b, 3.46f);
    fill_bf16(s, qb, (size_t)rows * qkvw, 60, 3.46f);
    {
        std::vector<uint16_t> hb((size_t)rows * qkvw);
        std::vector<float> hq(hb.size());
        if (hipMemcpy(hb.data(), qb, hb.size() * 2, hipMemcpyDeviceToHost) != hipSuccess)
            return fail(YUE2_ERR_DEVICE, "attention benchmark input");
        for (size_t i = 0; i < hb.size(); ++i) hq[i] = bf16(hb[i]);
        std::vector<float> hc((size_t)cap * (D / 2)), hs(hc.size()), hg(D, 1.0f);
        for (int p = 0; p < cap; ++p)
            for (int i = 0; i < D / 2; ++i) {
                const float f = 1.0f / std::pow(10000.0f, (float)(2 * i) / (float)D);
                hc[(size_t)p * (D / 2) + i] = rb(std::cos((float)p * f));
                hs[(size_t)p * (D / 2) + i] = rb(std::sin((float)p * f));
            }
        StepState hst{};
        for (int b = 0; b < rows; ++b) hst.pos[b] = pos;
        if (hipMemcpy(qkv, hq.data(), hq.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(cos_t, hc.data(), hc.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(sin_t, hs.data(), hs.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(gam, hg.data(), D * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(st, &hst, sizeof(hst), hipMemcpyHostToDevice) != hipSuccess ||
            hipMemset(counters, 0, (size_t)rows * Hkv * 4 * sizeof(int32_t)) != hipSuccess ||
            hipMemset(tags, 0, (2 + D) * blk * sizeof(uint64_t)) != hipSuccess)
            return fail(YUE2_ERR_DEVICE, "attention benchmark input");
    }
    AttnArgs aa{};
    aa.qkv = qkv;
    aa.qkv_stride = (int)qkvw;
    aa.kv = kv;
    aa.heads = Hq;
    aa.kv_heads = Hkv;
    aa.dim = D;
    aa.rows = rows;
    aa.scale = 1.0f / std::sqrt((float)D);
    aa.eps = 1e-6f;
    aa.q_norm = gam;
    aa.k_norm = gam;
    aa.cos_t = cos_t;
    aa.sin_t = sin_t;
    aa.bmax = bmax;
    aa.bsum = bsum;
    aa.part = part;
    aa.out = out;
    aa.out_stride = Hq * D;
    aa.blk_stride = max_blocks;
    attention_geometry(Hkv, rows, max_blocks, &aa.wgs, &aa.bpw);
    aa.counters = counters;
    aa.st = st;
    aa.tbmax = tags;
    aa.tbsum = tags + blk;
    aa.tpart = tags + 2 * blk;
    Events ev;
    if (!ev.ok()) return fail(YUE2_ERR_DEVICE, "hipEventCreate");
    hipError_t e = hipSuccess;
    // the tagged-word attention's tags take the sequence and the layer: the
    // sequence advances after each pass over the layers (as after a decode
    // step), so no launch can pass a poll on an earlier launch's word
    for (int l = 0; l < layers && e == hipSuccess; ++l) {
        aa.layer = l;
        e = launch_attention(s, aa);
    }
    launch_sequence(s, st, 0, 1);
    if (e == hipSuccess) e = hipEventRecord(ev.a, s);
    for (int i = 0; i < iters && e == hipSuccess; ++i) {
        aa.layer = i % layers;
        e = launch_attention(s, aa);
        if (aa.layer == layers - 1) launch_sequence(s, st, 0, 1);
    }
    if (e == hipSuccess) e = hipEventRecord(ev.b, s);
    if (e == hipSuccess) e = hipEventSynchronize(ev.b);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.a, ev.b);
    if (e != hipSuccess) return hip_fail(e, "attention benchmark");
    StepState hst{};
    if (hipMemcpy(&hst, st, sizeof(hst), hipMemcpyDeviceToHost) != hipSuccess)
        return fail(YUE2_ERR_DEVICE, "attention benchmark state");
    if (hst.error) return fail(YUE2_ERR_DEVICE, "attention benchmark: device error");
    *avg_ms = ms / (float)iters;
    // K and V of every attended position, 8 heads x 128 x BF16 each, per row
    *bytes = (double)rows * 2.0 * Hkv * D * 2.0 * context;
    return YUE2_OK;
}
