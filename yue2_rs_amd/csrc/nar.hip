// nar.hip -- the NAR velocity stack, Model::velocity (src/model.rs:611-698),
// on the matrix cores.
//
// The reference runs the acoustic stage's layers through yue2_metal_stack
// (src/metal.m:429-538) and the small linears around them on the CPU.  Here
// the whole velocity runs on the device: the padded latents through vae2llm
// (a BF16 MFMA GEMM with the bias in its epilogue), the timestep MLP (two
// one-row GEMMs, the SiLU fused), the time and latent-position rows, every
// NAR layer as in the prefill (GEMMs, QK-norm + RoPE, flash attention) but
// with non-causal attention over the cache's prefix and the rows' own keys,
// and llm2vae over the final-normed rows 1 .. n-2.  The rows' own keys go to
// a scratch K/V buffer: the cache is never written.  Only the timestep's
// scalar and its 256 sinusoid values (libm cos/sin of one number, host work
// in the reference too) are computed on the host.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "../../include/yue2_hip.h"
#include "dev_mem.h"
#include "kernels.h"
#include "prefill.h"
#include "runtime.h"
#include "y2_math.h"

using namespace y2;

namespace y2 {
namespace {

// x[r][i] = rb(rb(x[r][i] + time[i]) + pe[min(r, max_frames - 1)][i])
// (src/model.rs:640-649; the position rows are BF16, so rb(pe) = pe).
__global__ __launch_bounds__(256) void time_position_kernel(float* x, const float* time, const uint16_t* pe,
                                                            int H, int max_frames) {
    const int r = blockIdx.x, pr = min(r, max_frames - 1);
    for (int i = threadIdx.x; i < H; i += 256) {
        float* v = x + (size_t)r * H + i;
        *v = rb(rb(*v + time[i]) + bf16(pe[(size_t)pr * H + i]));
    }
}

// 256-byte aligned sub-allocations of one block.
struct Carve {
    size_t offset = 0;
    template <class T>
    size_t take(size_t n) {
        const size_t o = offset;
        offset = (offset + n * sizeof(T) + 255) / 256 * 256;
        return o;
    }
};

}  // namespace
}  // namespace y2

extern "C" int32_t yue2_hip_nar_load(Yue2Model* m, const Yue2NarWeights* w) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || !w || !w->layers) return fail(YUE2_ERR_ARG, "null model or NAR weights");
    const Yue2Config& c = m->c;
    const int H = c.hidden_size, D = c.head_dim, I = c.intermediate_size, Lat = w->latent_dim;
    const int qw = c.num_attention_heads * D, kw = c.num_key_value_heads * D, qkvw = qw + 2 * kw;
    if (Lat <= 0 || Lat % kGemmTK || w->max_latent_frames < 1 || !(w->timestep_shift > 0.0f) ||
        !std::isfinite(w->timestep_shift))
        return fail(YUE2_ERR_CONFIG, "Invalid transformer configuration");
    if (H % kGemmTK || I % kGemmTK || qw % kGemmTK || (D != 64 && D != 128))
        return fail(YUE2_ERR_ARG, "shape without an MFMA NAR stack");
    if (!w->vae2llm || !w->llm2vae || !w->time_in || !w->time_out || !w->latent_pos || !w->vae2llm_bias ||
        !w->llm2vae_bias || !w->time_in_bias || !w->time_out_bias)
        return fail(YUE2_ERR_ARG, "null NAR weight");
    for (int l = 0; l < c.num_hidden_layers; ++l) {
        const Yue2LayerWeights& s = w->layers[l];
        if (!s.q_proj || !s.k_proj || !s.v_proj || !s.o_proj || !s.gate_proj || !s.up_proj || !s.down_proj ||
            !s.input_layernorm || !s.q_norm || !s.k_norm || !s.post_attention_layernorm)
            return fail(YUE2_ERR_ARG, "null layer weight");
    }
    Carve cv;
    struct Off { size_t qkv, o, g, u, d, in, qn, kn, post; };
    std::vector<Off> offs(c.num_hidden_layers);
    for (auto& o : offs) {
        o.qkv = cv.take<uint16_t>((size_t)qkvw * H);
        o.o = cv.take<uint16_t>((size_t)H * qw);
        o.g = cv.take<uint16_t>((size_t)I * H);
        o.u = cv.take<uint16_t>((size_t)I * H);
        o.d = cv.take<uint16_t>((size_t)H * I);
        o.in = cv.take<float>(H);
        o.qn = cv.take<float>(D);
        o.kn = cv.take<float>(D);
        o.post = cv.take<float>(H);
    }
    const size_t o_v2l = cv.take<uint16_t>((size_t)H * Lat), o_l2v = cv.take<uint16_t>((size_t)Lat * H);
    const size_t o_tin = cv.take<uint16_t>((size_t)H * 256), o_tout = cv.take<uint16_t>((size_t)H * H);
    const size_t o_pe = cv.take<uint16_t>((size_t)w->max_latent_frames * H);
    const size_t o_bv = cv.take<float>(H), o_bl = cv.take<float>(Lat), o_bi = cv.take<float>(H),
                 o_bo = cv.take<float>(H);
    (void)hipStreamSynchronize(m->stream);
    if (m->nar.block) (void)hipFree(m->nar.block);
    m->nar = NarDev{};
    void* block = nullptr;
    hipError_t e = hipMalloc(&block, cv.offset);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(NAR weights)");
    char* base = static_cast<char*>(block);
    NarDev& n = m->nar;
    bool ok = true;
    auto up = [&](void* dst, const void* src, size_t bytes) {
        if (ok && hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) != hipSuccess) ok = false;
    };
    // norm gammas and biases rounded to BF16 as Norm::new and Linear::finish do
    auto up_rb = [&](float* dst, const float* src, int count) {
        std::vector<float> tmp(src, src + count);
        for (float& v : tmp) v = rb(v);
        up(dst, tmp.data(), sizeof(float) * count);
    };
    n.layers.resize(c.num_hidden_layers);
    for (int l = 0; l < c.num_hidden_layers; ++l) {
        const Yue2LayerWeights& s = w->layers[l];
        LayerDev& L = n.layers[l];
        const Off& o = offs[l];
        L.wqkv = reinterpret_cast<uint16_t*>(base + o.qkv);
        L.wo = reinterpret_cast<uint16_t*>(base + o.o);
        L.wg = reinterpret_cast<uint16_t*>(base + o.g);
        L.wu = reinterpret_cast<uint16_t*>(base + o.u);
        L.wd = reinterpret_cast<uint16_t*>(base + o.d);
        L.in_norm = reinterpret_cast<float*>(base + o.in);
        L.q_norm = reinterpret_cast<float*>(base + o.qn);
        L.k_norm = reinterpret_cast<float*>(base + o.kn);
        L.post_norm = reinterpret_cast<float*>(base + o.post);
        up(L.wqkv, s.q_proj, sizeof(uint16_t) * (size_t)qw * H);
        up(L.wqkv + (size_t)qw * H, s.k_proj, sizeof(uint16_t) * (size_t)kw * H);
        up(L.wqkv + (size_t)(qw + kw) * H, s.v_proj, sizeof(uint16_t) * (size_t)kw * H);
        up(L.wo, s.o_proj, sizeof(uint16_t) * (size_t)H * qw);
        up(L.wg, s.gate_proj, sizeof(uint16_t) * (size_t)I * H);
        up(L.wu, s.up_proj, sizeof(uint16_t) * (size_t)I * H);
        up(L.wd, s.down_proj, sizeof(uint16_t) * (size_t)H * I);
        up_rb(L.in_norm, s.input_layernorm, H);
        up_rb(L.q_norm, s.q_norm, D);
        up_rb(L.k_norm, s.k_norm, D);
        up_rb(L.post_norm, s.post_attention_layernorm, H);
    }
    n.vae2llm = reinterpret_cast<uint16_t*>(base + o_v2l);
    n.llm2vae = reinterpret_cast<uint16_t*>(base + o_l2v);
    n.time_in = reinterpret_cast<uint16_t*>(base + o_tin);
    n.time_out = reinterpret_cast<uint16_t*>(base + o_tout);
    n.latent_pos = reinterpret_cast<uint16_t*>(base + o_pe);
    n.vae2llm_b = reinterpret_cast<float*>(base + o_bv);
    n.llm2vae_b = reinterpret_cast<float*>(base + o_bl);
    n.time_in_b = reinterpret_cast<float*>(base + o_bi);
    n.time_out_b = reinterpret_cast<float*>(base + o_bo);
    up(n.vae2llm, w->vae2llm, sizeof(uint16_t) * (size_t)H * Lat);
    up(n.llm2vae, w->llm2vae, sizeof(uint16_t) * (size_t)Lat * H);
    up(n.time_in, w->time_in, sizeof(uint16_t) * (size_t)H * 256);
    up(n.time_out, w->time_out, sizeof(uint16_t) * (size_t)H * H);
    up(n.latent_pos, w->latent_pos, sizeof(uint16_t) * (size_t)w->max_latent_frames * H);
    up_rb(n.vae2llm_b, w->vae2llm_bias, H);
    up_rb(n.llm2vae_b, w->llm2vae_bias, Lat);
    up_rb(n.time_in_b, w->time_in_bias, H);
    up_rb(n.time_out_b, w->time_out_bias, H);
    if (!ok) {
        (void)hipFree(block);
        m->nar = NarDev{};
        return fail(YUE2_ERR_DEVICE, "NAR weight upload failed");
    }
    n.block = block;
    n.latent = Lat;
    n.max_frames = w->max_latent_frames;
    n.shift = w->timestep_shift;
    return YUE2_OK;
}

namespace {

// The timestep embedding's input (src/model.rs:624-634): t from raw_t, then
// rb(cos(t f_i)) and rb(sin(t f_i)), f_i = exp(-ln(10000) i / 128), as BF16
// bits.  exp is the correctly rounded f32 exp the device uses everywhere.
void timestep_sinus(double raw_t, float shift, uint16_t* sinus) {
    const float raw = rb((float)raw_t);
    const float sig = rb(1.0f / (1.0f + expf_cr(-raw)));
    const float top = rb(shift * sig);
    const float bottom = rb(1.0f + rb((shift - 1.0f) * sig));
    const float t = rb(top / bottom);
    const float ln = logf(10000.0f);
    for (int i = 0; i < 128; ++i) {
        const float f = expf_cr(-ln * (float)i / 128.0f);
        sinus[i] = bf16_bits(rb(cosf(t * f)));
        sinus[128 + i] = bf16_bits(rb(sinf(t * f)));
    }
}

}  // namespace

extern "C" int32_t yue2_hip_velocity(Yue2Model* m, const Yue2Cache* c, const float* state, int32_t frames,
                                     double raw_t, int32_t nar_cond_end, float* out) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || !c || !state || !out || c->m != m) return fail(YUE2_ERR_ARG, "null model, cache, state or output");
    if (!m->nar.block) return fail(YUE2_ERR_ARG, "NAR weights not loaded");
    const Yue2Config& cf = m->c;
    const NarDev& nd = m->nar;
    const int H = cf.hidden_size, D = cf.head_dim, Hq = cf.num_attention_heads, Hkv = cf.num_key_value_heads;
    const int I = cf.intermediate_size, qw = Hq * D, qkvw = (Hq + 2 * Hkv) * D, Lat = nd.latent;
    if (frames < 1) return fail(YUE2_ERR_ARG, "Expected nonempty latent frames");
    const int n = frames + 2;
    if (c->length + n > cf.max_position_embeddings) return fail(YUE2_ERR_CONTEXT, "AR input exceeds cache/model context");
    for (size_t i = 0; i < (size_t)frames * Lat; ++i)
        if (!(rb(state[i]) == state[i])) return fail(YUE2_ERR_ARG, "latent state must hold finite BF16 values");
    const int visible = nar_cond_end > 0 ? std::min(nar_cond_end, c->length) : c->length;
    // host inputs: the padded latents (zero first and last rows) and the sinus row
    std::vector<uint16_t> pad((size_t)n * Lat, 0), sinus(256);
    for (size_t i = 0; i < (size_t)frames * Lat; ++i) pad[(size_t)Lat + i] = bf16_bits(state[i]);
    timestep_sinus(raw_t, nd.shift, sinus.data());
    Carve cv;
    const size_t o_pad = cv.take<uint16_t>(pad.size()), o_sin = cv.take<uint16_t>(256);
    const size_t o_t0 = cv.take<uint16_t>(H), o_tv = cv.take<float>(H);
    const size_t o_x = cv.take<float>((size_t)n * H), o_qkv = cv.take<float>((size_t)n * qkvw);
    const size_t o_h = cv.take<uint16_t>((size_t)n * std::max(H, I)), o_q = cv.take<uint16_t>((size_t)n * qw);
    const size_t o_att = cv.take<uint16_t>((size_t)n * qw), o_act = cv.take<uint16_t>((size_t)n * I);
    const size_t o_kv = cv.take<uint16_t>((size_t)cf.num_hidden_layers * 2 * Hkv * n * D);
    const size_t o_out = cv.take<float>((size_t)frames * Lat);
    void* block = nullptr;
    hipError_t e = hipMalloc(&block, cv.offset);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(NAR buffers)");
    char* base = static_cast<char*>(block);
    uint16_t* d_pad = reinterpret_cast<uint16_t*>(base + o_pad);
    uint16_t* d_sin = reinterpret_cast<uint16_t*>(base + o_sin);
    uint16_t* t0 = reinterpret_cast<uint16_t*>(base + o_t0);
    float* tv = reinterpret_cast<float*>(base + o_tv);
    float* x = reinterpret_cast<float*>(base + o_x);
    float* qkv = reinterpret_cast<float*>(base + o_qkv);
    uint16_t* h = reinterpret_cast<uint16_t*>(base + o_h);
    uint16_t* q = reinterpret_cast<uint16_t*>(base + o_q);
    uint16_t* att = reinterpret_cast<uint16_t*>(base + o_att);
    uint16_t* act = reinterpret_cast<uint16_t*>(base + o_act);
    uint16_t* kv2 = reinterpret_cast<uint16_t*>(base + o_kv);
    float* d_out = reinterpret_cast<float*>(base + o_out);
    hipStream_t s = m->stream;
    const float eps = cf.rms_norm_eps;
    auto run = [&]() -> int {
        if ((e = hipMemcpyAsync(d_pad, pad.data(), pad.size() * 2, hipMemcpyHostToDevice, s)) != hipSuccess ||
            (e = hipMemcpyAsync(d_sin, sinus.data(), 256 * 2, hipMemcpyHostToDevice, s)) != hipSuccess)
            return hip_fail(e, "NAR input upload");
        // vae2llm over the padded rows (:623)
        GemmArgs gv{d_pad, Lat, nd.vae2llm, nullptr, Lat, x, nullptr, H, n, H, Lat, nd.vae2llm_b};
        if ((e = launch_gemm(s, GEPI_BIAS, gv)) != hipSuccess) return hip_fail(e, "vae2llm");
        // time_embedder: mlp.0, rb(silu), mlp.2 (:635-639)
        GemmArgs gi{d_sin, 256, nd.time_in, nullptr, 256, nullptr, t0, H, 1, H, 256, nd.time_in_b};
        if ((e = launch_gemm(s, GEPI_BIAS_SILU_BF16, gi)) != hipSuccess) return hip_fail(e, "time_in");
        GemmArgs go{t0, H, nd.time_out, nullptr, H, tv, nullptr, H, 1, H, H, nd.time_out_b};
        if ((e = launch_gemm(s, GEPI_BIAS, go)) != hipSuccess) return hip_fail(e, "time_out");
        time_position_kernel<<<n, 256, 0, s>>>(x, tv, nd.latent_pos, H, nd.max_frames);
        if ((e = hipGetLastError()) != hipSuccess) return hip_fail(e, "time and position rows");
        // the NAR layers (:680-695); RoPE positions start at the cache length
        for (int l = 0; l < cf.num_hidden_layers; ++l) {
            const LayerDev& L = nd.layers[l];
            if ((e = launch_norm_rows(s, x, L.in_norm, h, n, H, eps)) != hipSuccess) return hip_fail(e, "NAR norm");
            GemmArgs g{h, H, L.wqkv, nullptr, H, qkv, nullptr, qkvw, n, qkvw, H, nullptr};
            if ((e = launch_gemm(s, GEPI_ROUND, g)) != hipSuccess) return hip_fail(e, "NAR qkv");
            RopeArgs ra{qkv, q, c->kv, c->capacity, l, Hq, Hkv, D, c->length, L.q_norm, L.k_norm,
                        m->rope_cos, m->rope_sin, eps, kv2, 0, n};
            if ((e = launch_rope_append(s, ra, n)) != hipSuccess) return hip_fail(e, "NAR rope");
            FlashArgs fa{q, c->kv, c->capacity, l, Hq, Hkv, 0, n, 1.0f / std::sqrt((float)D), att, kv2, n,
                         visible, 1};
            if ((e = launch_flash(s, fa, D)) != hipSuccess) return hip_fail(e, "NAR attention");
            GemmArgs ga{att, qw, L.wo, nullptr, qw, x, nullptr, H, n, H, qw, nullptr};
            if ((e = launch_gemm(s, GEPI_RESID, ga)) != hipSuccess) return hip_fail(e, "NAR o");
            if ((e = launch_norm_rows(s, x, L.post_norm, h, n, H, eps)) != hipSuccess) return hip_fail(e, "NAR norm");
            GemmArgs gu{h, H, L.wg, L.wu, H, nullptr, act, I, n, I, H, nullptr};
            if ((e = launch_gemm(s, GEPI_SWIGLU_BF16, gu)) != hipSuccess) return hip_fail(e, "NAR gate/up");
            GemmArgs gd{act, I, L.wd, nullptr, I, x, nullptr, H, n, H, I, nullptr};
            if ((e = launch_gemm(s, GEPI_RESID, gd)) != hipSuccess) return hip_fail(e, "NAR down");
        }
        // llm2vae(final_norm(x)[1 .. n-1]) (:696-697)
        if ((e = launch_norm_rows(s, x + H, m->final_norm, h, frames, H, eps)) != hipSuccess)
            return hip_fail(e, "final norm");
        GemmArgs gl{h, H, nd.llm2vae, nullptr, H, d_out, nullptr, Lat, frames, Lat, H, nd.llm2vae_b};
        if ((e = launch_gemm(s, GEPI_BIAS, gl)) != hipSuccess) return hip_fail(e, "llm2vae");
        if ((e = hipMemcpyAsync(out, d_out, sizeof(float) * (size_t)frames * Lat, hipMemcpyDeviceToHost, s)) !=
            hipSuccess)
            return hip_fail(e, "velocity readback");
        if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "velocity");
        return YUE2_OK;
    };
    const int rc = run();
    (void)hipStreamSynchronize(s);
    (void)hipFree(block);
    return rc;
}

namespace {

// Generator::normal_tensor (src/sampling.rs:64-79): n uniform_f32 draws of
// MT19937(seed), then Box-Muller within each block of 16 (libm logf, sqrtf,
// cosf, sinf in f32; the angle 2 pi u in f64).  Host work in the reference.
void normal_tensor(uint64_t seed, size_t n, float* out) {
    uint32_t st[624];
    st[0] = (uint32_t)seed;
    for (int i = 1; i < 624; ++i) st[i] = 1812433253u * (st[i - 1] ^ (st[i - 1] >> 30)) + (uint32_t)i;
    int next = 624;
    auto draw = [&]() {
        if (next == 624) {
            for (int i = 0; i < 624; ++i) {
                const uint32_t bits = (st[i] & 0x80000000u) | (st[(i + 1) % 624] & 0x7fffffffu);
                st[i] = st[(i + 397) % 624] ^ (bits >> 1) ^ ((bits & 1u) ? 0x9908b0dfu : 0u);
            }
            next = 0;
        }
        uint32_t y = st[next++];
        y ^= y >> 11;
        y ^= (y << 7) & 0x9d2c5680u;
        y ^= (y << 15) & 0xefc60000u;
        y ^= y >> 18;
        return y;
    };
    for (size_t i = 0; i < n; ++i) out[i] = (float)(draw() & 0x00ffffffu) / 16777216.0f;
    for (size_t b = 0; b + 16 <= n; b += 16) {
        float* blk = out + b;
        for (int i = 0; i < 8; ++i) {
            const float radius = sqrtf(-2.0f * logf(1.0f - blk[i]));
            const float theta = (float)(2.0 * M_PI * (double)blk[i + 8]);
            blk[i] = radius * cosf(theta);
            blk[i + 8] = radius * sinf(theta);
        }
    }
}

// logit (src/model.rs:777-779)
double logit(double t) { return std::clamp(std::log(t / (1.0 - t)), -20.0, 20.0); }

}  // namespace

extern "C" int32_t yue2_hip_synthesize(Yue2Model* m, const int32_t* prefix, int32_t prefix_len, const int32_t* codec,
                                       int32_t codec_len, uint64_t seed, int32_t steps, float* out) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || (prefix_len > 0 && !prefix) || !codec || !out || prefix_len < 0)
        return fail(YUE2_ERR_ARG, "null model, ids or output");
    if (!m->nar.block) return fail(YUE2_ERR_ARG, "NAR weights not loaded");
    const int Lat = m->nar.latent;
    bool codec_ok = codec_len > 0 && steps > 0 && Lat == 64;
    for (int i = 0; codec_ok && i < codec_len; ++i) codec_ok = codec[i] >= 0 && codec[i] < kCodecSize;
    if (!codec_ok) return fail(YUE2_ERR_ARG, "Expected nonempty codec tokens and a 64-dimensional latent model");
    const int capacity = std::min(kContext, m->c.max_position_embeddings);
    if (capacity - prefix_len - 3 < 2) return fail(YUE2_ERR_CONTEXT, "Prefix leaves no acoustic context");
    const int size = (capacity - prefix_len - 3) / 2;
    // the whole song's noise once, sliced at the chunks (:724-726)
    std::vector<float> noise((size_t)codec_len * Lat), first((size_t)size * Lat), mid(first.size());
    normal_tensor(seed, noise.size(), noise.data());
    const float dt = 1.0f / (float)steps;
    std::vector<int32_t> ids;
    for (int start = 0; start < codec_len; start += size) {
        const int end = std::min(start + size, codec_len), frames = end - start;
        ids.assign(prefix, prefix + prefix_len);
        for (int i = start; i < end; ++i) ids.push_back(codec[i] + kCodecOffset);
        ids.push_back(kMusicEnd);
        Yue2Cache* cache = yue2_hip_cache_new(m, (int)ids.size());
        if (!cache) return YUE2_ERR_ALLOC;
        int rc = yue2_hip_prefill_mfma(m, cache, ids.data(), (int)ids.size(), YUE2_PHASE_NONE, nullptr);
        float* state = out + (size_t)start * Lat;
        for (size_t i = 0; i < (size_t)frames * Lat; ++i) state[i] = rb(noise[(size_t)start * Lat + i]);
        // the midpoint steps (:745-758)
        for (int step = 0; step < steps && rc == YUE2_OK; ++step) {
            const double t = 1.0 - (double)step / (double)steps;
            rc = yue2_hip_velocity(m, cache, state, frames, logit(t), 0, first.data());
            if (rc) break;
            for (size_t i = 0; i < (size_t)frames * Lat; ++i) mid[i] = rb(state[i] - rb(first[i] * (dt / 2.0f)));
            rc = yue2_hip_velocity(m, cache, mid.data(), frames, logit(t - 0.5 / (double)steps), 0, first.data());
            if (rc) break;
            for (size_t i = 0; i < (size_t)frames * Lat; ++i) state[i] = rb(state[i] - rb(first[i] * dt));
        }
        yue2_hip_cache_free(cache);
        if (rc) return rc;
        for (size_t i = 0; i < (size_t)frames * Lat; ++i)
            if (!std::isfinite(state[i])) return fail(YUE2_ERR_LOGITS, "Flow matching produced nonfinite latents");
    }
    return YUE2_OK;
}
