// decoder.hip -- the captured token loop of sampling::generate
// (src/sampling.rs:222-294) on the device.
//
// The loop's first choose() (over the prefill logits) runs when the decoder
// starts; after that one hipGraph launch forwards the chosen token and
// chooses the next one: embed -> every layer for every row -> LM head ->
// CFG mix + choose() -> advance the device positions.  So the token a run
// returns last has already been chosen when the run ends, and its forward is
// the next run's first launch.
//  * Fused: where the persistent step kernel serves the shape and the
//    sampler settings fit its candidate lists, the graph is that one kernel:
//    its last workgroup generates the token's 2 * vocab MT19937 outputs and
//    finishes choose() while the other workgroups run the layers and score
//    their rows of the LM head (step.hip).
//  * Otherwise the forward (step kernel or per-phase kernels) is followed by
//    the sampler kernels of sampler.hip and an advance kernel, and a side
//    branch of the same graph generates the draws while the layers run.
// Positions, ids, the step counter and the penalty history live in device
// memory, so the graph replays without parameter updates and only the
// chosen ids are copied back.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/yue2_hip.h"
#include "kernels.h"
#include "runtime.h"
#include "sampler.h"
#include "step.h"
#include "y2_math.h"

using namespace y2;

struct Yue2Decoder {
    Yue2Model* m = nullptr;
    Yue2Cache* caches[kMaxRows] = {nullptr, nullptr};
    int rows = 1, phase = YUE2_PHASE_NONE;
    bool need_rng = false;
    Workspace w;
    SampleArgs sa{};
    MtState* mt = nullptr;
    uint32_t* streams = nullptr;
    void* cand = nullptr;  // chunked choose(): candidate lists and chunk totals
    void* big = nullptr;   // choose(): survivors beyond the LDS capacity
    void* fcand = nullptr; // fused sampler: the workers' candidate lists
    bool fused = false;    // choose() inside the step kernel
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool started = false;
    int steps_done = 0;
    bool ended = false;
    std::vector<hipEvent_t> events;
    uint64_t seed = 0;
};

// Sampling::validate (src/protocol.rs:191-207).
static int validate_sampling(const Yue2Sampling* s) {
    if (!s) return fail(YUE2_ERR_ARG, "null sampling");
    if (!std::isfinite(s->temperature) || !(s->temperature >= 0.0f && s->temperature <= 5.0f) ||
        !std::isfinite(s->top_p) || s->top_p <= 0.0f || s->top_p > 1.0f || s->top_k < 1 ||
        !std::isfinite(s->repetition_penalty) || s->repetition_penalty <= 0.0f ||
        s->penalty_window < 1 || s->penalty_window > 100 || s->min_tokens > s->max_tokens ||
        s->max_tokens < 1)
        return fail(YUE2_ERR_SAMPLING, "Invalid sampling configuration");
    return YUE2_OK;
}

extern "C" int32_t yue2_hip_sampling_validate(const Yue2Sampling* s) { return validate_sampling(s); }

// MT19937 seeding (src/sampling.rs:15-24).
static void mt_seed(MtState* out, uint64_t seed) {
    out->state[0] = (uint32_t)seed;
    for (int i = 1; i < 624; ++i)
        out->state[i] = 1812433253u * (out->state[i - 1] ^ (out->state[i - 1] >> 30)) + (uint32_t)i;
    out->next = 624;
}

static KvView kv_view(const Yue2Decoder* d) {
    KvView kv{};
    for (int b = 0; b < d->rows; ++b) {
        kv.base[b] = d->caches[b]->kv;
        kv.capacity[b] = d->caches[b]->capacity;
    }
    return kv;
}

// The most keys a row attends in the decoder's next launch (its schedule,
// not its arithmetic, depends on it).
static int keys_now(const Yue2Decoder* d) {
    int n = 0;
    for (int b = 0; b < d->rows; ++b) n = std::max(n, d->caches[b]->length + 1);
    return n;
}

static void decoder_release(Yue2Decoder* d) {
    if (d->exec) (void)hipGraphExecDestroy(d->exec);
    if (d->graph) (void)hipGraphDestroy(d->graph);
    for (hipEvent_t e : d->events) (void)hipEventDestroy(e);
    if (d->fork) (void)hipEventDestroy(d->fork);
    if (d->join) (void)hipEventDestroy(d->join);
    if (d->side) (void)hipStreamDestroy(d->side);
    if (d->mt) (void)hipFree(d->mt);
    if (d->streams) (void)hipFree(d->streams);
    if (d->cand) (void)hipFree(d->cand);
    if (d->big) (void)hipFree(d->big);
    if (d->fcand) (void)hipFree(d->fcand);
    d->w.release();
}

extern "C" Yue2Decoder* yue2_hip_decoder_new(Yue2Model* m, Yue2Cache* cond, Yue2Cache* uncond,
                                             const Yue2Sampling* sampling, uint64_t seed,
                                             int32_t phase, float scale, int32_t legacy) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || !cond || cond->m != m || (uncond && uncond->m != m)) {
        fail(YUE2_ERR_ARG, "null or foreign model/cache");
        return nullptr;
    }
    if (sampling && validate_sampling(sampling) != YUE2_OK) return nullptr;
    if (check_phase_vocab(phase, m->c.vocab_size) != YUE2_OK) return nullptr;
    // The unconditional row is used only when guidance is on (src/sampling.rs:250-255).
    if (scale != 1.0f && !uncond) {
        fail(YUE2_ERR_GUIDANCE, "Guidance requires negative prefix");
        return nullptr;
    }
    auto* d = new Yue2Decoder();
    d->m = m;
    d->phase = phase;
    d->seed = seed;
    d->caches[0] = cond;
    d->rows = 1;
    if (scale != 1.0f) {
        d->caches[1] = uncond;
        d->rows = 2;
    }
    int cap = cond->capacity;
    if (d->rows == 2) cap = std::max(cap, uncond->capacity);
    const int V = m->c.vocab_size;
    int rc = d->w.ensure(d->rows, (cap + kBlockKeys - 1) / kBlockKeys, m->c);
    d->need_rng = sampling && sampling->temperature != 0.0f;
    hipError_t e = hipSuccess;
    if (rc == YUE2_OK && d->need_rng) {
        e = hipMalloc(&d->mt, sizeof(MtState));
        if (e == hipSuccess) e = hipMalloc(&d->streams, sizeof(uint32_t) * 4 * (size_t)V);
        if (e == hipSuccess) {
            MtState host;
            mt_seed(&host, seed);
            e = hipMemcpy(d->mt, &host, sizeof(MtState), hipMemcpyHostToDevice);
        }
    }
    const int mode = sampling ? 1 : 0;
    const float temp = sampling ? sampling->temperature : 0.0f;
    const int list = choose_list_len(V, mode, temp, sampling ? sampling->top_k : 1);
    const int chunks = (V + kChooseChunk - 1) / kChooseChunk;
    if (rc == YUE2_OK && e == hipSuccess && list > 0)
        e = hipMalloc(&d->cand, sizeof(uint64_t) * (size_t)chunks * list + sizeof(int2) * chunks);
    if (rc == YUE2_OK && e == hipSuccess && d->need_rng) e = hipMalloc(&d->big, survivor_bytes(V));
    const int flist = (mode == 0 || temp == 0.0f) ? 1 : (sampling ? sampling->top_k : 1);
    int head_lo, head_n, head_stop;
    head_rows(phase, V, &head_lo, &head_n, &head_stop);
    d->fused = m->step_kernel &&
               fused_sampler_supported(m->c, d->rows, m->cus, mode, temp, sampling ? sampling->top_k : 1, head_n);
    if (rc == YUE2_OK && e == hipSuccess && d->fused)
        e = hipMalloc(&d->fcand, sizeof(uint64_t) * (size_t)(m->cus - 1) * flist);
    if (rc == YUE2_OK && e == hipSuccess) e = hipStreamCreateWithFlags(&d->side, hipStreamNonBlocking);
    if (rc == YUE2_OK && e == hipSuccess) e = hipEventCreateWithFlags(&d->fork, hipEventDisableTiming);
    if (rc == YUE2_OK && e == hipSuccess) e = hipEventCreateWithFlags(&d->join, hipEventDisableTiming);
    if (rc != YUE2_OK || e != hipSuccess) {
        if (e != hipSuccess) hip_fail(e, "decoder allocation");
        decoder_release(d);
        delete d;
        return nullptr;
    }
    SampleArgs& a = d->sa;
    a.logits = d->w.logits;
    a.scores = d->w.mixed;
    a.stream[0] = d->streams;
    a.stream[1] = d->streams ? d->streams + 2 * (size_t)V : nullptr;
    a.history = d->w.token_log;
    a.hist_len = -1;
    a.token_log = d->w.token_log;
    a.st = d->w.st;
    a.rows = d->rows;
    a.vocab = V;
    a.phase = phase;
    a.end_id = phase_end_id(phase);
    a.mode = mode;
    if (d->cand) {
        a.cand = static_cast<uint64_t*>(d->cand);
        a.meta = reinterpret_cast<int2*>(a.cand + (size_t)chunks * list);
        a.chunks = chunks;
        a.list = list;
    }
    if (d->big) set_survivor_buffers(a, d->big, V);
    a.cfg_scale = scale;
    a.legacy = legacy;
    if (sampling) {
        a.temperature = sampling->temperature;
        a.top_p = sampling->top_p;
        a.top_k = sampling->top_k;
        a.repetition_penalty = sampling->repetition_penalty;
        a.window = sampling->penalty_window;
        a.min_tokens = sampling->min_tokens;
    }
    // the graph's choose() picks the token after the one its launch forwards
    a.step_offset = 1;
    m->decoders.push_back(d);  // detached by the free of the model or of a cache
    rc = YUE2_OK;
    if (d->fused) {
        FusedSampler fs{};
        fs.a = a;
        fs.a.stream[0] = fs.a.stream[1] = d->streams;  // one token's draws per launch
        fs.mt = d->mt;
        fs.draws = d->streams;
        fs.cand = static_cast<uint64_t*>(d->fcand);
        fs.list = flist;
        rc = prepare_step(m, d->w, &fs);
        d->fused = rc == YUE2_OK;  // 1: no resident step kernel with a sampler workgroup
    }
    if (rc >= 0 && !d->fused && m->step_kernel) rc = prepare_step(m, d->w);
    if (rc < 0) {
        decoder_detach(d);
        delete d;
        return nullptr;
    }
    return d;
}

namespace y2 {
void decoder_detach(Yue2Decoder* d) {
    if (!d->m) return;
    decoder_release(d);
    auto& v = d->m->decoders;
    v.erase(std::remove(v.begin(), v.end(), d), v.end());
    d->m = nullptr;
    d->caches[0] = d->caches[1] = nullptr;
}

bool decoder_uses(const Yue2Decoder* d, const Yue2Cache* c) {
    return d->m && (d->caches[0] == c || (d->rows > 1 && d->caches[1] == c));
}
}  // namespace y2

// Legal in any order with the free of its model and caches: a decoder they
// detached holds no device objects any more.
extern "C" void yue2_hip_decoder_free(Yue2Decoder* d) {
    if (!d) return;
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (d->m) {
        (void)hipStreamSynchronize(d->m->stream);
        decoder_detach(d);
    }
    delete d;
}

static int check_attached(const Yue2Decoder* d) {
    return d->m ? YUE2_OK : fail(YUE2_ERR_ARG, "the decoder's model or cache was freed");
}

// Capture one loop iteration (forward -> choose -> advance) as a graph.
static int capture(Yue2Decoder* d) {
    Yue2Model* m = d->m;
    hipStream_t s = m->stream;
    const size_t draws = 2 * (size_t)m->c.vocab_size;
    hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
    int rc = YUE2_OK;
    if (d->fused) {
        rc = enqueue_step_fused(m, d->w, kv_view(d), d->rows, true, d->phase, s, nullptr, 0, 1, keys_now(d));
        if (rc == 1) rc = fail(YUE2_ERR_DEVICE, "fused step kernel unavailable");
    } else {
        if (d->need_rng) {
            (void)hipEventRecord(d->fork, s);
            (void)hipStreamWaitEvent(d->side, d->fork, 0);
            launch_mt_generate(d->side, d->mt, d->streams, d->streams + draws, draws, d->w.st, 1);
            (void)hipEventRecord(d->join, d->side);
        }
        rc = enqueue_step_fused(m, d->w, kv_view(d), d->rows, true, d->phase, s, nullptr, 0, 0, keys_now(d));
        if (rc == 1) rc = enqueue_step(m, d->w, kv_view(d), d->rows, true, d->phase, s);
        if (d->need_rng) (void)hipStreamWaitEvent(s, d->join, 0);
        launch_choose(s, d->sa);
        launch_advance(s, d->w.st, d->rows);
    }
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(s, &g);
    if (rc != YUE2_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    d->graph = g;
    e = hipGraphInstantiate(&d->exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    return YUE2_OK;
}

static int start(Yue2Decoder* d, const float* first_logits) {
    Yue2Model* m = d->m;
    hipStream_t s = m->stream;
    const size_t V = m->c.vocab_size;
    if (!first_logits) return fail(YUE2_ERR_ARG, "first logits required");
    hipError_t e = hipMemcpyAsync(d->w.logits, first_logits, sizeof(float) * V * d->rows,
                                  hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return hip_fail(e, "logits upload");
    d->w.reset(s);
    launch_set_state(s, d->w.st, d->rows, d->caches[0]->length,
                     d->rows > 1 ? d->caches[1]->length : 0, 0, 0);
    if (d->need_rng)
        launch_mt_generate(s, d->mt, d->streams, d->streams + 2 * V, 2 * V, d->w.st, 0);
    // the loop's first choose() (step 0), over the prefill logits
    SampleArgs first = d->sa;
    first.step_offset = 0;
    launch_choose(s, first);
    if (int rc = capture(d)) return rc;
    d->started = true;
    return YUE2_OK;
}

static int check_room(Yue2Decoder* d, int steps) {
    for (int b = 0; b < d->rows; ++b) {
        const Yue2Cache* c = d->caches[b];
        if (c->length + steps > c->capacity || c->length + steps > d->m->c.max_position_embeddings)
            return fail(YUE2_ERR_CONTEXT, "AR input exceeds cache/model context");
    }
    if (d->steps_done + steps + 1 > d->w.log_cap) return fail(YUE2_ERR_CONTEXT, "token log full");
    return YUE2_OK;
}

static int read_tokens(Yue2Decoder* d, int from, int n, int32_t* tokens) {
    if (n <= 0 || !tokens) return YUE2_OK;
    hipError_t e = hipMemcpy(tokens, d->w.token_log + from, sizeof(int32_t) * n, hipMemcpyDeviceToHost);
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "token readback");
}

extern "C" int32_t yue2_hip_decoder_run(Yue2Decoder* d, const float* first_logits, int32_t steps,
                                        int32_t* tokens, float* step_ms) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!d || steps < 0) return fail(YUE2_ERR_ARG, "null decoder or negative steps");
    if (int rc = check_attached(d)) return rc;
    if (d->ended || steps == 0) return 0;
    if (int rc = check_room(d, steps)) return rc;
    hipStream_t s = d->m->stream;
    d->w.reserve_launches(s, steps);
    if (!d->started)
        if (int rc = start(d, first_logits)) return rc;
    if (step_ms && (int)d->events.size() < 2 * steps) {
        while ((int)d->events.size() < 2 * steps) {
            hipEvent_t ev;
            if (hipEventCreate(&ev) != hipSuccess) return fail(YUE2_ERR_DEVICE, "hipEventCreate");
            d->events.push_back(ev);
        }
    }
    // Token steps_done + i is chosen before launch i forwards it.  Phases
    // with an end token stop at the first end id, which gets no forward
    // (src/sampling.rs:268-271).
    const int end = phase_end_id(d->phase);
    int launches = 0, ran = 0;
    for (int i = 0; i < steps; ++i) {
        if (end >= 0) {
            int32_t id = -1;
            if (int rc = read_step_error(d->w, s)) return rc;
            if (int rc = read_tokens(d, d->steps_done + i, 1, &id)) return rc;
            if (id == end) {
                d->ended = true;
                ran = i + 1;
                break;
            }
        }
        if (step_ms) (void)hipEventRecord(d->events[2 * i], s);
        hipError_t e = hipGraphLaunch(d->exec, s);
        if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
        if (step_ms) (void)hipEventRecord(d->events[2 * i + 1], s);
        ++launches;
    }
    if (!d->ended) ran = launches;
    if (int rc = read_step_error(d->w, s)) return rc;
    if (step_ms)
        for (int i = 0; i < launches; ++i)
            (void)hipEventElapsedTime(&step_ms[i], d->events[2 * i], d->events[2 * i + 1]);
    if (int rc = read_tokens(d, d->steps_done, ran, tokens)) return rc;
    for (int b = 0; b < d->rows; ++b) d->caches[b]->length += launches;
    d->steps_done += ran;
    return ran;
}

extern "C" int32_t yue2_hip_decoder_logits(Yue2Decoder* d, float* out) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!d || !out) return fail(YUE2_ERR_ARG, "null decoder or output");
    if (int rc = check_attached(d)) return rc;
    if (!d->started) return fail(YUE2_ERR_ARG, "decoder has not run");
    hipStream_t s = d->m->stream;
    hipError_t e = hipMemcpyAsync(out, d->w.logits, sizeof(float) * (size_t)d->rows * d->m->c.vocab_size,
                                  hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "logits readback");
}

// The token chosen after the last run (the loop's next token), without a
// forward (src/sampling.rs:281: the last step chooses but does not forward).
static int next_token(Yue2Decoder* d, const float* first_logits, int32_t* token) {
    if (!d->started)
        if (int rc = start(d, first_logits)) return rc;
    if (int rc = read_step_error(d->w, d->m->stream)) return rc;
    return read_tokens(d, d->steps_done, 1, token);
}

// The persistent step kernel of this decoder, launched `iters` times at the
// decoder's current position (every launch recomputes the same token: it
// rewrites the same K/V slots and logits, and the state is not advanced).
// bytes: every weight once, each row's K/V over its current context plus
// the new position, the embedding rows.
static int time_step_kernel(Yue2Decoder* d, int32_t iters, float* avg_ms, double* bytes) {
    Yue2Model* m = d->m;
    const Yue2Config& c = m->c;
    const int sample = d->fused ? 2 : 0;  // the fused sampler's work, nothing published
    if (!m->step_kernel || !step_supported(c, d->rows, m->cus - (sample ? 1 : 0)))
        return fail(YUE2_ERR_ARG, "the decoder does not run the step kernel");
    const double H = c.hidden_size, D = c.head_dim, I = c.intermediate_size, V = c.vocab_size;
    const double q = c.num_attention_heads * D, kv = c.num_key_value_heads * D, L = c.num_hidden_layers;
    // the LM head reads the phase's rows and its stop row (project_phase)
    int lo = 0, n = 0, stop = -1;
    head_rows(d->phase, (int)V, &lo, &n, &stop);
    const double head = 2.0 * H * (n + (stop >= 0 && (stop < lo || stop >= lo + n) ? 1.0 : 0.0));
    const double weights = L * (2.0 * (H * (q + 2.0 * kv) + q * H + 3.0 * H * I) + 4.0 * (2.0 * H + 2.0 * D)) +
                           head + 4.0 * H;
    double kvb = 0.0;
    for (int b = 0; b < d->rows; ++b) {
        // the timed launches write the new token's K/V at position `length`
        const Yue2Cache* ch = d->caches[b];
        if (ch->length >= ch->capacity || ch->length >= c.max_position_embeddings)
            return fail(YUE2_ERR_CONTEXT, "no free cache position to time the step kernel at");
        kvb += L * 2.0 * kv * 2.0 * (ch->length + 1) + 2.0 * H;
    }
    hipStream_t s = m->stream;
    d->w.reserve_launches(s, (int64_t)iters + 1);
    hipEvent_t b0, b1;
    if (hipEventCreate(&b0) != hipSuccess) return fail(YUE2_ERR_DEVICE, "hipEventCreate");
    if (hipEventCreate(&b1) != hipSuccess) {
        (void)hipEventDestroy(b0);
        return fail(YUE2_ERR_DEVICE, "hipEventCreate");
    }
    int rc = enqueue_step_fused(m, d->w, kv_view(d), d->rows, true, d->phase, s, nullptr, 0, sample,
                                keys_now(d));  // untimed
    if (rc == YUE2_OK) (void)hipEventRecord(b0, s);
    for (int i = 0; i < iters && rc == YUE2_OK; ++i)
        rc = enqueue_step_fused(m, d->w, kv_view(d), d->rows, true, d->phase, s, nullptr, 0, sample, keys_now(d));
    if (rc == YUE2_OK) {
        (void)hipEventRecord(b1, s);
        hipError_t e = hipEventSynchronize(b1);
        float ms = 0.0f;
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, b0, b1);
        if (e != hipSuccess) rc = hip_fail(e, "step kernel timing");
        *avg_ms = ms / (float)iters;
        *bytes = weights + kvb;
    } else if (rc > 0) {
        rc = fail(YUE2_ERR_ARG, "the decoder does not run the step kernel");
    }
    if (rc == YUE2_OK) rc = read_step_error(d->w, s);
    (void)hipEventDestroy(b0);
    (void)hipEventDestroy(b1);
    return rc;
}

extern "C" int32_t yue2_hip_decoder_time_kernel(Yue2Decoder* d, int32_t kernel, int32_t iters,
                                                float* avg_ms, double* bytes) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!d || !avg_ms || !bytes || iters <= 0 || kernel < 0 || kernel > 5)
        return fail(YUE2_ERR_ARG, "bad kernel timing request");
    if (int rc = check_attached(d)) return rc;
    if (!d->started) return fail(YUE2_ERR_ARG, "decoder has not run");
    Yue2Model* m = d->m;
    const Yue2Config& c = m->c;
    if (kernel == 5) return time_step_kernel(d, iters, avg_ms, bytes);
    const int H = c.hidden_size, D = c.head_dim, I = c.intermediate_size, V = c.vocab_size;
    const int qw = c.num_attention_heads * D, qkvw = qw + 2 * c.num_key_value_heads * D;
    const int rows = d->rows, L = c.num_hidden_layers;
    const size_t out_n = (size_t)rows * std::max(std::max(V, qkvw), std::max(I, H));
    float* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, out_n * sizeof(float));
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(timing)");
    hipEvent_t b0, b1;
    (void)hipEventCreate(&b0);
    (void)hipEventCreate(&b1);
    hipStream_t s = m->stream;
    auto args = [&](int l, int* epi) {
        const LayerDev& Lw = m->layers[l];
        switch (kernel) {
            case 0: *epi = EPI_SWIGLU; return GemvArgs{Lw.wg, Lw.wu, d->w.x, tmp, H, I, I, H, rows, Lw.post_norm, c.rms_norm_eps, nullptr};
            case 1: *epi = EPI_RESID; return GemvArgs{Lw.wd, nullptr, d->w.act, tmp, I, H, H, I, rows};
            case 2: *epi = EPI_STORE; return GemvArgs{Lw.wqkv, nullptr, d->w.x, tmp, H, qkvw, qkvw, H, rows, Lw.in_norm, c.rms_norm_eps, nullptr};
            case 3: *epi = EPI_RESID; return GemvArgs{Lw.wo, nullptr, d->w.att, tmp, qw, H, H, qw, rows};
            default: *epi = EPI_STORE; return GemvArgs{m->lm_head, nullptr, d->w.x, tmp, H, V, V, H, rows, m->final_norm, c.rms_norm_eps, nullptr};
        }
    };
    int rc = YUE2_OK;
    // one untimed pass over every layer, then the timed launches
    for (int i = 0; i < L + iters && rc == YUE2_OK; ++i) {
        if (i == L) (void)hipEventRecord(b0, s);
        int epi;
        const GemvArgs a = args(i % L, &epi);
        if ((e = launch_gemv(s, epi, a)) != hipSuccess) rc = hip_fail(e, "timed gemv");
    }
    (void)hipEventRecord(b1, s);
    if (rc == YUE2_OK && (e = hipEventSynchronize(b1)) != hipSuccess) rc = hip_fail(e, "timing sync");
    float ms = 0.0f;
    if (rc == YUE2_OK) (void)hipEventElapsedTime(&ms, b0, b1);
    *avg_ms = ms / (float)iters;
    const double w = 2.0, f = 4.0;
    switch (kernel) {
        case 0: *bytes = w * 2.0 * I * H + f * rows * (H + (double)I); break;
        case 1: *bytes = w * (double)H * I + f * rows * ((double)I + 2.0 * H); break;
        case 2: *bytes = w * (double)qkvw * H + f * rows * ((double)H + qkvw); break;
        case 3: *bytes = w * (double)H * qw + f * rows * ((double)qw + 2.0 * H); break;
        default: *bytes = w * (double)V * H + f * rows * ((double)H + V); break;
    }
    (void)hipEventDestroy(b0);
    (void)hipEventDestroy(b1);
    (void)hipFree(tmp);
    return rc;
}

// Device buffers of one choose() call, carved from one region: the step
// state, the logits, the tempered scores, the draws, the penalty window, the
// chunk candidate lists and totals, and the survivor overflow arrays.
struct ChooseLayout {
    size_t st, logits, scores, draws, hist, cand, meta, big, total;
    int list, chunks, hist_n;
};

static ChooseLayout choose_layout(int vocab, const Yue2Sampling* sampling, int history_len) {
    ChooseLayout L{};
    const bool rng = sampling->temperature != 0.0f;
    L.list = choose_list_len(vocab, 1, sampling->temperature, sampling->top_k);
    L.chunks = (vocab + kChooseChunk - 1) / kChooseChunk;
    // only the last penalty_window ids of the history are read (:130-131)
    L.hist_n = std::min(history_len, sampling->penalty_window);
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t o = at;
        at = (at + bytes + 255) / 256 * 256;
        return o;
    };
    const size_t V = vocab;
    L.st = take(sizeof(StepState));
    L.logits = take(sizeof(float) * V);
    L.scores = take(sizeof(float) * V);
    L.draws = take(rng ? sizeof(uint32_t) * 2 * V : 0);
    L.hist = take(sizeof(int32_t) * std::max(L.hist_n, 1));
    L.cand = take(L.list > 0 ? sizeof(uint64_t) * (size_t)L.chunks * L.list : 0);
    L.meta = take(L.list > 0 ? sizeof(int2) * L.chunks : 0);
    L.big = take(rng ? survivor_bytes(vocab) : 0);
    L.total = at;
    return L;
}

// One choose() in the region p (laid out by L) on stream s: inputs copied in,
// the kernels, the chosen id copied out.  Every field the kernels read before
// writing is written here first (the step state in full), so p may hold
// anything on entry.
static int choose_run(char* p, const ChooseLayout& L, hipStream_t s, const float* logits, int32_t vocab,
                      const Yue2Sampling* sampling, const int32_t* history, int32_t history_len,
                      int32_t step, int32_t phase, int32_t legacy, const uint32_t* draws, int32_t* id) {
    const bool rng = sampling->temperature != 0.0f;
    const size_t V = vocab;
    StepState st{};
    st.step = step;
    hipError_t e = hipMemcpyAsync(p + L.st, &st, sizeof(st), hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(p + L.logits, logits, sizeof(float) * V, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && rng)
        e = hipMemcpyAsync(p + L.draws, draws, sizeof(uint32_t) * 2 * V, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && L.hist_n > 0)
        e = hipMemcpyAsync(p + L.hist, history + (history_len - L.hist_n), sizeof(int32_t) * L.hist_n,
                           hipMemcpyHostToDevice, s);
    if (e == hipSuccess) {
        SampleArgs a{};
        a.logits = reinterpret_cast<const float*>(p + L.logits);
        a.scores = reinterpret_cast<float*>(p + L.scores);
        a.stream[0] = a.stream[1] = rng ? reinterpret_cast<const uint32_t*>(p + L.draws) : nullptr;
        a.history = reinterpret_cast<const int32_t*>(p + L.hist);
        a.hist_len = L.hist_n;
        a.token_log = nullptr;
        a.st = reinterpret_cast<StepState*>(p + L.st);
        a.rows = 1;
        a.vocab = vocab;
        a.phase = phase;
        a.end_id = phase_end_id(phase);
        a.mode = 1;
        a.cfg_scale = 1.0f;
        a.temperature = sampling->temperature;
        a.top_p = sampling->top_p;
        a.top_k = sampling->top_k;
        a.repetition_penalty = sampling->repetition_penalty;
        a.window = sampling->penalty_window;
        a.min_tokens = sampling->min_tokens;
        a.legacy = legacy;
        if (L.list > 0) {
            a.cand = reinterpret_cast<uint64_t*>(p + L.cand);
            a.meta = reinterpret_cast<int2*>(p + L.meta);
            a.chunks = L.chunks;
            a.list = L.list;
        }
        if (rng) set_survivor_buffers(a, p + L.big, vocab);
        launch_choose(s, a);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpyAsync(&st, p + L.st, sizeof(st), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        // nothing enqueued may still run over p when the caller reuses it
        // (the allocation-free entry's shared scratch)
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "choose");
    }
    if (int rc = step_error(st)) return rc;
    *id = st.ids[0];
    return YUE2_OK;
}

static int choose_check(const float* logits, int32_t vocab, const Yue2Sampling* sampling, const int32_t* history,
                        int32_t history_len, int32_t step, int32_t phase, const uint32_t* draws, int32_t* id) {
    if (!logits || !id || vocab < 1 || history_len < 0 || step < 0 || (history_len > 0 && !history))
        return fail(YUE2_ERR_ARG, "bad choose arguments");
    if (int rc = validate_sampling(sampling)) return rc;
    if (int rc = check_phase_vocab(phase, vocab)) return rc;
    if (sampling->temperature != 0.0f && !draws) return fail(YUE2_ERR_ARG, "choose needs 2 * vocab draws");
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no gfx950 HIP device");
    return YUE2_OK;
}

// sampling::choose (src/sampling.rs:103-215) for one row of logits.
extern "C" int32_t yue2_hip_choose(const float* logits, int32_t vocab, const Yue2Sampling* sampling,
                                   const int32_t* history, int32_t history_len, int32_t step,
                                   int32_t phase, int32_t legacy, const uint32_t* draws,
                                   int32_t* id) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (int rc = choose_check(logits, vocab, sampling, history, history_len, step, phase, draws, id)) return rc;
    const ChooseLayout L = choose_layout(vocab, sampling, history_len);
    char* p = nullptr;
    hipError_t e = hipMalloc(&p, L.total);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(choose)");
    hipStream_t s = nullptr;
    e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    int rc = e == hipSuccess ? choose_run(p, L, s, logits, vocab, sampling, history, history_len, step, phase,
                                          legacy, draws, id)
                             : hip_fail(e, "hipStreamCreate(choose)");
    if (s) (void)hipStreamDestroy(s);
    (void)hipFree(p);
    return rc;
}

// ---- choose() without allocation -------------------------------------------
//
// The scratch of yue2_hip_choose_noalloc: one region per device, laid out by
// choose_layout for each call.  Its size covers a vocabulary of
// kNoAllocVocabMax entries with any sampling settings.  In host code the
// array's name stands for nothing usable: the device address comes from
// hipGetSymbolAddress, once per device, and only that address is used.
constexpr int kNoAllocVocabMax = 262144;
constexpr size_t kNoAllocScratchBytes = 9u << 20;  // 8.13 MiB at 262144 entries
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
constexpr int kNoAllocDevices = 64;
static char* g_scratch_dev[kNoAllocDevices];

// The scratch address on the current device (resolved on its first use).
static int noalloc_scratch(char** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kNoAllocDevices) return fail(YUE2_ERR_DEVICE, "device index beyond the scratch table");
    if (!g_scratch_dev[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) return hip_fail(e, "hipGetSymbolAddress(choose scratch)");
        g_scratch_dev[dev] = static_cast<char*>(ptr);
    }
    *out = g_scratch_dev[dev];
    return YUE2_OK;
}

extern "C" int32_t yue2_hip_choose_noalloc(const float* logits, int32_t vocab, const Yue2Sampling* sampling,
                                           const int32_t* history, int32_t history_len, int32_t step,
                                           int32_t phase, int32_t legacy, const uint32_t* draws, int32_t* id) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (int rc = choose_check(logits, vocab, sampling, history, history_len, step, phase, draws, id)) return rc;
    if (vocab > kNoAllocVocabMax)
        return fail(YUE2_ERR_ARG, "vocabulary above the allocation-free choose() limit of 262144 entries");
    const ChooseLayout L = choose_layout(vocab, sampling, history_len);
    if (L.total > kNoAllocScratchBytes)
        return fail(YUE2_ERR_ARG, "choose() request larger than the allocation-free scratch");
    char* p = nullptr;
    if (int rc = noalloc_scratch(&p)) return rc;
    // the null stream: creating one of our own would allocate
    return choose_run(p, L, nullptr, logits, vocab, sampling, history, history_len, step, phase, legacy, draws,
                      id);
}

extern "C" int32_t yue2_hip_generate(Yue2Model* m, const int32_t* prefix, int32_t prefix_len,
                                     const Yue2Sampling* sampling, uint64_t seed, int32_t phase,
                                     const int32_t* negative, int32_t negative_len, float scale,
                                     int32_t legacy, int32_t* tokens, int32_t* count,
                                     int32_t* truncated) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || !sampling || !tokens || !count || !truncated) return fail(YUE2_ERR_ARG, "null argument");
    if (int rc = validate_sampling(sampling)) return rc;
    if (prefix_len + sampling->max_tokens > kContext ||
        (negative && negative_len + sampling->max_tokens > kContext))
        return fail(YUE2_ERR_BUDGET, "Prefix + requested generation budget exceeds 24576; no implicit truncation");
    if (scale != 1.0f && !negative) return fail(YUE2_ERR_GUIDANCE, "Guidance requires negative prefix");
    if (int rc = check_phase_vocab(phase, m->c.vocab_size)) return rc;
    if (prefix_len <= 0 || (scale != 1.0f && negative_len <= 0)) return fail(YUE2_ERR_ARG, "Empty prefill");
    *count = 0;
    *truncated = 1;
    const size_t V = m->c.vocab_size;
    std::vector<float> first(V * 2);
    Yue2Cache* cond = yue2_hip_cache_new(m, prefix_len + sampling->max_tokens);
    Yue2Cache* neg = nullptr;
    Yue2Decoder* d = nullptr;
    int rc = cond ? YUE2_OK : YUE2_ERR_ALLOC;
    // prefill_phase of both rows (src/sampling.rs:246, 252): decode order
    // (bit-exact with the CPU path) or the matrix cores (the reference's own
    // GPU prefill, src/tensor.rs:991-993), as yue2_hip_model_set_prefill chose
    auto prefill = m->prefill_mfma ? yue2_hip_prefill_mfma : yue2_hip_prefill;
    if (rc == YUE2_OK) rc = prefill(m, cond, prefix, prefix_len, phase, first.data());
    if (rc == YUE2_OK && scale != 1.0f) {
        neg = yue2_hip_cache_new(m, negative_len + sampling->max_tokens);
        rc = neg ? YUE2_OK : YUE2_ERR_ALLOC;
        if (rc == YUE2_OK) rc = prefill(m, neg, negative, negative_len, phase, first.data() + V);
    }
    if (rc == YUE2_OK) {
        d = yue2_hip_decoder_new(m, cond, neg, sampling, seed, phase, scale, legacy);
        if (!d) rc = YUE2_ERR_ALLOC;
    }
    const int end = phase_end_id(phase);
    if (rc == YUE2_OK) {
        const int loop = sampling->max_tokens - 1;
        int ran = loop > 0 ? yue2_hip_decoder_run(d, first.data(), loop, tokens, nullptr) : 0;
        if (ran < 0) rc = ran;
        if (rc == YUE2_OK) {
            if (d->ended) {
                *count = ran - 1;  // the end id is not pushed (:268-271)
                *truncated = 0;
            } else {
                int32_t last = -1;
                rc = next_token(d, first.data(), &last);
                if (rc == YUE2_OK) {
                    if (last == end) {
                        *count = ran;
                        *truncated = 0;
                    } else {
                        tokens[ran] = last;
                        *count = ran + 1;
                    }
                }
            }
        }
    }
    if (d) yue2_hip_decoder_free(d);
    yue2_hip_cache_free(neg);
    yue2_hip_cache_free(cond);
    return rc;
}
