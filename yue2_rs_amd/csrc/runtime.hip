// runtime.hip -- device-resident model, KV caches and the captured token step
// behind the session half of include/yue2_hip.h.
//
// Model::open / Cache::new / forward_phase / prefill_phase / generate of the
// reference (src/model.rs:292-610, src/sampling.rs:222-294) become: weights
// uploaded once into one HBM allocation; BF16 KV caches in HBM; a workspace
// per batch size; and a token step that is enqueued either directly (parity
// API) or captured once as a hipGraph and replayed (decoder).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/yue2_hip.h"
#include "kernels.h"
#include "runtime.h"
#include "step.h"
#include "y2_math.h"

using namespace y2;

namespace y2 {

std::recursive_mutex& library_lock() {
    static std::recursive_mutex m;
    return m;
}

static thread_local std::string t_error;

int fail(int code, const std::string& msg) {
    t_error = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(YUE2_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

bool device_ready() {
    static int state = -1;  // -1 unknown, 0 no, 1 yes
    if (state < 0) {
        int count = 0;
        state = 0;
        if (hipGetDeviceCount(&count) == hipSuccess && count > 0) {
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, 0) == hipSuccess &&
                std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 && hipSetDevice(0) == hipSuccess)
                state = 1;
        }
    }
    return state == 1;
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Bump allocator over one device allocation.
struct Carve {
    size_t offset = 0;
    template <typename T>
    size_t take(size_t count) {
        const size_t at = offset;
        offset = align_up(offset + count * sizeof(T), 256);
        return at;
    }
};

// Word counts of the tagged-word buffers (flow_block, in this order): the
// step kernel's exchanges, and the block maxima, sums and partials that the
// step kernel and the per-phase attention both use.
struct FlowLayout {
    size_t x, qkv, att, act, blk, part, smp;
    FlowLayout(const Yue2Config& c, int rows, int blk_stride) {
        const size_t D = c.head_dim, Hq = c.num_attention_heads, Hkv = c.num_key_value_heads;
        x = rows * (size_t)c.hidden_size;
        qkv = rows * (Hq + 2 * Hkv) * D;
        att = rows * Hq * D;
        act = rows * (size_t)c.intermediate_size;
        blk = rows * Hq * (size_t)blk_stride;
        part = blk * D;
        smp = kStepThreadsMax;  // one sampler word per worker
    }
    size_t total() const { return x + qkv + att + act + 2 * blk + part + smp; }
    size_t bmax() const { return x + qkv + att + act; }
    size_t bsum() const { return bmax() + blk; }
    size_t part_at() const { return bsum() + blk; }
    size_t smp_at() const { return part_at() + part; }
};

int Workspace::ensure(int want_rows, int want_blocks, const Yue2Config& c) {
    if (block && rows == want_rows && max_blocks >= want_blocks) return YUE2_OK;
    release();
    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_attention_heads;
    const int Hkv = c.num_key_value_heads, I = c.intermediate_size, V = c.vocab_size;
    const int qkvw = (Hq + 2 * Hkv) * D;
    rows = want_rows;
    max_blocks = want_blocks;
    blk_stride = max_blocks;
    log_cap = 24576 + 64;
    Carve cv;
    const size_t o_x = cv.take<float>((size_t)rows * H);
    const size_t o_h = cv.take<float>((size_t)rows * H);
    const size_t o_qkv = cv.take<float>((size_t)rows * qkvw);
    const size_t o_att = cv.take<float>((size_t)rows * Hq * D);
    const size_t o_act = cv.take<float>((size_t)rows * I);
    const size_t o_logits = cv.take<float>((size_t)rows * V);
    const size_t o_mixed = cv.take<float>((size_t)V);
    const size_t o_counters = cv.take<int32_t>((size_t)rows * Hkv * 4);
    const size_t o_bars = cv.take<int32_t>(2);
    const size_t o_bmax = cv.take<float>((size_t)rows * Hq * blk_stride);
    const size_t o_bsum = cv.take<float>((size_t)rows * Hq * blk_stride);
    const size_t o_part = cv.take<float>((size_t)rows * Hq * blk_stride * D);
    const size_t o_st = cv.take<StepState>(1);
    const size_t o_log = cv.take<int32_t>((size_t)log_cap);
    const size_t o_args = cv.take<StepArgs>(1);
    hipError_t e = hipMalloc(&block, cv.offset);
    if (e != hipSuccess) {
        block = nullptr;
        return hip_fail(e, "hipMalloc(workspace)");
    }
    char* p = static_cast<char*>(block);
    x = reinterpret_cast<float*>(p + o_x);
    h = reinterpret_cast<float*>(p + o_h);
    qkv = reinterpret_cast<float*>(p + o_qkv);
    att = reinterpret_cast<float*>(p + o_att);
    act = reinterpret_cast<float*>(p + o_act);
    logits = reinterpret_cast<float*>(p + o_logits);
    mixed = reinterpret_cast<float*>(p + o_mixed);
    counters = reinterpret_cast<int32_t*>(p + o_counters);
    bars = reinterpret_cast<int32_t*>(p + o_bars);
    bmax = reinterpret_cast<float*>(p + o_bmax);
    bsum = reinterpret_cast<float*>(p + o_bsum);
    part = reinterpret_cast<float*>(p + o_part);
    st = reinterpret_cast<StepState*>(p + o_st);
    token_log = reinterpret_cast<int32_t*>(p + o_log);
    step_args = p + o_args;
    step_args_ready = false;
    if (!step_host) step_host = new StepArgs{};
    e = hipMemset(st, 0, sizeof(StepState));
    counter_n = rows * Hkv * 4;
    if (e == hipSuccess) e = hipMemset(counters, 0, sizeof(int32_t) * rows * Hkv * 4);
    if (e == hipSuccess) e = hipMemset(bars, 0, sizeof(int32_t) * 2);
    if (e != hipSuccess) return hip_fail(e, "hipMemset(step state)");
    // tagged words, zero (= no tag) until first written; the sequence (in
    // the cleared state) starts at 0 with them
    const FlowLayout fl(c, rows, blk_stride);
    const size_t words = fl.total();
    e = hipMalloc(&flow_block, words * sizeof(uint64_t));
    if (e != hipSuccess) {
        flow_block = nullptr;
        return hip_fail(e, "hipMalloc(dataflow words)");
    }
    e = hipMemset(flow_block, 0, words * sizeof(uint64_t));
    if (e != hipSuccess) return hip_fail(e, "hipMemset(dataflow words)");
    flow_words = words;
    seq_bound = 0;
    uint64_t* fw = static_cast<uint64_t*>(flow_block);
    tbmax = fw + fl.bmax();
    tbsum = fw + fl.bsum();
    tpart = fw + fl.part_at();
    return YUE2_OK;
}

void Workspace::reserve_launches(hipStream_t s, int64_t n) {
    if (!flow_block) return;  // not allocated yet: no tagged words
    if (seq_bound + n + 2 + 8 < kEpochLaunches) {
        seq_bound += n;
        return;
    }
    launch_fill(s, static_cast<float*>(flow_block), 2 * flow_words, 0.0f);  // tag 0 matches no poll
    launch_sequence(s, st, 1, 0);
    seq_bound = n;
}

void Workspace::release() {
    if (block) (void)hipFree(block);
    if (flow_block) (void)hipFree(flow_block);
    block = nullptr;
    flow_block = nullptr;
    flow_words = 0;
    seq_bound = 0;
    tbmax = tbsum = tpart = nullptr;
    step_args = nullptr;
    step_args_ready = false;
    rows = max_blocks = 0;
}

Workspace::~Workspace() {
    release();
    delete static_cast<StepArgs*>(step_host);
}

// Enqueue one token step for `rows` batch rows reading ids/positions from the
// workspace's StepState.  head: 0 none, else the phase's LM head.
int enqueue_step(Yue2Model* m, Workspace& w, const KvView& kv, int rows, bool head, int phase,
                 hipStream_t s) {
    const Yue2Config& c = m->c;
    const int H = c.hidden_size, D = c.head_dim, Hq = c.num_attention_heads;
    const int Hkv = c.num_key_value_heads, I = c.intermediate_size, V = c.vocab_size;
    const int qkvw = (Hq + 2 * Hkv) * D, qw = Hq * D;
    const float eps = c.rms_norm_eps;
    hipError_t e;
    launch_embed(s, m->embed, w.st, w.x, H, V, rows);
    for (int l = 0; l < c.num_hidden_layers; ++l) {
        const LayerDev& L = m->layers[l];
        // RMSNorm(x) is computed in the GEMV prologue of every workgroup.
        GemvArgs qa{L.wqkv, nullptr, w.x, w.qkv, H, qkvw, qkvw, H, rows, L.in_norm, eps, w.st};
        if ((e = launch_gemv(s, EPI_STORE, qa)) != hipSuccess) return hip_fail(e, "gemv(qkv)");
        // QK-norm + RoPE + KV append + attention: one kernel.
        AttnArgs aa{};
        aa.qkv = w.qkv;
        aa.qkv_stride = qkvw;
        aa.kv = kv;
        aa.layer = l;
        aa.heads = Hq;
        aa.kv_heads = Hkv;
        aa.dim = D;
        aa.rows = rows;
        aa.scale = 1.0f / std::sqrt((float)D);
        aa.eps = eps;
        aa.q_norm = L.q_norm;
        aa.k_norm = L.k_norm;
        aa.cos_t = m->rope_cos;
        aa.sin_t = m->rope_sin;
        aa.bmax = w.bmax;
        aa.bsum = w.bsum;
        aa.part = w.part;
        aa.out = w.att;
        aa.out_stride = qw;
        aa.blk_stride = w.blk_stride;
        attention_geometry(Hkv, rows, w.max_blocks, &aa.wgs, &aa.bpw);
        aa.counters = w.counters;
        aa.st = w.st;
        // the tagged-word attention where the shape allows; its tags take the
        // sequence, which advances after the step
        aa.tbmax = w.tbmax;
        aa.tbsum = w.tbsum;
        aa.tpart = w.tpart;
        if ((e = launch_attention(s, aa)) != hipSuccess) return hip_fail(e, "attention");
        GemvArgs oa{L.wo, nullptr, w.att, w.x, qw, H, H, qw, rows};
        if ((e = launch_gemv(s, EPI_RESID, oa)) != hipSuccess) return hip_fail(e, "gemv(o)");
        GemvArgs ga{L.wg, L.wu, w.x, w.act, H, I, I, H, rows, L.post_norm, eps, w.st};
        if ((e = launch_gemv(s, EPI_SWIGLU, ga)) != hipSuccess) return hip_fail(e, "gemv(gate/up)");
        GemvArgs da{L.wd, nullptr, w.act, w.x, I, H, H, I, rows};
        if ((e = launch_gemv(s, EPI_RESID, da)) != hipSuccess) return hip_fail(e, "gemv(down)");
    }
    // the next step's tags (one sequence value per step, as a step-kernel
    // launch takes; the callers reserve one per step)
    launch_sequence(s, w.st, 0, 1);
    if (!head) return YUE2_OK;
    return enqueue_head(m, w, w.x, phase, s, rows);
}

int enqueue_head(Yue2Model* m, Workspace& w, const float* x, int phase, hipStream_t s, int rows) {
    const Yue2Config& c = m->c;
    const int H = c.hidden_size, V = c.vocab_size;
    const float eps = c.rms_norm_eps;
    hipError_t e;
    // final_norm (src/model.rs:590) runs in the LM-head GEMV prologue.
    if (phase == YUE2_PHASE_NONE) {
        GemvArgs la{m->lm_head, nullptr, x, w.logits, H, V, V, H, rows, m->final_norm, eps, w.st};
        if ((e = launch_gemv(s, EPI_STORE, la)) != hipSuccess) return hip_fail(e, "gemv(lm_head)");
        return YUE2_OK;
    }
    // project_phase (src/model.rs:478-507): the phase's rows plus the stop
    // row; every other logit is -inf.
    int start, end, stop;
    phase_range(phase, &start, &end, &stop);
    launch_fill(s, w.logits, (size_t)rows * V, -INFINITY);
    GemvArgs ra{m->lm_head + (size_t)start * H, nullptr, x, w.logits + start, H, V, end - start, H, rows,
                m->final_norm, eps, w.st};
    if ((e = launch_gemv(s, EPI_STORE, ra)) != hipSuccess) return hip_fail(e, "gemv(lm_head range)");
    GemvArgs sa{m->lm_head + (size_t)stop * H, nullptr, x, w.logits + stop, H, V, 1, H, rows,
                m->final_norm, eps, nullptr};
    if ((e = launch_gemv(s, EPI_STORE, sa)) != hipSuccess) return hip_fail(e, "gemv(lm_head stop)");
    return YUE2_OK;
}

int prepare_step(Yue2Model* m, Workspace& w, const FusedSampler* smp) {
    const Yue2Config& c = m->c;
    const int rows = w.rows, sample = smp ? 1 : 0;
    if (!step_supported(c, rows, m->cus - sample)) return 1;
    if (w.step_args_ready && w.step_sample == sample) return YUE2_OK;
    const int D = c.head_dim, Hq = c.num_attention_heads, Hkv = c.num_key_value_heads;
    const int H = c.hidden_size, I = c.intermediate_size;
    StepArgs a{};
    a.layers = m->layers_dev;
    a.embed = m->embed;
    a.lm_head = m->lm_head;
    a.final_norm = m->final_norm;
    a.rope_cos = m->rope_cos;
    a.rope_sin = m->rope_sin;
    a.layers_n = c.num_hidden_layers;
    a.hidden = H;
    a.intermediate = I;
    a.vocab = c.vocab_size;
    a.heads = Hq;
    a.kv_heads = Hkv;
    a.head_dim = D;
    a.rows = rows;
    a.blk_stride = w.blk_stride;
    a.max_blocks = w.max_blocks;
    a.eps = c.rms_norm_eps;
    a.scale = 1.0f / std::sqrt((float)D);
    a.logits = w.logits;
    a.st = w.st;
    if (smp) a.smp = *smp;
    if (step_launch_lds(a, m->cus, sample) > kStepLdsMax) return 1;
    // one workgroup per CU, all resident together: the polls between them
    // would otherwise wait for a workgroup that cannot start
    if (step_resident_per_cu(a, m->cus, sample) < 1) return 1;
    // the tagged-word buffers (allocated and cleared with the workspace)
    if (!w.flow_block) return fail(YUE2_ERR_DEVICE, "no dataflow words");
    const FlowLayout fl(c, rows, w.blk_stride);
    uint64_t* p = static_cast<uint64_t*>(w.flow_block);
    a.tx = p;
    a.tqkv = a.tx + fl.x;
    a.tatt = a.tqkv + fl.qkv;
    a.tact = a.tatt + fl.att;
    a.tbmax = p + fl.bmax();
    a.tbsum = p + fl.bsum();
    a.tpart = p + fl.part_at();
    a.tsmp = p + fl.smp_at();
    hipError_t e = hipMemcpy(w.step_args, &a, sizeof(StepArgs), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "step arguments upload");
    *reinterpret_cast<StepArgs*>(w.step_host) = a;
    w.step_args_ready = true;
    w.step_sample = sample;
    return YUE2_OK;
}

int enqueue_step_fused(Yue2Model* m, Workspace& w, const KvView& kv, int rows, bool head, int phase,
                       hipStream_t s, unsigned long long* trace, int trace_slots, int sample, int context) {
    if (!trace && !m->step_kernel) return 1;
    if (!w.step_args_ready || (sample != 0) != (w.step_sample != 0)) return 1;  // not prepared for this call
    if (rows != w.rows || !step_supported(m->c, rows, m->cus - (sample ? 1 : 0))) return 1;
    StepCall call{};
    call.kv = kv;
    call.head = head ? 1 : 0;
    head_rows(phase, m->c.vocab_size, &call.head_lo, &call.head_n, &call.head_stop);
    call.sample = sample;
    call.context = context;
    call.trace = trace;
    call.trace_slots = trace ? trace_slots : 0;
    hipError_t e = launch_step(s, static_cast<const StepArgs*>(w.step_args),
                               *reinterpret_cast<const StepArgs*>(w.step_host), call, m->cus);
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "step kernel");
}

void phase_range(int phase, int* start, int* end, int* stop) {
    if (phase == YUE2_PHASE_ABC) {
        *start = 0;
        *end = kEod;
        *stop = kAbcEnd;
    } else {
        *start = kCodecOffset;
        *end = kCodecOffset + kCodecSize;
        *stop = kMusicEnd;
    }
}

void head_rows(int phase, int vocab, int* lo, int* n, int* stop) {
    if (phase == YUE2_PHASE_NONE) {
        *lo = 0;
        *n = vocab;
        *stop = -1;
        return;
    }
    int end;
    phase_range(phase, lo, &end, stop);
    *n = end - *lo;
}

int phase_end_id(int phase) {
    return phase == YUE2_PHASE_ABC ? kAbcEnd : phase == YUE2_PHASE_SEMANTIC ? kMusicEnd : -1;
}

int check_phase_vocab(int phase, int vocab) {
    if (phase == YUE2_PHASE_NONE) return YUE2_OK;
    if (phase != YUE2_PHASE_ABC && phase != YUE2_PHASE_SEMANTIC) return fail(YUE2_ERR_ARG, "unknown phase");
    int start, end, stop;
    phase_range(phase, &start, &end, &stop);
    if (vocab <= stop || vocab < end)
        return fail(YUE2_ERR_VOCAB, "Vocabulary does not support native music protocol");
    return YUE2_OK;
}

int read_step_error(Workspace& w, hipStream_t s) {
    StepState st;
    hipError_t e = hipMemcpyAsync(&st, w.st, sizeof(StepState), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "step state readback");
    return step_error(st);
}

int step_error(const StepState& st) {
    if (st.error == 1) return fail(YUE2_ERR_CONTEXT, "AR input exceeds cache/model context");
    if (st.error == 2) return fail(YUE2_ERR_TOKEN, "Token outside model vocabulary");
    if (st.error == 3) return fail(YUE2_ERR_EMPTY, "Empty sampling distribution");
    if (st.error == 4) return fail(YUE2_ERR_LOGITS, "Model produced invalid logits");
    if (st.error == 5) return fail(YUE2_ERR_TIES, "top-k survivors exceed the device sort capacity");
    if (st.error == 8)
        return fail(YUE2_ERR_DEVICE,
                    "device error 8: a step-kernel workgroup waited too long for another's output "
                    "(workgroups not all resident, or the device shared with other work)");
    if (st.error != 0) return fail(YUE2_ERR_DEVICE, "device error " + std::to_string(st.error));
    return YUE2_OK;
}

}  // namespace y2

// ---------------------------------------------------------------------------
// C ABI: configuration, model, cache
// ---------------------------------------------------------------------------

extern "C" const char* yue2_hip_last_error(void) { return t_error.c_str(); }

extern "C" int32_t yue2_hip_config_validate(const Yue2Config* c) {
    if (!c) return fail(YUE2_ERR_ARG, "null config");
    const int32_t sizes[] = {c->hidden_size, c->num_hidden_layers, c->num_attention_heads,
                             c->num_key_value_heads, c->head_dim, c->intermediate_size,
                             c->vocab_size, c->max_position_embeddings};
    for (int32_t v : sizes)
        if (v <= 0) return fail(YUE2_ERR_CONFIG, "Invalid transformer configuration");
    if (c->num_attention_heads % c->num_key_value_heads != 0 || c->head_dim % 2 != 0 ||
        !(c->rope_theta > 0.0f) || !std::isfinite(c->rope_theta) || !(c->rms_norm_eps > 0.0f) ||
        !std::isfinite(c->rms_norm_eps))
        return fail(YUE2_ERR_CONFIG, "Invalid transformer configuration");
    return YUE2_OK;
}

// Shapes the kernels support (beyond Config validation).
static int check_supported(const Yue2Config* c) {
    const int D = c->head_dim;
    if (D != 64 && D != 128 && D != 256) return fail(YUE2_ERR_ARG, "head_dim must be 64, 128 or 256");
    if (c->num_attention_heads / c->num_key_value_heads > 8)
        return fail(YUE2_ERR_ARG, "at most 8 query heads per KV head");
    if (c->hidden_size % 8 || c->intermediate_size % 8)
        return fail(YUE2_ERR_ARG, "hidden and intermediate sizes must be multiples of 8");
    if (c->hidden_size > 16384 || c->intermediate_size > 16384 ||
        c->num_attention_heads * D > 16384)
        return fail(YUE2_ERR_ARG, "GEMV inner dimension above 16384");
    if (c->max_position_embeddings > 24576) return fail(YUE2_ERR_ARG, "context above 24576");
    return YUE2_OK;
}

extern "C" Yue2Model* yue2_hip_model_open(const Yue2Config* c, const uint16_t* embed,
                                          const uint16_t* lm_head, const float* final_norm,
                                          const Yue2LayerWeights* layers) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (yue2_hip_config_validate(c) != YUE2_OK) return nullptr;
    if (check_supported(c) != YUE2_OK) return nullptr;
    if (!embed || !lm_head || !final_norm || !layers) {
        fail(YUE2_ERR_ARG, "null weight pointer");
        return nullptr;
    }
    if (!device_ready()) {
        fail(YUE2_ERR_DEVICE, "no gfx950 device");
        return nullptr;
    }
    const int H = c->hidden_size, D = c->head_dim, Hq = c->num_attention_heads;
    const int Hkv = c->num_key_value_heads, I = c->intermediate_size, V = c->vocab_size;
    const int qkvw = (Hq + 2 * Hkv) * D, qw = Hq * D, kw = Hkv * D;
    auto* m = new Yue2Model();
    m->c = *c;
    Carve cv;
    const size_t o_embed = cv.take<uint16_t>((size_t)V * H);
    const size_t o_head = cv.take<uint16_t>((size_t)V * H);
    const size_t o_fnorm = cv.take<float>((size_t)H);
    const int half = D / 2;
    const size_t o_cos = cv.take<float>((size_t)c->max_position_embeddings * half);
    const size_t o_sin = cv.take<float>((size_t)c->max_position_embeddings * half);
    struct Off { size_t qkv, o, g, u, d, in, qn, kn, post; };
    std::vector<Off> offs(c->num_hidden_layers);
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
    hipError_t e = hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        hip_fail(e, "hipStreamCreate");
        delete m;
        return nullptr;
    }
    e = hipMalloc(&m->block, cv.offset);
    if (e != hipSuccess) {
        hip_fail(e, "hipMalloc(weights)");
        (void)hipStreamDestroy(m->stream);
        delete m;
        return nullptr;
    }
    m->block_bytes = cv.offset;
    char* base = static_cast<char*>(m->block);
    m->embed = reinterpret_cast<uint16_t*>(base + o_embed);
    m->lm_head = reinterpret_cast<uint16_t*>(base + o_head);
    m->final_norm = reinterpret_cast<float*>(base + o_fnorm);
    m->rope_cos = reinterpret_cast<float*>(base + o_cos);
    m->rope_sin = reinterpret_cast<float*>(base + o_sin);
    bool ok = true;
    auto up = [&](void* dst, const void* src, size_t bytes) {
        if (ok && hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) != hipSuccess) ok = false;
    };
    // Norm gammas are rounded to BF16 as Norm::new does with bf16 = true.
    auto up_norm = [&](float* dst, const float* src, int n) {
        std::vector<float> tmp(src, src + n);
        for (float& v : tmp) v = rb(v);
        up(dst, tmp.data(), sizeof(float) * n);
    };
    up(m->embed, embed, sizeof(uint16_t) * (size_t)V * H);
    up(m->lm_head, lm_head, sizeof(uint16_t) * (size_t)V * H);
    up_norm(m->final_norm, final_norm, H);
    // RoPE table for every position, Rotary::new (src/model.rs:137-149):
    // libm powf/cosf/sinf in f32, each value rounded to BF16.
    {
        std::vector<float> ct((size_t)c->max_position_embeddings * half), st(ct.size());
        for (int i = 0; i < half; ++i) {
            const float freq = 1.0f / powf(c->rope_theta, (float)(2 * i) / (float)D);
            for (int p = 0; p < c->max_position_embeddings; ++p) {
                const float angle = (float)p * freq;
                ct[(size_t)p * half + i] = rb(cosf(angle));
                st[(size_t)p * half + i] = rb(sinf(angle));
            }
        }
        up(m->rope_cos, ct.data(), sizeof(float) * ct.size());
        up(m->rope_sin, st.data(), sizeof(float) * st.size());
    }
    m->layers.resize(c->num_hidden_layers);
    for (int l = 0; l < c->num_hidden_layers && ok; ++l) {
        const Yue2LayerWeights& src = layers[l];
        if (!src.q_proj || !src.k_proj || !src.v_proj || !src.o_proj || !src.gate_proj ||
            !src.up_proj || !src.down_proj || !src.input_layernorm || !src.q_norm || !src.k_norm ||
            !src.post_attention_layernorm) {
            ok = false;
            fail(YUE2_ERR_ARG, "null layer weight");
            break;
        }
        LayerDev& L = m->layers[l];
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
        up(L.wqkv, src.q_proj, sizeof(uint16_t) * (size_t)qw * H);
        up(L.wqkv + (size_t)qw * H, src.k_proj, sizeof(uint16_t) * (size_t)kw * H);
        up(L.wqkv + (size_t)(qw + kw) * H, src.v_proj, sizeof(uint16_t) * (size_t)kw * H);
        up(L.wo, src.o_proj, sizeof(uint16_t) * (size_t)H * qw);
        up(L.wg, src.gate_proj, sizeof(uint16_t) * (size_t)I * H);
        up(L.wu, src.up_proj, sizeof(uint16_t) * (size_t)I * H);
        up(L.wd, src.down_proj, sizeof(uint16_t) * (size_t)H * I);
        up_norm(L.in_norm, src.input_layernorm, H);
        up_norm(L.q_norm, src.q_norm, D);
        up_norm(L.k_norm, src.k_norm, D);
        up_norm(L.post_norm, src.post_attention_layernorm, H);
    }
    // The layer table in device memory, for the persistent step kernel.
    if (ok && hipMalloc(&m->layers_dev, sizeof(LayerDev) * m->layers.size()) != hipSuccess) ok = false;
    up(m->layers_dev, m->layers.data(), sizeof(LayerDev) * m->layers.size());
    if (ok && (hipDeviceGetAttribute(&m->cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess ||
               m->cus <= 0))
        ok = false;
    if (!ok) {
        if (t_error.empty()) fail(YUE2_ERR_DEVICE, "weight upload failed");
        yue2_hip_model_free(m);
        return nullptr;
    }
    // the persistent step kernel is the default where the shape has one
    m->step_kernel = step_supported(m->c, 1, m->cus);
    return m;
}

extern "C" void yue2_hip_model_free(Yue2Model* m) {
    if (!m) return;
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    (void)hipStreamSynchronize(m->stream);
    // children outlive the model detached from it (see Yue2Model::caches)
    for (Yue2Decoder* d : std::vector<Yue2Decoder*>(m->decoders)) decoder_detach(d);
    for (Yue2Cache* c : m->caches) c->m = nullptr;
    m->decoders.clear();
    m->caches.clear();
    m->ws.release();
    if (m->layers_dev) (void)hipFree(m->layers_dev);
    if (m->block) (void)hipFree(m->block);
    if (m->nar.block) (void)hipFree(m->nar.block);
    (void)hipStreamDestroy(m->stream);
    delete m;
}

extern "C" int32_t yue2_hip_model_set_step_kernel(Yue2Model* m, int32_t on) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m) return fail(YUE2_ERR_ARG, "null model");
    m->step_kernel = on != 0 && step_supported(m->c, 1, m->cus);
    return m->step_kernel ? 1 : 0;
}

extern "C" int32_t yue2_hip_model_set_prefill(Yue2Model* m, int32_t mfma) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m) return fail(YUE2_ERR_ARG, "null model");
    m->prefill_mfma = mfma != 0;
    return m->prefill_mfma ? 1 : 0;
}

extern "C" int32_t yue2_hip_model_advance_sequence(Yue2Model* m, int32_t add) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || add < 0) return fail(YUE2_ERR_ARG, "null model or negative advance");
    Workspace& w = m->ws;
    if (!w.flow_block) return fail(YUE2_ERR_ARG, "the model has run no forward");
    launch_sequence(m->stream, w.st, 0, add);
    w.seq_bound += add;
    hipError_t e = hipStreamSynchronize(m->stream);
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "sequence advance");
}

extern "C" int32_t yue2_hip_norm_fallbacks(const Yue2Model* m) {
    if (!m) return 0;
    return m->norm_fallbacks;
}

extern "C" Yue2Cache* yue2_hip_cache_new(Yue2Model* m, int32_t capacity) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || capacity <= 0) {
        fail(YUE2_ERR_ARG, "invalid cache capacity");
        return nullptr;
    }
    const Yue2Config& c = m->c;
    const size_t elems = (size_t)c.num_hidden_layers * 2 * c.num_key_value_heads * capacity * c.head_dim;
    auto* cache = new Yue2Cache();
    cache->m = m;
    cache->capacity = capacity;
    cache->layers = c.num_hidden_layers;
    cache->kv_heads = c.num_key_value_heads;
    cache->head_dim = c.head_dim;
    hipError_t e = hipMalloc(&cache->kv, elems * sizeof(uint16_t));
    if (e != hipSuccess) {
        hip_fail(e, "hipMalloc(kv cache)");
        delete cache;
        return nullptr;
    }
    m->caches.push_back(cache);
    return cache;
}

// Cache's Drop (src/model.rs:286-290, which releases the GPU context of the
// cache id): legal before or after the model's free.  Decoders running on
// the cache are detached with it.
extern "C" void yue2_hip_cache_free(Yue2Cache* c) {
    if (!c) return;
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (Yue2Model* m = c->m) {
        (void)hipStreamSynchronize(m->stream);
        for (Yue2Decoder* d : std::vector<Yue2Decoder*>(m->decoders))
            if (decoder_uses(d, c)) decoder_detach(d);
        m->caches.erase(std::remove(m->caches.begin(), m->caches.end(), c), m->caches.end());
    }
    (void)hipFree(c->kv);  // hipFree waits for the device
    delete c;
}

extern "C" int32_t yue2_hip_cache_length(const Yue2Cache* c) { return c ? c->length : 0; }

// The device context of a cache from its host K/V mirror, as the reference's
// Metal bridge does when a cache first reaches the GPU (contextEntry,
// src/metal.m:633-666): mirror rows hold kv_heads * head_dim BF16-exact f32
// values, whose high 16 bits are the BF16 the device stores.
extern "C" int32_t yue2_hip_cache_load(Yue2Cache* c, const float* key, const float* value, int32_t length,
                                       int32_t stride) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!c || !key || !value) return fail(YUE2_ERR_ARG, "null cache or mirror");
    if (!c->m) return fail(YUE2_ERR_ARG, "the cache's model was freed");
    const Yue2Config& cf = c->m->c;
    if (length < 0 || length > c->capacity || length > cf.max_position_embeddings || stride < length)
        return fail(YUE2_ERR_CONTEXT, "AR input exceeds cache/model context");
    const int Hkv = cf.num_key_value_heads, D = cf.head_dim, width = Hkv * D;
    hipError_t e = hipStreamSynchronize(c->m->stream);  // no step may be writing the cache
    if (e != hipSuccess) return hip_fail(e, "cache load sync");
    std::vector<uint16_t> slab((size_t)width * std::max(length, 1));
    for (int l = 0; l < cf.num_hidden_layers && length > 0; ++l) {
        for (int which = 0; which < 2; ++which) {
            const float* src = (which == 0 ? key : value) + (size_t)l * stride * width;
            // [kv_heads][length][head_dim]: one head's rows are contiguous on the device
            for (int p = 0; p < length; ++p)
                for (int h = 0; h < Hkv; ++h) {
                    const uint32_t* row = reinterpret_cast<const uint32_t*>(src + (size_t)p * width + (size_t)h * D);
                    uint16_t* dst = slab.data() + ((size_t)h * length + p) * D;
                    for (int d = 0; d < D; ++d) dst[d] = (uint16_t)(row[d] >> 16);
                }
            uint16_t* base = c->kv + ((size_t)l * 2 + which) * Hkv * (size_t)c->capacity * D;
            e = hipMemcpy2D(base, (size_t)c->capacity * D * sizeof(uint16_t), slab.data(),
                            (size_t)length * D * sizeof(uint16_t), (size_t)length * D * sizeof(uint16_t), Hkv,
                            hipMemcpyHostToDevice);
            if (e != hipSuccess) return hip_fail(e, "cache load");
        }
    }
    c->length = length;
    return YUE2_OK;
}

// The host K/V mirror rows of a device cache: the reverse of cache_load, and
// what the reference's fast path hands back per token as `shadow` so that the
// Rust side can append it to its mirror and the CPU path can take over after
// a failed step (src/metal.m:846-871, src/model.rs:556-566).  Rows
// [start, start + n) of every layer go to key/value at row l * stride + p, as
// f32 holding the stored BF16 (exact).  Works after the model's free.
extern "C" int32_t yue2_hip_cache_export(const Yue2Cache* c, float* key, float* value, int32_t start, int32_t n,
                                         int32_t stride) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!c || !key || !value) return fail(YUE2_ERR_ARG, "null cache or mirror");
    if (start < 0 || n < 0 || start + n > c->length || stride < start + n)
        return fail(YUE2_ERR_CONTEXT, "export rows outside the cache length or the mirror stride");
    if (n == 0) return YUE2_OK;
    const int Hkv = c->kv_heads, D = c->head_dim, width = Hkv * D;
    hipError_t e = c->m ? hipStreamSynchronize(c->m->stream) : hipSuccess;  // every step has landed
    if (e != hipSuccess) return hip_fail(e, "cache export sync");
    std::vector<uint16_t> slab((size_t)width * n);
    for (int l = 0; l < c->layers; ++l) {
        for (int which = 0; which < 2; ++which) {
            const uint16_t* base = c->kv + ((size_t)l * 2 + which) * Hkv * (size_t)c->capacity * D + (size_t)start * D;
            e = hipMemcpy2D(slab.data(), (size_t)n * D * sizeof(uint16_t), base,
                            (size_t)c->capacity * D * sizeof(uint16_t), (size_t)n * D * sizeof(uint16_t), Hkv,
                            hipMemcpyDeviceToHost);
            if (e != hipSuccess) return hip_fail(e, "cache export");
            float* dst = (which == 0 ? key : value) + ((size_t)l * stride + start) * width;
            for (int p = 0; p < n; ++p)
                for (int h = 0; h < Hkv; ++h) {
                    const uint16_t* src = slab.data() + ((size_t)h * n + p) * D;
                    uint32_t* row = reinterpret_cast<uint32_t*>(dst + (size_t)p * width + (size_t)h * D);
                    for (int d = 0; d < D; ++d) row[d] = (uint32_t)src[d] << 16;
                }
        }
    }
    return YUE2_OK;
}

// Model::forward_phase: token-by-token through the decode-order kernels, so a
// prefill produces bit-for-bit the cache a sequence of decode steps would.
extern "C" int32_t yue2_hip_forward(Yue2Model* m, Yue2Cache* c, const int32_t* ids, int32_t n,
                                    int32_t phase, float* logits) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || !c || !ids || c->m != m) return fail(YUE2_ERR_ARG, "null model, cache or ids");
    if (int rc = check_phase_vocab(phase, m->c.vocab_size)) return rc;
    if (n <= 0 || c->length + n > c->capacity || c->length + n > m->c.max_position_embeddings)
        return fail(YUE2_ERR_CONTEXT, "AR input exceeds cache/model context");
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= m->c.vocab_size)
            return fail(YUE2_ERR_TOKEN, "Token outside model vocabulary");
    const int blocks = (c->capacity + kBlockKeys - 1) / kBlockKeys;
    if (int rc = m->ws.ensure(1, blocks, m->c)) return rc;
    if (m->step_kernel)
        if (int rc = prepare_step(m, m->ws); rc < 0) return rc;
    KvView kv{};
    kv.base[0] = c->kv;
    kv.capacity[0] = c->capacity;
    hipStream_t s = m->stream;
    m->ws.reserve_launches(s, n);
    m->ws.reset(s);
    for (int t = 0; t < n; ++t) {
        launch_set_state(s, m->ws.st, 1, c->length + t, 0, ids[t], 0);
        const bool head = logits && t == n - 1;
        int rc = enqueue_step_fused(m, m->ws, kv, 1, head, phase, s, nullptr, 0, 0, c->length + t + 1);
        if (rc == 1) rc = enqueue_step(m, m->ws, kv, 1, head, phase, s);
        if (rc) return rc;
    }
    if (int rc = read_step_error(m->ws, s)) return rc;
    StepState st;
    if (hipMemcpy(&st, m->ws.st, sizeof(st), hipMemcpyDeviceToHost) == hipSuccess)
        m->norm_fallbacks += st.norm_fallbacks;
    c->length += n;
    if (logits) {
        hipError_t e = hipMemcpy(logits, m->ws.logits, sizeof(float) * m->c.vocab_size,
                                 hipMemcpyDeviceToHost);
        if (e != hipSuccess) return hip_fail(e, "logits readback");
    }
    return YUE2_OK;
}

extern "C" int32_t yue2_hip_trace_step(Yue2Model* m, Yue2Cache* c, Yue2Cache* c2, int32_t id, uint64_t* stamps,
                                       int32_t cap, int32_t* wgs, int32_t* slots) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!m || !c || !stamps || !wgs || !slots || c->m != m || (c2 && (c2->m != m || c2 == c)))
        return fail(YUE2_ERR_ARG, "null model, cache or output");
    const int rows = c2 ? 2 : 1;
    Yue2Cache* cs[2] = {c, c2};
    if (!step_supported(m->c, rows, m->cus)) return fail(YUE2_ERR_ARG, "no step kernel for this shape");
    int cap_max = 0;
    for (int b = 0; b < rows; ++b) {
        if (cs[b]->length + 1 > cs[b]->capacity || cs[b]->length + 1 > m->c.max_position_embeddings)
            return fail(YUE2_ERR_CONTEXT, "AR input exceeds cache/model context");
        cap_max = std::max(cap_max, cs[b]->capacity);
    }
    if (id < 0 || id >= m->c.vocab_size) return fail(YUE2_ERR_TOKEN, "Token outside model vocabulary");
    const int nb = 1 + kTraceSlotsPerLayer * m->c.num_hidden_layers;
    const size_t n = (size_t)nb * m->cus;
    if ((size_t)cap < n) return fail(YUE2_ERR_ARG, "stamp buffer too small");
    // a workspace of its own for batch 2 (the model's serves batch-1 forwards)
    Workspace w2;
    Workspace& w = rows == 1 ? m->ws : w2;
    const int blocks = (cap_max + kBlockKeys - 1) / kBlockKeys;
    if (int rc = w.ensure(rows, blocks, m->c)) return rc;
    if (int rc = prepare_step(m, w)) return rc < 0 ? rc : fail(YUE2_ERR_ARG, "no step kernel for this shape");
    unsigned long long* dev = nullptr;
    if (hipMalloc(&dev, n * sizeof(*dev)) != hipSuccess) return fail(YUE2_ERR_ALLOC, "trace buffer");
    KvView kv{};
    for (int b = 0; b < rows; ++b) {
        kv.base[b] = cs[b]->kv;
        kv.capacity[b] = cs[b]->capacity;
    }
    hipStream_t s = m->stream;
    w.reserve_launches(s, 1);
    w.reset(s);
    launch_set_state(s, w.st, rows, c->length, rows > 1 ? c2->length : 0, id, rows > 1 ? id : 0);
    int rc = enqueue_step_fused(m, w, kv, rows, false, YUE2_PHASE_NONE, s, dev, nb);
    if (rc == 0) rc = read_step_error(w, s);
    if (rc == 0) {
        hipError_t e = hipMemcpy(stamps, dev, n * sizeof(*dev), hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_fail(e, "trace readback");
    }
    (void)hipFree(dev);
    if (rc) return rc;
    for (int b = 0; b < rows; ++b) cs[b]->length += 1;
    *wgs = m->cus;
    *slots = nb;
    return YUE2_OK;
}

extern "C" int32_t yue2_hip_prefill(Yue2Model* m, Yue2Cache* c, const int32_t* ids, int32_t n,
                                    int32_t phase, float* logits) {
    if (!c) return fail(YUE2_ERR_ARG, "null cache");
    if (n <= 0 || c->length != 0) return fail(YUE2_ERR_ARG, "Invalid prefill/cache capacity");
    return yue2_hip_forward(m, c, ids, n, phase, logits);
}

extern "C" int32_t yue2_hip_synchronize(void) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no gfx950 device");
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "hipDeviceSynchronize");
}

extern "C" int32_t yue2_hip_selftest_math(int32_t which, const void* in, void* out, size_t n) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!device_ready()) return fail(YUE2_ERR_DEVICE, "no gfx950 device");
    if (which < 0 || which > 18 || !in || !out || (which >= 4 && n % 256 != 0))
        return fail(YUE2_ERR_ARG, "bad selftest request");
    const size_t elem = which == 1 ? sizeof(double) : sizeof(float);
    void *din = nullptr, *dout = nullptr;
    hipError_t e = hipMalloc(&din, n * elem);
    if (e == hipSuccess) e = hipMalloc(&dout, n * elem);
    if (e == hipSuccess) e = hipMemcpy(din, in, n * elem, hipMemcpyHostToDevice);
    if (e == hipSuccess) {
        launch_math_selftest(nullptr, which, din, dout, n);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(out, dout, n * elem, hipMemcpyDeviceToHost);
    (void)hipFree(din);
    (void)hipFree(dout);
    return e == hipSuccess ? YUE2_OK : hip_fail(e, "selftest");
}
