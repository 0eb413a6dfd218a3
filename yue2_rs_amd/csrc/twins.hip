// twins.hip -- drop-in twins of the reference's native decode bridge
// (yue2_metal_* of src/metal.m, declared at src/tensor.rs:91-220).
//
// They keep the bridge's contract: host pointers borrowed for the call, 1 on
// success and 0 for "not done, fall back to the CPU", device copies of
// weights cached under (mapping, raw, rows, cols, dtype), device KV contexts
// keyed by (cache, layer) and mirrored from the caller's host KV rows, and
// every context discarded after a failed ar_stack so the CPU recomputes the
// token (src/metal.m:869-871).  The arithmetic is the same kernels and order
// spec as the session API.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <map>
#include <tuple>
#include <vector>

#include "../../include/yue2_hip.h"
#include "kernels.h"
#include "prefill.h"
#include "runtime.h"
#include "y2_math.h"

using namespace y2;

namespace {

struct WeightKey {
    size_t mapping;
    const void* raw;
    size_t rows, cols;
    int dtype;
    bool operator<(const WeightKey& o) const {
        return std::tie(mapping, raw, rows, cols, dtype) < std::tie(o.mapping, o.raw, o.rows, o.cols, o.dtype);
    }
};

struct Context {
    uint16_t* data = nullptr;  // [K, V][kv][capacity][dim] BF16
    size_t capacity = 0, length = 0, kv = 0, dim = 0;
};

struct TwinState {
    hipStream_t stream = nullptr;
    std::map<WeightKey, uint16_t*> weights;
    size_t weight_bytes = 0;
    // the prefill bridge's weights as f32 rows (src/metal.m:184-214), keyed
    // as above with the rounding flag in the dtype's sign
    std::map<WeightKey, float*> weights_f32;
    rocblas_handle blas = nullptr;
    std::map<std::pair<size_t, size_t>, Context> contexts;
    // scratch
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    StepState* st = nullptr;
    int32_t* counters = nullptr;  // attention group counters (zero between launches)
};

TwinState& twin() {
    static TwinState t;
    return t;
}

bool twin_ready() {
    if (!device_ready()) return false;
    TwinState& t = twin();
    if (!t.stream && hipStreamCreateWithFlags(&t.stream, hipStreamNonBlocking) != hipSuccess) return false;
    if (!t.st && hipMalloc(&t.st, sizeof(StepState)) != hipSuccess) return false;
    if (!t.counters) {
        if (hipMalloc(&t.counters, 4096 * sizeof(int32_t)) != hipSuccess) return false;
        if (hipMemset(t.counters, 0, 4096 * sizeof(int32_t)) != hipSuccess) return false;
    }
    return true;
}

void* scratch(size_t bytes) {
    TwinState& t = twin();
    if (t.scratch_bytes >= bytes) return t.scratch;
    if (t.scratch) (void)hipFree(t.scratch);
    t.scratch = nullptr;
    t.scratch_bytes = 0;
    if (hipMalloc(&t.scratch, bytes) != hipSuccess) return nullptr;
    t.scratch_bytes = bytes;
    return t.scratch;
}

void drop_contexts() {
    TwinState& t = twin();
    for (auto& kv : t.contexts) (void)hipFree(kv.second.data);
    t.contexts.clear();
}

void drop_weights() {
    TwinState& t = twin();
    for (auto& kv : t.weights) (void)hipFree(kv.second);
    t.weights.clear();
    for (auto& kv : t.weights_f32) (void)hipFree(kv.second);
    t.weights_f32.clear();
    t.weight_bytes = 0;
}

// Device BF16 copy of a host weight: BF16 as is; F32/F16 rounded to BF16 when
// the Linear rounds (src/tensor.rs:436-438, src/metal.m:173).
uint16_t* device_weight(const Yue2GpuWeight& w) {
    TwinState& t = twin();
    WeightKey key{w.mapping, w.raw, w.rows, w.cols, w.dtype};
    auto it = t.weights.find(key);
    if (it != t.weights.end()) return it->second;
    if (!w.raw || w.dtype < 0 || w.dtype > 2 || (w.dtype != 0 && !w.rounded)) return nullptr;
    const size_t n = w.rows * w.cols;
    std::vector<uint16_t> host;
    const void* src = w.raw;
    if (w.dtype != 0) {
        host.resize(n);
        for (size_t i = 0; i < n; ++i) {
            float v;
            if (w.dtype == 1) {
                std::memcpy(&v, w.raw + 4 * i, 4);
            } else {
                uint16_t hbits;
                std::memcpy(&hbits, w.raw + 2 * i, 2);
                v = (float)__builtin_bit_cast(_Float16, hbits);
            }
            host[i] = bf16_bits(rb(v));
        }
        src = host.data();
    }
    uint16_t* dev = nullptr;
    if (hipMalloc(&dev, n * sizeof(uint16_t)) != hipSuccess) return nullptr;
    if (hipMemcpy(dev, src, n * sizeof(uint16_t), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(dev);
        return nullptr;
    }
    t.weights[key] = dev;
    t.weight_bytes += n * sizeof(uint16_t);
    return dev;
}

// contextEntry of src/metal.m:633-668: reserve, then copy host rows
// [length, keys) as BF16 (the host values are BF16-exact).
Context* context_entry(const float* k, const float* v, size_t keys, size_t kv, size_t dim,
                       size_t cache, size_t layer, size_t reserve) {
    TwinState& t = twin();
    Context& e = t.contexts[{cache, layer}];
    if (!e.data || e.capacity < keys + reserve || e.length > keys || e.kv != kv || e.dim != dim) {
        if (e.data) (void)hipFree(e.data);
        e = Context{};
        const size_t capacity = (keys + reserve + 127) & ~(size_t)127;
        if (hipMalloc(&e.data, 2 * kv * capacity * dim * sizeof(uint16_t)) != hipSuccess) {
            t.contexts.erase({cache, layer});
            return nullptr;
        }
        e.capacity = capacity;
        e.kv = kv;
        e.dim = dim;
    }
    if (keys > e.length) {
        const size_t rows = keys - e.length, width = kv * dim;
        std::vector<uint16_t> kh(rows * dim), vh(rows * dim);
        for (size_t head = 0; head < kv; ++head) {
            for (size_t r = 0; r < rows; ++r)
                for (size_t d = 0; d < dim; ++d) {
                    const size_t src = (e.length + r) * width + head * dim + d;
                    kh[r * dim + d] = (uint16_t)(f2u(k[src]) >> 16);
                    vh[r * dim + d] = (uint16_t)(f2u(v[src]) >> 16);
                }
            uint16_t* kd = e.data + (head * e.capacity + e.length) * dim;
            uint16_t* vd = e.data + ((kv + head) * e.capacity + e.length) * dim;
            if (hipMemcpy(kd, kh.data(), rows * dim * 2, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(vd, vh.data(), rows * dim * 2, hipMemcpyHostToDevice) != hipSuccess)
                return nullptr;
        }
        e.length = keys;
    }
    return &e;
}

// Attention scratch for one row with `keys` keys.
struct AttnScratch {
    float *q, *out, *bmax, *bsum, *part;
    int blocks;
};

bool attn_scratch(size_t heads, size_t dim, size_t keys, size_t extra, AttnScratch* s, float** extra_out) {
    const int blocks = (int)((keys + kBlockKeys - 1) / kBlockKeys);
    const size_t n_q = heads * dim;
    const size_t n_blk = heads * (size_t)blocks, n_part = n_blk * dim;
    auto al = [](size_t n) { return (n + 63) & ~(size_t)63; };
    const size_t total = al(n_q) * 2 + 2 * al(n_blk) + al(n_part) + al(extra);
    float* p = static_cast<float*>(scratch(total * sizeof(float)));
    if (!p) return false;
    s->q = p;
    p += al(n_q);
    s->out = p;
    p += al(n_q);
    s->bmax = p;
    p += al(n_blk);
    s->bsum = p;
    p += al(n_blk);
    s->part = p;
    p += al(n_part);
    if (extra_out) *extra_out = p;
    s->blocks = blocks;
    return true;
}

// Attention over one context entry.  qkv_stride = heads*dim when q is final
// (no norms); the ar_stack passes the whole q|k|v row with its norms.
AttnArgs attn_args(const AttnScratch& s, const float* qkv, int qkv_stride, const Context& e, int heads,
                   int dim, float* out, int out_stride) {
    AttnArgs a{};
    a.qkv = qkv;
    a.qkv_stride = qkv_stride;
    a.kv.base[0] = e.data;
    a.kv.capacity[0] = (int)e.capacity;
    a.layer = 0;
    a.heads = heads;
    a.kv_heads = (int)e.kv;
    a.dim = dim;
    a.rows = 1;
    a.scale = 1.0f / std::sqrt((float)dim);
    a.bmax = s.bmax;
    a.bsum = s.bsum;
    a.part = s.part;
    a.out = out;
    a.out_stride = out_stride;
    a.blk_stride = s.blocks;
    attention_geometry((int)e.kv, 1, s.blocks, &a.wgs, &a.bpw);
    a.counters = twin().counters;
    a.st = twin().st;
    return a;
}

bool shapes_ok(size_t heads, size_t kv, size_t dim) {
    return kv && heads && heads % kv == 0 && heads / kv <= 8 && (dim == 64 || dim == 128 || dim == 256);
}

}  // namespace

extern "C" int32_t yue2_hip_available(void) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    return device_ready() ? 1 : 0;
}

extern "C" int32_t yue2_hip_vector_default(void) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!device_ready()) return 0;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return 0;
    return total_b >= ((size_t)2 << 30) ? 1 : 0;
}

extern "C" const char* yue2_hip_name(void) {
    static char name[256] = "CPU";
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (device_ready()) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, 0) == hipSuccess) {
            std::strncpy(name, prop.name[0] ? prop.name : prop.gcnArchName, sizeof(name) - 1);
            name[sizeof(name) - 1] = 0;
        }
    }
    return name;
}

extern "C" uint64_t yue2_physical_memory(void) {
    const long pages = sysconf(_SC_PHYS_PAGES), size = sysconf(_SC_PAGE_SIZE);
    return pages > 0 && size > 0 ? (uint64_t)pages * (uint64_t)size : 0;
}

extern "C" int32_t yue2_hip_vector(const float* input, const uint8_t* raw, size_t mapping,
                                   int32_t dtype, int32_t rounded, int32_t priority, float* out,
                                   size_t rows, size_t cols) {
    (void)priority;
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!input || !raw || !out || !rows || !cols || cols % 8 || cols > 16384 || rows > INT32_MAX)
        return 0;
    if (!twin_ready()) return 0;
    Yue2GpuWeight w{raw, mapping, rows, cols, dtype, rounded};
    uint16_t* dev = device_weight(w);
    if (!dev) return 0;
    float* buf = static_cast<float*>(scratch((cols + rows + 64) * sizeof(float)));
    if (!buf) return 0;
    float* x = buf;
    float* y = buf + ((cols + 63) & ~(size_t)63);
    hipStream_t s = twin().stream;
    if (hipMemcpyAsync(x, input, cols * sizeof(float), hipMemcpyHostToDevice, s) != hipSuccess) return 0;
    GemvArgs a{dev, nullptr, x, y, (int)cols, (int)rows, (int)rows, (int)cols, 1};
    if (launch_gemv(s, EPI_RAW, a) != hipSuccess) return 0;
    if (hipMemcpyAsync(out, y, rows * sizeof(float), hipMemcpyDeviceToHost, s) != hipSuccess) return 0;
    return hipStreamSynchronize(s) == hipSuccess ? 1 : 0;
}

extern "C" int32_t yue2_hip_cached_attention(const float* q, const float* k, const float* v,
                                             float* out, size_t keys, size_t heads, size_t kv,
                                             size_t dim, size_t cache, size_t layer) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!q || !k || !v || !out || keys == 0 || keys > (size_t)kContext || !shapes_ok(heads, kv, dim))
        return 0;
    if (!twin_ready()) return 0;
    Context* e = context_entry(k, v, keys, kv, dim, cache, layer, 0);
    if (!e) return 0;
    AttnScratch s;
    if (!attn_scratch(heads, dim, keys, 0, &s, nullptr)) return 0;
    hipStream_t st = twin().stream;
    if (hipMemcpyAsync(s.q, q, heads * dim * sizeof(float), hipMemcpyHostToDevice, st) != hipSuccess)
        return 0;
    launch_reset_state(st, twin().st, twin().counters, 4096);
    launch_set_state(st, twin().st, 1, (int)keys - 1, 0, 0, 0);
    if (launch_attention(st, attn_args(s, s.q, (int)(heads * dim), *e, (int)heads, (int)dim, s.out,
                                       (int)(heads * dim))) != hipSuccess)
        return 0;
    if (hipMemcpyAsync(out, s.out, heads * dim * sizeof(float), hipMemcpyDeviceToHost, st) != hipSuccess)
        return 0;
    return hipStreamSynchronize(st) == hipSuccess ? 1 : 0;
}

// One token through `count` layers (src/metal.m:718-874).
extern "C" int32_t yue2_hip_ar_stack(const float* input, float* out, float* shadow,
                                     const Yue2GpuLayer* layers, size_t count, size_t hidden,
                                     size_t heads, size_t kv, size_t dim, size_t intermediate,
                                     size_t prefix, size_t capacity, size_t cache, float eps,
                                     const float* cos_row, const float* sin_row) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!input || !out || !shadow || !layers || !cos_row || !sin_row || !count || !kv || !dim ||
        prefix >= (size_t)kContext || capacity <= prefix || capacity > (size_t)kContext)
        return 0;
    if (!shapes_ok(heads, kv, dim) || hidden % 8 || intermediate % 8 || hidden > 16384 ||
        intermediate > 16384 || heads * dim > 16384)
        return 0;
    if (!twin_ready()) return 0;
    TwinState& t = twin();
    hipStream_t s = t.stream;
    const size_t qw = heads * dim, kw = kv * dim, qkvw = qw + 2 * kw, half = dim / 2;
    const size_t extra = 2 * hidden + qkvw + qw + intermediate + 2 * half * capacity + 2 * hidden + 2 * dim;
    AttnScratch as;
    float* ex = nullptr;
    bool ok = attn_scratch(heads, dim, capacity, extra, &as, &ex);
    int32_t result = 0;
    if (ok) {
        float* x = ex;
        float* h = x + hidden;
        float* qkv = h + hidden;
        float* att = qkv + qkvw;
        float* act = att + qw;
        float* cos_t = act + intermediate;
        float* sin_t = cos_t + half * capacity;
        float* g_in = sin_t + half * capacity;
        float* g_post = g_in + hidden;
        float* g_q = g_post + hidden;
        float* g_k = g_q + dim;
        launch_reset_state(s, t.st, t.counters, 4096);
        launch_set_state(s, t.st, 1, (int)prefix, 0, 0, 0);
        ok = hipMemcpyAsync(x, input, hidden * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
             hipMemcpyAsync(cos_t + prefix * half, cos_row, half * 4, hipMemcpyHostToDevice, s) == hipSuccess &&
             hipMemcpyAsync(sin_t + prefix * half, sin_row, half * 4, hipMemcpyHostToDevice, s) == hipSuccess;
        std::vector<float> gam(2 * hidden + 2 * dim);
        for (size_t l = 0; l < count && ok; ++l) {
            const Yue2GpuLayer& L = layers[l];
            for (int j = 0; j < 4; ++j) ok = ok && L.norms[j];
            uint16_t* w[7];
            for (int j = 0; j < 7 && ok; ++j) {
                w[j] = device_weight(L.weights[j]);
                ok = w[j] != nullptr;
            }
            if (!ok) break;
            const Yue2GpuWeight* W = L.weights;
            ok = W[0].rows == qw && W[1].rows == kw && W[2].rows == kw && W[3].rows == hidden &&
                 W[4].rows == intermediate && W[5].rows == intermediate && W[6].rows == hidden &&
                 W[0].cols == hidden && W[1].cols == hidden && W[2].cols == hidden &&
                 W[3].cols == qw && W[4].cols == hidden && W[5].cols == hidden &&
                 W[6].cols == intermediate;
            Context* e = ok ? context_entry(L.key, L.value, prefix, kv, dim, cache, l, capacity - prefix) : nullptr;
            if (!e) {
                ok = false;
                break;
            }
            // Norm gammas arrive BF16-rounded (Norm::new); copy them per call
            // as the reference does (src/metal.m:766-775).
            std::memcpy(gam.data(), L.norms[0], hidden * 4);
            std::memcpy(gam.data() + hidden, L.norms[3], hidden * 4);
            std::memcpy(gam.data() + 2 * hidden, L.norms[1], dim * 4);
            std::memcpy(gam.data() + 2 * hidden + dim, L.norms[2], dim * 4);
            ok = hipMemcpyAsync(g_in, gam.data(), gam.size() * 4, hipMemcpyHostToDevice, s) == hipSuccess;
            // input RMSNorm in each projection's prologue
            GemvArgs qa{w[0], nullptr, x, qkv, (int)hidden, (int)qkvw, (int)qw, (int)hidden, 1, g_in, eps, t.st};
            GemvArgs ka{w[1], nullptr, x, qkv + qw, (int)hidden, (int)qkvw, (int)kw, (int)hidden, 1, g_in, eps, nullptr};
            GemvArgs va{w[2], nullptr, x, qkv + qw + kw, (int)hidden, (int)qkvw, (int)kw, (int)hidden, 1, g_in, eps, nullptr};
            ok = ok && launch_gemv(s, EPI_STORE, qa) == hipSuccess &&
                 launch_gemv(s, EPI_STORE, ka) == hipSuccess && launch_gemv(s, EPI_STORE, va) == hipSuccess;
            // QK-norm + RoPE + append of the new K/V + attention
            AttnArgs aa = attn_args(as, qkv, (int)qkvw, *e, (int)heads, (int)dim, att, (int)qw);
            aa.q_norm = g_q;
            aa.k_norm = g_k;
            aa.eps = eps;
            aa.cos_t = cos_t;
            aa.sin_t = sin_t;
            ok = ok && launch_attention(s, aa) == hipSuccess;
            GemvArgs oa{w[3], nullptr, att, x, (int)qw, (int)hidden, (int)hidden, (int)qw, 1};
            ok = ok && launch_gemv(s, EPI_RESID, oa) == hipSuccess;
            GemvArgs ga{w[4], w[5], x, act, (int)hidden, (int)intermediate, (int)intermediate, (int)hidden, 1, g_post, eps, nullptr};
            GemvArgs da{w[6], nullptr, act, x, (int)intermediate, (int)hidden, (int)hidden, (int)intermediate, 1};
            ok = ok && launch_gemv(s, EPI_SWIGLU, ga) == hipSuccess && launch_gemv(s, EPI_RESID, da) == hipSuccess;
            // gammas are reused by the next layer's upload: wait for this layer
            ok = ok && hipStreamSynchronize(s) == hipSuccess;
            if (ok) {
                StepState stv;
                ok = hipMemcpy(&stv, t.st, sizeof(stv), hipMemcpyDeviceToHost) == hipSuccess && stv.error == 0;
            }
            if (ok) {
                // shadow: the new token's K and V (src/metal.m:319-333)
                std::vector<uint16_t> kb(kw), vb(kw);
                for (size_t head = 0; head < kv && ok; ++head) {
                    ok = hipMemcpy(kb.data() + head * dim, e->data + (head * e->capacity + prefix) * dim, dim * 2,
                                   hipMemcpyDeviceToHost) == hipSuccess &&
                         hipMemcpy(vb.data() + head * dim, e->data + ((kv + head) * e->capacity + prefix) * dim,
                                   dim * 2, hipMemcpyDeviceToHost) == hipSuccess;
                }
                for (size_t i = 0; i < kw; ++i) {
                    shadow[l * 2 * kw + i] = bf16(kb[i]);
                    shadow[l * 2 * kw + kw + i] = bf16(vb[i]);
                }
                e->length = prefix + 1;
            }
        }
        if (ok) ok = hipMemcpy(out, x, hidden * 4, hipMemcpyDeviceToHost) == hipSuccess;
        result = ok ? 1 : 0;
    }
    // A failed stack leaves no partially appended context behind.
    if (!result) drop_contexts();
    return result;
}

extern "C" void yue2_hip_release_cache(size_t cache) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    TwinState& t = twin();
    for (auto it = t.contexts.begin(); it != t.contexts.end();) {
        if (it->first.first == cache) {
            (void)hipFree(it->second.data);
            it = t.contexts.erase(it);
        } else {
            ++it;
        }
    }
}

extern "C" void yue2_hip_clear_weights(void) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    drop_weights();
    drop_contexts();
}

extern "C" void yue2_hip_release_model(void) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    drop_weights();
    drop_contexts();
    TwinState& t = twin();
    if (t.scratch) (void)hipFree(t.scratch);
    t.scratch = nullptr;
    t.scratch_bytes = 0;
}

// ---- the prefill / NAR bridge: yue2_metal_gemm, linear, attention -----------
//
// The reference's GPU prefill hands plain FP32 matrix products (MPS,
// src/metal.m:164-237) and the multi-row attention (src/metal.m:330-361) to
// its bridge; the Rust caller rounds the results where its CPU path would
// (Linear::finish).  Here the products go to the platform BLAS (a plain
// library GEMM, column-major rocBLAS SGEMM on row-major operands by computing
// C^T = op(B)^T A^T), the attention to the matrix-core flash kernel of the
// matrix-core prefill.  As on the reference's GPU, the summation order is not
// the CPU path's, so results agree with it within FP32 rounding (the GEMMs)
// or the prefill's tolerance (the attention).  1 = done, 0 = fall back.

namespace {

rocblas_handle blas() {
    TwinState& t = twin();
    if (!t.blas) {
        if (rocblas_create_handle(&t.blas) != rocblas_status_success) {
            t.blas = nullptr;
            return nullptr;
        }
        if (rocblas_set_stream(t.blas, t.stream) != rocblas_status_success) return nullptr;
    }
    return t.blas;
}

bool fits_int(size_t v) { return v <= 0x7fffffffu; }

// C [m x n] (row stride ldc) = A [m x k] (lda) op(B) + beta C, row-major
// device operands; op(B) = B [k x n] (ldb) or, tb, B^T with B [n x k] (ldb).
bool sgemm_rows(const float* A, const float* B, float* C, size_t m, size_t n, size_t k, bool tb, size_t lda,
                size_t ldb, size_t ldc, float beta) {
    rocblas_handle h = blas();
    if (!h) return false;
    const float one = 1.0f;
    return rocblas_sgemm(h, tb ? rocblas_operation_transpose : rocblas_operation_none, rocblas_operation_none,
                         (rocblas_int)n, (rocblas_int)m, (rocblas_int)k, &one, B, (rocblas_int)ldb, A,
                         (rocblas_int)lda, &beta, C, (rocblas_int)ldc) == rocblas_status_success;
}

// Device f32 rows of a host weight, as convert_weight reads it
// (src/attention.metal:161-176): BF16 exactly, F32 and F16 as they are or
// rounded to BF16 when the Linear rounds.
float* device_weight_f32(const uint8_t* raw, size_t mapping, int dtype, int rounded, size_t n, size_t k) {
    TwinState& t = twin();
    const WeightKey key{mapping, raw, n, k, rounded ? -1 - dtype : dtype};
    auto it = t.weights_f32.find(key);
    if (it != t.weights_f32.end()) return it->second;
    if (!raw || dtype < 0 || dtype > 2) return nullptr;
    std::vector<float> host(n * k);
    for (size_t i = 0; i < n * k; ++i) {
        float v;
        if (dtype == 0) {
            uint16_t b;
            std::memcpy(&b, raw + 2 * i, 2);
            v = u2f((uint32_t)b << 16);
        } else if (dtype == 1) {
            std::memcpy(&v, raw + 4 * i, 4);
        } else {
            uint16_t b;
            std::memcpy(&b, raw + 2 * i, 2);
            v = (float)__builtin_bit_cast(_Float16, b);
        }
        host[i] = rounded && dtype != 0 ? rb(v) : v;
    }
    float* dev = nullptr;
    if (hipMalloc(&dev, host.size() * sizeof(float)) != hipSuccess) return nullptr;
    if (hipMemcpy(dev, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(dev);
        return nullptr;
    }
    t.weights_f32[key] = dev;
    t.weight_bytes += host.size() * sizeof(float);
    return dev;
}

}  // namespace

// yue2_metal_gemm (src/tensor.rs:207-219; src/metal.m:164-182): C = A op(B) +
// beta C for row-major host matrices with row strides lda, ldb, ldc.
extern "C" int32_t yue2_hip_gemm(const float* a, const float* b, float* c, size_t m, size_t n, size_t k,
                                 int32_t transpose_b, size_t lda, size_t ldb, size_t ldc, float beta) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!a || !b || !c || m == 0 || n == 0 || k == 0 || lda < k || ldc < n || ldb < (transpose_b ? k : n) ||
        !fits_int(m) || !fits_int(n) || !fits_int(k) || !twin_ready())
        return 0;
    const size_t brows = transpose_b ? n : k, bcols = transpose_b ? k : n;
    float* d = static_cast<float*>(scratch(sizeof(float) * (m * k + brows * bcols + m * n)));
    if (!d) return 0;
    float *da = d, *db = da + m * k, *dc = db + brows * bcols;
    TwinState& t = twin();
    hipError_t e = hipMemcpy2DAsync(da, k * 4, a, lda * 4, k * 4, m, hipMemcpyHostToDevice, t.stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(db, bcols * 4, b, ldb * 4, bcols * 4, brows, hipMemcpyHostToDevice, t.stream);
    if (e == hipSuccess && beta != 0.0f)
        e = hipMemcpy2DAsync(dc, n * 4, c, ldc * 4, n * 4, m, hipMemcpyHostToDevice, t.stream);
    bool ok = e == hipSuccess && sgemm_rows(da, db, dc, m, n, k, transpose_b != 0, k, bcols, n, beta);
    if (ok) ok = hipMemcpy2DAsync(c, ldc * 4, dc, n * 4, n * 4, m, hipMemcpyDeviceToHost, t.stream) == hipSuccess;
    return hipStreamSynchronize(t.stream) == hipSuccess && ok ? 1 : 0;
}

// yue2_metal_linear (src/tensor.rs:135-145; src/metal.m:216-237): c [m x n] =
// a [m x k] W^T for the host weight W [n x k] (dtype 0 BF16, 1 F32, 2 F16;
// rounded: F32/F16 rounded to BF16 first), the weight cached on the device
// under (mapping, raw, n, k, dtype, rounded).  Not rounded: the caller's
// Linear::finish rounds.
extern "C" int32_t yue2_hip_linear(const float* a, const uint8_t* raw, size_t mapping, int32_t dtype,
                                   int32_t rounded, float* c, size_t m, size_t n, size_t k) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!a || !raw || !c || m == 0 || n == 0 || k == 0 || !fits_int(m) || !fits_int(n) || !fits_int(k) ||
        !twin_ready())
        return 0;
    const float* w = device_weight_f32(raw, mapping, dtype, rounded, n, k);
    if (!w) return 0;
    float* d = static_cast<float*>(scratch(sizeof(float) * (m * k + m * n)));
    if (!d) return 0;
    float *da = d, *dc = d + m * k;
    TwinState& t = twin();
    bool ok = hipMemcpyAsync(da, a, m * k * 4, hipMemcpyHostToDevice, t.stream) == hipSuccess &&
              sgemm_rows(da, w, dc, m, n, k, true, k, k, n, 0.0f) &&
              hipMemcpyAsync(c, dc, m * n * 4, hipMemcpyDeviceToHost, t.stream) == hipSuccess;
    return hipStreamSynchronize(t.stream) == hipSuccess && ok ? 1 : 0;
}

// yue2_metal_attention (src/tensor.rs:194-206; src/metal.m:330-361): rows
// query rows q [rows x heads*dim] over keys rows of k, v [keys x kv*dim];
// row r sees keys [0, min(keys, causal + r + 1)) (causal >= 0) or all of them
// (causal < 0); softmax with `scale`; out [rows x heads*dim], BF16-rounded
// (unpack_attention, src/attention.metal:55-64).  Runs the matrix-core flash
// kernel, whose operands are BF16: inputs that are not BF16-exact (the
// model's always are), other head sizes than 64 and 128, a scale other than
// 1/sqrt(dim) and causal windows that reach past `keys` fall back (0).
extern "C" int32_t yue2_hip_attention(const float* q, const float* k, const float* v, float* out, size_t rows,
                                      size_t keys, size_t heads, size_t kv, size_t dim, int64_t causal,
                                      float scale) {
    std::lock_guard<std::recursive_mutex> guard(library_lock());
    if (!q || !k || !v || !out || rows == 0 || keys == 0 || kv == 0 || heads % kv || (dim != 64 && dim != 128) ||
        scale != 1.0f / sqrtf((float)dim) || !fits_int(rows) || !fits_int(keys) || !twin_ready())
        return 0;
    const bool noncausal = causal < 0;
    if (!noncausal && (size_t)causal + rows > keys) return 0;
    if (noncausal && rows > keys) return 0;
    const size_t qn = rows * heads * dim, kn = keys * kv * dim;
    auto exact = [](const float* x, size_t n) {
        for (size_t i = 0; i < n; ++i)
            if (f2u(x[i]) & 0xffffu) return false;
        return true;
    };
    if (!exact(q, qn) || !exact(k, kn) || !exact(v, kn)) return 0;
    // q as [rows][heads][dim] BF16; K and V as one layer of the cache layout
    // [K, V][kv][keys][dim]; the output [rows][heads * dim] BF16
    std::vector<uint16_t> hq(qn), hkv(2 * kn);
    for (size_t i = 0; i < qn; ++i) hq[i] = (uint16_t)(f2u(q[i]) >> 16);
    for (size_t r = 0; r < keys; ++r)
        for (size_t h = 0; h < kv; ++h)
            for (size_t d = 0; d < dim; ++d) {
                const size_t src = (r * kv + h) * dim + d;
                hkv[(h * keys + r) * dim + d] = (uint16_t)(f2u(k[src]) >> 16);
                hkv[((kv + h) * keys + r) * dim + d] = (uint16_t)(f2u(v[src]) >> 16);
            }
    uint16_t* d = static_cast<uint16_t*>(scratch(sizeof(uint16_t) * (2 * qn + 2 * kn)));
    if (!d) return 0;
    uint16_t *dq = d, *dkv = dq + qn, *dout = dkv + 2 * kn;
    TwinState& t = twin();
    bool ok = hipMemcpyAsync(dq, hq.data(), qn * 2, hipMemcpyHostToDevice, t.stream) == hipSuccess &&
              hipMemcpyAsync(dkv, hkv.data(), 2 * kn * 2, hipMemcpyHostToDevice, t.stream) == hipSuccess;
    FlashArgs f{};
    f.q = dq;
    f.kv_base = dkv;
    f.cap = (int)keys;
    f.layer = 0;
    f.heads = (int)heads;
    f.kv_heads = (int)kv;
    f.rows = (int)rows;
    f.scale = scale;
    f.out = dout;
    if (noncausal) {
        // every row sees keys [0, split + rows), all from the one buffer
        f.noncausal = 1;
        f.split = (int)(keys - rows);
        f.p0 = (int)(keys - rows);
    } else {
        f.p0 = (int)causal;
    }
    if (ok) ok = launch_flash(t.stream, f, (int)dim) == hipSuccess;
    std::vector<uint16_t> ho(qn);
    if (ok) ok = hipMemcpyAsync(ho.data(), dout, qn * 2, hipMemcpyDeviceToHost, t.stream) == hipSuccess;
    if (hipStreamSynchronize(t.stream) != hipSuccess || !ok) return 0;
    for (size_t i = 0; i < qn; ++i) out[i] = u2f((uint32_t)ho[i] << 16);
    return 1;
}
