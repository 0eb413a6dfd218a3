// attention.hip -- standalone launch of the fused decode attention: one
// kernel per layer, grid (workgroups per group, kv heads, rows).  Two
// bodies: attn_flow (dev_flow.h: the persistent step kernel's attention,
// block statistics and partials exchanged as tagged words) where the caller
// passes tagged buffers and the shape allows, else attn_group (dev_attn.h:
// counter syncs).  Both compute the same bits.
#include <algorithm>

#include "dev_attn.h"
#include "dev_flow.h"
#include "kernels.h"

namespace y2 {

constexpr int kAttnThreads = 512;

template <int D, int MAXG>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(const AttnArgs a) {
    extern __shared__ __align__(16) float e_s[];  // [G][bpw * 64]
    // no key/value append for a token the sampler chose as the phase's end
    // (the reference stops before its forward, src/sampling.rs:268-271)
    if (ld_dev_i(&a.st->done)) return;
    attn_group<kAttnThreads, D, MAXG>(a, blockIdx.x, blockIdx.y, blockIdx.z, e_s);
}

// The tagged-word body: the group's workgroups poll each other's words, so
// the launch holds at most one workgroup per CU (all resident at once).  The
// tags carry st->seq + 1 and the layer: a word left by an earlier launch of
// the same layer under the same sequence value would pass a poll.
template <int D, int G, bool GRT>
__global__ __launch_bounds__(kAttnThreads) void attention_flow_kernel(const AttnArgs a) {
    extern __shared__ __align__(16) float lds[];
    StepState* st = a.st;
    if (ld_dev_i(&st->done)) return;  // as attention_kernel
    const int b = blockIdx.z;
    const int pos = *gbl(&st->pos[b]);
    // (selects, not an indexed load: a runtime index would place the
    // argument copy in scratch memory)
    const int cap = b == 0 ? a.kv.capacity[0] : a.kv.capacity[1];
    // every workgroup of the group sees the same position, so all of them
    // leave here or none
    if (pos < 0 || pos >= cap || (pos + kBlockKeys) / kBlockKeys > a.blk_stride) {
        if (threadIdx.x == 0 && blockIdx.x == 0) set_error(&st->error, 1);
        return;
    }
    FlowAttn f;
    f.qkv = nullptr;
    f.qkv_stride = a.qkv_stride;
    f.packed = false;
    f.kv_base = b == 0 ? a.kv.base[0] : a.kv.base[1];
    f.cap = cap;
    f.pos = pos;
    f.layer = a.layer;
    f.heads = a.heads;
    f.kv_heads = a.kv_heads;
    f.blk_stride = a.blk_stride;
    f.att_stride = a.out_stride;
    f.wpg = gridDim.x;
    f.scale = a.scale;
    f.eps = a.eps;
    f.q_norm = a.q_norm;
    f.k_norm = a.k_norm;
    f.cos_t = a.cos_t;
    f.sin_t = a.sin_t;
    f.bmax = a.tbmax;
    f.bsum = a.tbsum;
    f.part = a.tpart;
    f.att = nullptr;
    f.epoch = ((uint32_t)*gbl(&st->seq) + 1u) & 0xFFFFFu;
    f.st = st;
    f.qkv_f = a.qkv;
    f.out_f = a.out;
    attn_flow<kAttnThreads, D, G, GRT, true>(f, blockIdx.x, blockIdx.y, b, lds, [] {}, [] {});
}

static int g_attn_cus = 0;
// dynamic LDS the tagged-word body may take
constexpr size_t kFlowLdsMax = 128 * 1024;

static int attn_cus() {
    if (g_attn_cus <= 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || v <= 0) v = 256;
        g_attn_cus = v;
    }
    return g_attn_cus;
}

void attention_geometry(int kv_heads, int rows, int max_blocks, int* wgs, int* bpw) {
    const int groups = kv_heads * rows;
    int w = std::max(1, std::min(32, attn_cus() / groups));
    w = std::min(w, std::max(1, max_blocks));
    *wgs = w;
    *bpw = attn_bpw_max(max_blocks, w);
}

// Dynamic LDS of the tagged-word body for this launch, or 0 when it does not
// take the launch: no tagged buffers, q already final (no QK-norm / append),
// head_dim other than 64 / 128, or the staged scores, p and the merge's
// partials of the longest context (blk_stride blocks) outgrow its K/V region.
static size_t flow_lds(const AttnArgs& a, int G, int wpg) {
    if (!a.tbmax || !a.tbsum || !a.tpart || !a.q_norm || (a.dim != 64 && a.dim != 128)) return 0;
    if (wpg < 1 || a.blk_stride < 1 || a.blk_stride > 24576 / kBlockKeys) return 0;
    const int D = a.dim, bpw = attn_bpw_max(a.blk_stride, wpg);
    const size_t kv_region = (size_t)2 * kAttnChunk * kBlockKeys * D * sizeof(uint16_t);
    const size_t merge = ((size_t)G * D * bpw + 2 * (size_t)a.blk_stride + 3 * (size_t)G * D) * sizeof(float);
    if (merge > kv_region || (size_t)G * bpw * kBlockKeys * sizeof(float) > kv_region / 2) return 0;
    const size_t lds = attn_flow_lds(G, D, bpw);
    return lds <= kFlowLdsMax ? lds : 0;
}

// Launches attention_flow_kernel<D, G, GRT> when one workgroup of it fits a
// CU with lds bytes of dynamic LDS (the polls need every workgroup of the
// grid resident); false (nothing launched) when it does not.
template <int D, int G, bool GRT>
static bool launch_flow_t(hipStream_t s, const AttnArgs& a, int wpg, size_t lds, hipError_t* e) {
    const void* fn = reinterpret_cast<const void*>(&attention_flow_kernel<D, G, GRT>);
    static const hipError_t attr = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kFlowLdsMax);
    static size_t fits = 0;  // the largest lds found to fit (fewer bytes fit as well)
    if (attr != hipSuccess) return false;
    if (lds > fits) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kAttnThreads, lds) != hipSuccess || per_cu < 1)
            return false;
        fits = lds;
    }
    attention_flow_kernel<D, G, GRT><<<dim3(wpg, a.kv_heads, a.rows), kAttnThreads, lds, s>>>(a);
    *e = hipGetLastError();
    return true;
}

static bool launch_flow(hipStream_t s, const AttnArgs& a, int G, hipError_t* e) {
    const int wpg = attn_cus() / (a.kv_heads * a.rows);
    const size_t lds = flow_lds(a, G, wpg);
    if (!lds) return false;
    if (a.dim == 128) {
        if (G == 3) return launch_flow_t<128, 3, false>(s, a, wpg, lds, e);
        if (G == 2) return launch_flow_t<128, 2, false>(s, a, wpg, lds, e);
        return G <= 4 ? launch_flow_t<128, 4, true>(s, a, wpg, lds, e) : launch_flow_t<128, 8, true>(s, a, wpg, lds, e);
    }
    return G <= 4 ? launch_flow_t<64, 4, true>(s, a, wpg, lds, e) : launch_flow_t<64, 8, true>(s, a, wpg, lds, e);
}

hipError_t launch_attention(hipStream_t s, const AttnArgs& a) {
    const int G = a.heads / a.kv_heads;
    if (G < 1 || G > 8 || a.heads % a.kv_heads) return hipErrorInvalidValue;
    if (a.rows < 1 || a.rows > kMaxRows) return hipErrorInvalidValue;
    hipError_t e = hipSuccess;
    if (launch_flow(s, a, G, &e)) return e;
    if (a.wgs * a.kv_heads * a.rows > 1024) return hipErrorInvalidValue;
    // the block statistics are gathered for at most 384 blocks (24576 keys)
    // (wgs * bpw covers every block of the geometry's contexts, whole super-blocks)
    if (std::min(a.wgs * a.bpw, a.blk_stride) > 24576 / kBlockKeys) return hipErrorInvalidValue;
    const dim3 grid(a.wgs, a.kv_heads, a.rows);
    const size_t lds = attn_group_lds(G, a.dim, a.wgs, a.bpw);
    if (lds > 96 * 1024) return hipErrorInvalidValue;
    const bool small = G <= 4;
    switch (a.dim) {
        case 64:
            if (small) attention_kernel<64, 4><<<grid, kAttnThreads, lds, s>>>(a);
            else attention_kernel<64, 8><<<grid, kAttnThreads, lds, s>>>(a);
            break;
        case 128:
            if (small) attention_kernel<128, 4><<<grid, kAttnThreads, lds, s>>>(a);
            else attention_kernel<128, 8><<<grid, kAttnThreads, lds, s>>>(a);
            break;
        case 256:
            if (small) attention_kernel<256, 4><<<grid, kAttnThreads, lds, s>>>(a);
            else attention_kernel<256, 8><<<grid, kAttnThreads, lds, s>>>(a);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace y2
