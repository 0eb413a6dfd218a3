// attention.hip -- standalone launch of the fused decode attention
// (dev_attn.h): one kernel per layer, grid (workgroups per group, kv heads,
// rows).
#include <algorithm>

#include "dev_attn.h"
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

static int g_attn_cus = 0;

void attention_geometry(int kv_heads, int rows, int max_blocks, int* wgs, int* bpw) {
    if (g_attn_cus <= 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || v <= 0) v = 256;
        g_attn_cus = v;
    }
    const int groups = kv_heads * rows;
    int w = std::max(1, std::min(32, g_attn_cus / groups));
    w = std::min(w, std::max(1, max_blocks));
    *wgs = w;
    *bpw = attn_bpw_max(max_blocks, w);
}

hipError_t launch_attention(hipStream_t s, const AttnArgs& a) {
    const int G = a.heads / a.kv_heads;
    if (G < 1 || G > 8 || a.heads % a.kv_heads) return hipErrorInvalidValue;
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
