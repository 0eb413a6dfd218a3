// dev_mem.h -- device memory access helpers shared by the decode kernels.
//
// Pointers that a kernel loads from device memory (the per-layer weight
// table, fields of argument structs) are generic to the compiler, which then
// emits flat loads.  Flat loads count against both the vector-memory and the
// LDS counters, so every LDS read that follows waits for all of them and a
// weight-streaming loop loses its overlap.  gbl()/gblw() cast such pointers
// to the global address space, so loads and stores are global_* instructions
// tracked by the vector-memory counter only.
//
// ld_dev/st_dev access data that other workgroups of the same launch write
// or read: agent-scope relaxed atomics, i.e. sc1 loads and stores on gfx950,
// which read from and write through to the device-coherent level (the XCDs'
// L2s are not coherent with each other).  A producer completes its stores
// (stores_done) before it signals a counter; consumers spin on the counter
// with relaxed loads and then read with ld_dev.
#pragma once
#include <hip/hip_runtime.h>

#define Y2_GLOBAL __attribute__((address_space(1)))

namespace y2 {

template <typename T>
__device__ __forceinline__ const Y2_GLOBAL T* gbl(const T* p) {
    return (const Y2_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ Y2_GLOBAL T* gblw(T* p) {
    return (Y2_GLOBAL T*)p;
}

// 16-byte global load (through a native vector type: HIP's uint4 cannot be
// copied from an address-space-qualified reference).
typedef unsigned int y2_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg4(const void* p) {
    const y2_u32x4 v = *(const Y2_GLOBAL y2_u32x4*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float ld_dev(const float* p) {
    return __hip_atomic_load(gblw(const_cast<float*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev(float* p, float v) {
    __hip_atomic_store(gblw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_dev_i(const int* p) {
    return __hip_atomic_load(gblw(const_cast<int*>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_i(int* p, int v) {
    __hip_atomic_store(gblw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int add_dev(int* p, int v) {
    return __hip_atomic_fetch_add(gblw(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Sets *p to code when it is 0 (sticky first error).
__device__ __forceinline__ void set_error(int* p, int code) {
    int expected = 0;
    __hip_atomic_compare_exchange_strong(gblw(p), &expected, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}

// ---- exact lane exchanges ---------------------------------------------------
// xor_lane<M>(v): the value of v held by lane (this lane ^ M), M a power of
// two up to 32.  M <= 8 stays inside 16-lane rows and is one DPP move (M = 4
// composes the half-row mirror with the quad reversal: i -> 7 - i -> i ^ 4);
// 16 and 32 use the row and half-wave swaps of gfx950, which leave each lane
// holding either its own value or its partner's in each of the two results.
// These are ALU moves, against a round trip through the LDS crossbar for
// ds_bpermute / ds_swizzle, and the xor butterflies built on them keep their
// association exactly (a + b is the same bits as b + a).
template <int M>
__device__ __forceinline__ int xor_lane_i(int x) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane distance");
    if constexpr (M == 1) {
        return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
        const int m = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, false);  // row_half_mirror
        return __builtin_amdgcn_mov_dpp(m, 0x1B, 0xF, 0xF, false);          // quad_perm [3,2,1,0]
    } else if constexpr (M == 8) {
        return __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
        return (threadIdx.x & 16) ? (int)r[0] : (int)r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        return (threadIdx.x & 32) ? (int)r[0] : (int)r[1];
    }
}
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
    return __builtin_bit_cast(float, xor_lane_i<M>(__builtin_bit_cast(int, v)));
}
template <int M>
__device__ __forceinline__ double xor_lane(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)xor_lane_i<M>((int)(uint32_t)u), hi = (uint32_t)xor_lane_i<M>((int)(uint32_t)(u >> 32));
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// The xor butterfly over lane distances HI, HI/2, ..., LO: v = v + v(lane ^ m)
// (sum) or fmaxf(v, v(lane ^ m)) (max) at each step.
template <int HI, int LO = 1, class T>
__device__ __forceinline__ T xor_sum(T v) {
    v = v + xor_lane<HI>(v);
    if constexpr (HI / 2 >= LO) return xor_sum<HI / 2, LO>(v);
    else return v;
}
template <int HI, int LO = 1>
__device__ __forceinline__ float xor_max(float v) {
    v = fmaxf(v, xor_lane<HI>(v));
    if constexpr (HI / 2 >= LO) return xor_max<HI / 2, LO>(v);
    else return v;
}

// Every memory operation this thread issued has completed.
__device__ __forceinline__ void stores_done() { __builtin_amdgcn_s_waitcnt(0); }

}  // namespace y2
