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

// Every memory operation this thread issued has completed.
__device__ __forceinline__ void stores_done() { __builtin_amdgcn_s_waitcnt(0); }

}  // namespace y2
