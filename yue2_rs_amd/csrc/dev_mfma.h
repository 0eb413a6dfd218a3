// dev_mfma.h -- BF16 matrix-core (MFMA) tiles of the prefill for gfx950.
//
// Operand layouts of the gfx950 BF16 MFMA instructions (checked on the
// device with small-integer operands, whose products and sums are exact):
//  * v_mfma_f32_32x32x16_bf16: lane l holds A[l % 32][8 (l / 32) + e] and
//    B[8 (l / 32) + e][l % 32], e < 8; accumulator r of lane l is
//    C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32], r < 16.
//  * v_mfma_f32_16x16x32_bf16: lane l holds A[l % 16][8 (l / 16) + e] and
//    B[8 (l / 16) + e][l % 16]; accumulator r is C[4 (l / 16) + r][l % 16],
//    r < 4.
// Both want the contraction index contiguous in each lane's eight values:
// for C = X W^T with X [M, K] and W [N, K] row-major (activations and
// weights as stored), A rows are rows of X and B columns are rows of W, so
// every operand is one 16-byte load of a row.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace y2 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
    bf16x8 r;
    __builtin_memcpy(&r, &v, 16);
    return r;
}

__device__ __forceinline__ f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Row and column of accumulator r of lane l in a 32x32 tile.
__device__ __forceinline__ int acc32_row(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
__device__ __forceinline__ int acc32_col(int lane) { return lane & 31; }

}  // namespace y2
