// The split-operand layout of rows for the bf16 screen (k_screen4), shared by
// the kernels that write it (k_halves, and k_ema for the centroids it moves).
//
// A row is cut into slabs of 32 dimensions (dimensions past d are zero), each
// 128 bytes, one cache line, stored slab-major: slab j of row g of an n-row
// matrix at (j n + g) 128 bytes. A slab row holds eight 16-byte chunks: for
// MFMA step kk = 0, 1 (dimensions 16 kk .. 16 kk + 15), chunks 4 kk and
// 4 kk + 1 are the bf16 hi halves of its two 8-dimension groups and chunks
// 4 kk + 2 and 4 kk + 3 their lo halves. hi = bf16(x) and lo = bf16(x - hi),
// both rounded to nearest even (x - hi is exact in f32), so
// |x - hi - lo| <= 2^-16 |x| for normal values.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace emh {

constexpr int SLAB_BYTES = 128;  // one row's 32 dimensions (one cache line)

typedef __bf16 v4bf_h __attribute__((ext_vector_type(4)));

// Byte offset, within a slab row, of the hi quad of dimensions 4 c4 .. 4 c4 + 3
// of the slab (c4 = 0 .. 7); the lo quad sits 32 bytes later.
__device__ __forceinline__ int quad_hi_offset(int c4) {
  const int c8 = c4 >> 1;  // the 8-dimension group
  return 16 * (4 * (c8 >> 1) + (c8 & 1)) + 8 * (c4 & 1);
}

// The hi and lo halves of four values, as two 8-byte quads.
__device__ __forceinline__ void split_quad(float4 v, uint2& hi, uint2& lo) {
  const float e[4] = {v.x, v.y, v.z, v.w};
  v4bf_h h4, l4;
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const __bf16 h = (__bf16)e[t];
    h4[t] = h;
    l4[t] = (__bf16)(e[t] - (float)h);
  }
  hi = __builtin_bit_cast(uint2, h4);
  lo = __builtin_bit_cast(uint2, l4);
}

}  // namespace emh
