// The split-operand layout of rows for the large-tile screen (k_screen4),
// shared by the kernels that write it (k_halves, and k_ema, k_split_fused and
// the small-batch update for the centroids they move).
//
// A row is cut into slabs of 32 dimensions (dimensions past d are zero), each
// 128 bytes, one cache line, stored slab-major: slab j of row g of an n-row
// matrix at (j n + g) 128 bytes. A slab row holds eight 16-byte chunks: for
// MFMA step kk = 0, 1 (dimensions 16 kk .. 16 kk + 15), chunks 4 kk and
// 4 kk + 1 are the hi halves of its two 8-dimension groups and chunks
// 4 kk + 2 and 4 kk + 3 their lo halves. Two formats, rounded to nearest even
// (x - hi is exact in f32):
//   bf16: hi = bf16(x), lo = bf16(x - hi): |x - hi - lo| <= 2^-16 |x| for
//         normal values (the three-pass screen);
//   fp16: hi = fp16(x), lo = fp16(x - hi): |x - hi| <= 2^-11 |x| + 2^-25 and
//         |x - hi - lo| <= 2^-22 |x| + 2^-25 (1 + 2^-11) for |x| < 65520 (the
//         two-pass screen: rows hi + lo, centroids hi).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace emh {

constexpr int SLAB_BYTES = 128;  // one row's 32 dimensions (one cache line)

typedef __bf16 v4bf_h __attribute__((ext_vector_type(4)));
typedef _Float16 v4h_h __attribute__((ext_vector_type(4)));

// Byte offset, within a slab row, of the hi quad of dimensions 4 c4 .. 4 c4 + 3
// of the slab (c4 = 0 .. 7); the lo quad sits 32 bytes later.
__device__ __forceinline__ int quad_hi_offset(int c4) {
  const int c8 = c4 >> 1;  // the 8-dimension group
  return 16 * (4 * (c8 >> 1) + (c8 & 1)) + 8 * (c4 & 1);
}

// The hi and lo halves of four values, as two 8-byte quads (fp16 when f16,
// else bf16).
__device__ __forceinline__ void split_quad(float4 v, uint2& hi, uint2& lo, bool f16 = false) {
  const float e[4] = {v.x, v.y, v.z, v.w};
  if (f16) {
    v4h_h h4, l4;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const _Float16 h = (_Float16)e[t];
      h4[t] = h;
      l4[t] = (_Float16)(e[t] - (float)h);
    }
    hi = __builtin_bit_cast(uint2, h4);
    lo = __builtin_bit_cast(uint2, l4);
    return;
  }
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
