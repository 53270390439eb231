// Per-element GGUF decoding shared by the dequantizer and the fused GEMM.
//
// The element values follow benchmarks/kernels/showcase/triton_kernels.py:134-181
// in fp32 with the reference's operation order.  Every product is exact in
// fp32 and Q4_K's final subtraction is the only rounding, so the value is the
// exact reference value; converting it to fp16 rounds to nearest even.
#pragma once

#include "gguf_common.h"

namespace tensor_gguf {

// Decode the 8 consecutive elements e0..e0+7 (e0 % 8 == 0) of one block.
template <int TYPE>
__device__ __forceinline__ void decode8(const uint8_t* __restrict__ block, int e0, float v[8]) {
  if (TYPE == kQ4_K) {
    const float d = half_bits_to_float(block[0] | (block[1] << 8));
    const float dmin = half_bits_to_float(block[2] | (block[3] << 8));
    const int sub = e0 >> 5;
    int sc, mn;
    q4k_scale_min(block + 4, sub, sc, mn);
    const float ds = d * (float)sc, dm = dmin * (float)mn;
    const int shift = 4 * ((e0 & 63) >> 5);
    const uint2 q = load8(block + 16 + (e0 >> 6) * 32 + (e0 & 31));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      v[i] = ds * (float)((byte >> shift) & 15u) - dm;
    }
  } else if (TYPE == kQ6_K) {
    const float d = half_bits_to_float(block[208] | (block[209] << 8));
    const int half = e0 >> 7, quarter = (e0 & 127) >> 5, l = e0 & 31;
    const float sc = (float)(int8_t)block[192 + (e0 >> 4)];
    const uint2 lo = load8(block + 64 * half + 32 * (quarter & 1) + l);
    const uint2 hi = load8(block + 128 + 32 * half + l);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t lb = ((i < 4 ? lo.x : lo.y) >> (8 * (i & 3))) & 0xFFu;
      const uint32_t hb = ((i < 4 ? hi.x : hi.y) >> (8 * (i & 3))) & 0xFFu;
      const int q = (int)(((lb >> (4 * (quarter >> 1))) & 15u) | (((hb >> (2 * quarter)) & 3u) << 4));
      v[i] = (float)(q - 32) * sc * d;
    }
  } else if (TYPE == kQ8_0) {
    const float d = half_bits_to_float(block[0] | (block[1] << 8));
    const uint2 q = load8(block + 2 + e0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int8_t c = (int8_t)(((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu);
      v[i] = d * (float)c;
    }
  } else {  // Q4_0
    const float d = half_bits_to_float(block[0] | (block[1] << 8));
    const uint2 q = load8(block + 2 + (e0 & 15));
    const int shift = 4 * (e0 >> 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      v[i] = (float)((int)((byte >> shift) & 15u) - 8) * d;
    }
  }
}

}  // namespace tensor_gguf
