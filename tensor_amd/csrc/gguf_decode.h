// Per-element GGUF decoding shared by the dequantizer and the fused GEMM.
//
// The element values follow benchmarks/kernels/showcase/triton_kernels.py:134-181
// in fp32 with the reference's operation order.  Every product is exact in
// fp32 and Q4_K's final subtraction is the only rounding, so the value is the
// exact reference value; converting it to fp16 rounds to nearest even.  The
// encodings outside the reference (Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K) follow
// the public GGML definitions with the same property: exact products and at most
// one rounding, in the final addition or subtraction.
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
  } else if (TYPE == kQ4_0) {
    const float d = half_bits_to_float(block[0] | (block[1] << 8));
    const uint2 q = load8(block + 2 + (e0 & 15));
    const int shift = 4 * (e0 >> 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      v[i] = (float)((int)((byte >> shift) & 15u) - 8) * d;
    }
  } else if (TYPE == kQ4_1 || TYPE == kQ5_0 || TYPE == kQ5_1) {
    // element j < 16: low nibble of byte j; j + 16: its high nibble; Q5 bit 4 = bit j of qh
    const float d = half_bits_to_float(block[0] | (block[1] << 8));
    const float m = TYPE == kQ5_0 ? 0.0f : half_bits_to_float(block[2] | (block[3] << 8));
    const int head = TYPE == kQ4_1 ? 4 : TYPE == kQ5_0 ? 6 : 8;
    const uint32_t qh = TYPE == kQ4_1 ? 0u : load4(block + head - 4) >> e0;
    const uint2 q = load8(block + head + (e0 & 15));
    const int shift = 4 * (e0 >> 4);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      const int code = (int)(((byte >> shift) & 15u) | (((qh >> i) & 1u) << 4));
      // code*d is exact, so one rounding in the addition (fused or not)
      v[i] = TYPE == kQ5_0 ? (float)(code - 16) * d : (float)code * d + m;
    }
  } else if (TYPE == kQ2_K) {
    const uint32_t sc = block[e0 >> 4];
    const float d = half_bits_to_float(block[80] | (block[81] << 8));
    const float dmin = half_bits_to_float(block[82] | (block[83] << 8));
    const float dl = d * (float)(sc & 15u), ml = dmin * (float)(sc >> 4);
    const int shift = 2 * ((e0 & 127) >> 5);
    const uint2 q = load8(block + 16 + 32 * (e0 >> 7) + (e0 & 31));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      v[i] = dl * (float)((byte >> shift) & 3u) - ml;
    }
  } else if (TYPE == kQ3_K) {
    const int s = e0 >> 4;
    const uint8_t* scales = block + 96;
    const int low = s < 8 ? (scales[s] & 15) : (scales[s - 8] >> 4);
    const int high = (scales[8 + (s & 3)] >> (2 * (s >> 2))) & 3;
    const float dl = half_bits_to_float(block[108] | (block[109] << 8)) * (float)((low | (high << 4)) - 32);
    const int plane = (e0 & 127) >> 5, bit = 4 * (e0 >> 7) + plane;
    const uint2 q = load8(block + 32 + 32 * (e0 >> 7) + (e0 & 31));
    const uint2 hm = load8(block + (e0 & 31));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      const uint32_t mask = ((i < 4 ? hm.x : hm.y) >> (8 * (i & 3))) & 0xFFu;
      const int code = (int)((byte >> (2 * plane)) & 3u) - (((mask >> bit) & 1u) ? 0 : 4);
      v[i] = dl * (float)code;
    }
  } else {  // Q5_K
    const float d = half_bits_to_float(block[0] | (block[1] << 8));
    const float dmin = half_bits_to_float(block[2] | (block[3] << 8));
    const int sub = e0 >> 5;
    int sc, mn;
    q4k_scale_min(block + 4, sub, sc, mn);
    const float ds = d * (float)sc, dm = dmin * (float)mn;
    const int shift = 4 * (sub & 1);
    const uint2 q = load8(block + 48 + (e0 >> 6) * 32 + (e0 & 31));
    const uint2 qh = load8(block + 16 + (e0 & 31));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      const uint32_t high = ((i < 4 ? qh.x : qh.y) >> (8 * (i & 3))) & 0xFFu;
      v[i] = ds * (float)(((byte >> shift) & 15u) | (((high >> sub) & 1u) << 4)) - dm;
    }
  }
}

}  // namespace tensor_gguf
