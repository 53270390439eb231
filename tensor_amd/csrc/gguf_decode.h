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
    const uint4 hd = load16(block);  // fp16 d, fp16 dmin, 12 scale bytes in one load
    const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
    const int sub = e0 >> 5;
    int sc_lo, mn_lo, sc_hi, mn_hi;
    q4k_scale_pair(hd.y, hd.z, hd.w, sub >> 1, sc_lo, mn_lo, sc_hi, mn_hi);
    const int sc = (sub & 1) ? sc_hi : sc_lo, mn = (sub & 1) ? mn_hi : mn_lo;
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
    // the four 6-bit codes of a dword assembled with byte masks; (q - 32) * (sc * d) is the
    // reference's (q - 32) * sc * d bit for bit: every product is exact, sign of zero included
    const float scd = sc * d;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      const uint32_t codes = (((w ? lo.y : lo.x) >> (4 * (quarter >> 1))) & 0x0F0F0F0Fu) |
                             ((((w ? hi.y : hi.x) >> (2 * quarter)) & 0x03030303u) << 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[4 * w + i] = ((float)((codes >> (8 * i)) & 0xFFu) - 32.0f) * scd;
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
    const uint32_t head = load4(block);  // d, then m (Q4_1, Q5_1) or the first half of qh (Q5_0)
    const float d = half_bits_to_float(head);
    const float m = TYPE == kQ5_0 ? 0.0f : half_bits_to_float(head >> 16);
    const int qs = TYPE == kQ4_1 ? 4 : TYPE == kQ5_0 ? 6 : 8;
    const uint32_t qh = TYPE == kQ4_1 ? 0u : load4(block + qs - 4) >> e0;
    const uint2 q = load8(block + qs + (e0 & 15));
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
    const uint32_t dd = load4(block + 80);  // fp16 d, fp16 dmin
    const float dl = half_bits_to_float(dd) * (float)(sc & 15u), ml = half_bits_to_float(dd >> 16) * (float)(sc >> 4);
    const int shift = 2 * ((e0 & 127) >> 5);
    const uint2 q = load8(block + 16 + 32 * (e0 >> 7) + (e0 & 31));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t byte = ((i < 4 ? q.x : q.y) >> (8 * (i & 3))) & 0xFFu;
      v[i] = dl * (float)((byte >> shift) & 3u) - ml;
    }
  } else if (TYPE == kQ3_K) {
    // scale bytes 0-7 (low nibbles) and bytes 6-11 with d (top bits), in two loads inside the block
    const int s = e0 >> 4;
    const uint2 lo8 = load8(block + 96), hi8 = load8(block + 102);
    const uint32_t low_byte = ((s & 7) < 4 ? lo8.x : lo8.y) >> (8 * (s & 3));
    const int low = (int)((s < 8 ? low_byte : low_byte >> 4) & 15u);
    // byte 8 + s % 4 of the scales is byte 2 + s % 4 of hi8 (bytes 102-109)
    const uint32_t high_byte = ((s & 3) < 2 ? hi8.x >> (16 + 8 * (s & 3)) : hi8.y >> (8 * ((s & 3) - 2))) & 0xFFu;
    const int high = (int)((high_byte >> (2 * (s >> 2))) & 3u);
    const float dl = half_bits_to_float(hi8.y >> 16) * (float)((low | (high << 4)) - 32);
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
    const uint4 hd = load16(block);  // fp16 d, fp16 dmin, 12 scale bytes
    const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
    const int sub = e0 >> 5;
    int sc_lo, mn_lo, sc_hi, mn_hi;
    q4k_scale_pair(hd.y, hd.z, hd.w, sub >> 1, sc_lo, mn_lo, sc_hi, mn_hi);
    const int sc = (sub & 1) ? sc_hi : sc_lo, mn = (sub & 1) ? mn_hi : mn_lo;
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
