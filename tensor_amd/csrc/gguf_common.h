// Device-side building blocks shared by the GGUF kernels (gfx950, wave64).
//
// Block formats (GGML type id: elements per block, bytes per block):
//   Q4_0 (2):  32,  18  fp16 d | 16 B nibbles            y = (q - 8) * d
//   Q8_0 (8):  32,  34  fp16 d | 32 x int8               y = d * q
//   Q4_K (12): 256, 144 fp16 d | fp16 dmin | 12 B 6-bit scales/mins | 128 B nibbles
//                                                      y = d*sc*q - dmin*m
//   Q6_K (14): 256, 210 128 B ql | 64 B qh | 16 x int8 scales | fp16 d
//                                                      y = d*sc*(q - 32)
// (reference: benchmarks/kernels/showcase/triton_kernels.py:134-181; Q8_0 from
// the public GGML block definition).  Rows are stored one after another, each
// row K/QK consecutive blocks.
//
// The other GGML encodings the generic kernels decode (public GGML block
// definitions; the reference has no code for them):
//   Q4_1 (3):  32,  20  fp16 d | fp16 m | 16 B nibbles    y = q*d + m
//   Q5_0 (6):  32,  22  fp16 d | u32 qh | 16 B nibbles    y = (q - 16)*d, q = nibble | qh bit << 4
//   Q5_1 (7):  32,  24  fp16 d | fp16 m | u32 qh | 16 B   y = q*d + m
//   Q2_K (10): 256, 84  16 B scale|min<<4 | 64 B 2-bit codes | fp16 d | fp16 dmin
//                                                      y = d*sc*q - dmin*m
//   Q3_K (11): 256, 110 32 B high-bit mask | 64 B 2-bit codes | 12 B 6-bit scales | fp16 d
//                                                      y = d*(sc - 32)*(q - (hbit ? 0 : 4))
//   Q5_K (13): 256, 176 fp16 d | fp16 dmin | 12 B scales/mins (Q4_K's) | 32 B high bits | 128 B nibbles
//                                                      y = d*sc*q - dmin*m
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tensor_gguf {

constexpr int kQ4_0 = 2;
constexpr int kQ4_1 = 3;
constexpr int kQ5_0 = 6;
constexpr int kQ5_1 = 7;
constexpr int kQ8_0 = 8;
constexpr int kQ2_K = 10;
constexpr int kQ3_K = 11;
constexpr int kQ4_K = 12;
constexpr int kQ5_K = 13;
constexpr int kQ6_K = 14;

// Elements (QK) and bytes per block of each encoding.
template <int TYPE>
struct Block {
  static constexpr int QK = (TYPE == kQ2_K || TYPE == kQ3_K || TYPE == kQ4_K || TYPE == kQ5_K || TYPE == kQ6_K)
                                ? 256 : 32;
  static constexpr int BYTES = TYPE == kQ4_0 ? 18 : TYPE == kQ4_1 ? 20 : TYPE == kQ5_0 ? 22 : TYPE == kQ5_1 ? 24
                             : TYPE == kQ8_0 ? 34 : TYPE == kQ2_K ? 84 : TYPE == kQ3_K ? 110
                             : TYPE == kQ4_K ? 144 : TYPE == kQ5_K ? 176 : 210;
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float2_t __attribute__((ext_vector_type(2)));

// Two fp32 values to an fp16 pair, each rounded to nearest even from its fp32 value
// (one v_cvt_pk_f16_f32).  Dequantization rounds to fp32 and the cast to fp16 rounds
// again (the reference's order); the register barrier keeps the compiler from fusing a
// producing fma with the conversion into an fp16-result v_fma_mix, which rounds the
// exact value once and differs where the fp32 result is an fp16 rounding tie.
__device__ __forceinline__ uint32_t half2_from_fp32(float a, float b) {
  asm volatile("" : "+v"(a), "+v"(b));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((float2_t){a, b}, half2_t));
}

// fp16 1024.0 in both halves of a dword: OR-ing a byte b into the low mantissa
// byte of 0x6400 gives the fp16 value 1024 + b exactly (b < 1024).
constexpr uint32_t kMagic = 0x64646464u;

__device__ __forceinline__ half2_t as_half2(uint32_t v) {
  return __builtin_bit_cast(half2_t, v);
}

// Bytes 0 and 1 of q, each widened to the fp16 value 1024 + byte.
__device__ __forceinline__ uint32_t magic01(uint32_t q) {
  return __builtin_amdgcn_perm(kMagic, q, 0x04010400u);
}
// Bytes 2 and 3 of q, each widened to the fp16 value 1024 + byte.
__device__ __forceinline__ uint32_t magic23(uint32_t q) {
  return __builtin_amdgcn_perm(kMagic, q, 0x04030402u);
}

// c + a.lo*b.lo + a.hi*b.hi on packed fp16 pairs, fp32 accumulate.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(as_half2(a), as_half2(b), c, false);
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits16 & 0xFFFFu));
}

// Loads that accept any byte alignment; gfx950 global loads are unaligned-
// capable, so each becomes one global_load_dwordx{4,2,1}.
__device__ __forceinline__ uint4 load16(const uint8_t* p) {
  uint4 v;
  __builtin_memcpy(&v, p, 16);
  return v;
}
__device__ __forceinline__ uint2 load8(const uint8_t* p) {
  uint2 v;
  __builtin_memcpy(&v, p, 8);
  return v;
}
__device__ __forceinline__ uint32_t load4(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Sum of the 16 fp16 values held in two uint4.
__device__ __forceinline__ float sum16(const uint4& a, const uint4& b) {
  const uint32_t one = 0x3C003C00u;  // (1.0, 1.0)
  float s = dot2(a.x, one, 0.0f);
  s = dot2(a.y, one, s);
  s = dot2(a.z, one, s);
  s = dot2(a.w, one, s);
  s = dot2(b.x, one, s);
  s = dot2(b.y, one, s);
  s = dot2(b.z, one, s);
  return dot2(b.w, one, s);
}

// Sum of the 8 fp16 values held in one uint4.
__device__ __forceinline__ float sum8(const uint4& a) {
  const uint32_t one = 0x3C003C00u;
  return dot2(a.w, one, dot2(a.z, one, dot2(a.y, one, dot2(a.x, one, 0.0f))));
}

// v plus the value of the lane a DPP control selects (CONTROL: a dpp_ctrl encoding).
template <int CONTROL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CONTROL, 0xF, 0xF, true));
}

// v[lane] + v[lane ^ 1] + ... over the lane's quad, added as (a + b) + (c + d) in every lane of
// it (DPP quad permutes: no LDS traffic, no lane arithmetic).
__device__ __forceinline__ float quad_sum(float v) {
  v = dpp_add<0xB1>(v);     // quad_perm [1, 0, 3, 2]: lane ^ 1
  return dpp_add<0x4E>(v);  // quad_perm [2, 3, 0, 1]: lane ^ 2
}

// Total over the wave when every lane of each 16-lane row already holds its row's sum:
// (row 0 + row 1) + (row 2 + row 3), the order of a xor-16 then xor-32 butterfly, read into
// scalar registers with v_readlane.
__device__ __forceinline__ float rows_total(float v) {
  const int bits = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(bits, 48));
  return (r0 + r1) + (r2 + r3);
}

// The wave total in every lane: row sums by DPP (xor 1, xor 2, half mirror, mirror: no LDS
// traffic, unlike a shuffle butterfly), then the four rows through v_readlane.
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0xB1>(v);
  v = dpp_add<0x4E>(v);
  v = dpp_add<0x141>(v);
  v = dpp_add<0x140>(v);
  return rows_total(v);
}

// Q4_K: the (scale, min) 6-bit pairs of sub-blocks 2j and 2j+1 from the three
// scale dwords s0 = bytes 0-3, s1 = bytes 4-7, s2 = bytes 8-11.
// Sub-blocks 0-3: scale = byte[s] & 63, min = byte[s+4] & 63.
// Sub-blocks 4-7: scale = (byte[s+4] & 15) | (byte[s-4] >> 6) << 4,
//                 min   = (byte[s+4] >> 4) | (byte[s]   >> 6) << 4.
__device__ __forceinline__ void q4k_scale_pair(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                               int& sc_lo, int& mn_lo, int& sc_hi, int& mn_hi) {
  const int shift = 16 * (j & 1);
  const uint32_t b0 = s0 >> shift, b1 = s1 >> shift, b2 = s2 >> shift;
  if (j < 2) {
    sc_lo = b0 & 63;
    sc_hi = (b0 >> 8) & 63;
    mn_lo = b1 & 63;
    mn_hi = (b1 >> 8) & 63;
  } else {
    sc_lo = (b2 & 15) | ((b0 >> 2) & 48);
    sc_hi = ((b2 >> 8) & 15) | ((b0 >> 10) & 48);
    mn_lo = ((b2 >> 4) & 15) | ((b1 >> 2) & 48);
    mn_hi = ((b2 >> 12) & 15) | ((b1 >> 10) & 48);
  }
}

// Single sub-block version (sub in 0..7), used by the dequantizer.
__device__ __forceinline__ void q4k_scale_min(const uint8_t* scales, int sub, int& sc, int& mn) {
  if (sub < 4) {
    sc = scales[sub] & 63;
    mn = scales[sub + 4] & 63;
  } else {
    sc = (scales[sub + 4] & 15) | ((scales[sub - 4] >> 6) << 4);
    mn = (scales[sub + 4] >> 4) | ((scales[sub] >> 6) << 4);
  }
}

// SwiGLU epilogue of a gate / up pair in fp32: silu(g) * u = g / (1 + exp(-g)) * u
// (src/tensor/compiler/webgpu/schedules/packed_integer.py:204-205).
__device__ __forceinline__ float swiglu(float g, float u) {
  return g / (1.0f + expf(-g)) * u;
}

template <typename T>
__device__ __forceinline__ void store_out(T* out, size_t index, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* out, size_t index, float v) {
  out[index] = v;
}
// fp16 of v after v has been rounded to fp32: without the empty asm the compiler folds a
// multiply or fma that produces v into v_fma_mixlo_f16, which rounds the exact product to fp16
// once and differs from fp32-then-fp16 rounding next to fp16 midpoints.
__device__ __forceinline__ _Float16 fp16_of_fp32(float v) {
  asm("" : "+v"(v));
  return (_Float16)v;  // v_cvt_f16_f32: round to nearest even
}

template <>
__device__ __forceinline__ void store_out<_Float16>(_Float16* out, size_t index, float v) {
  out[index] = fp16_of_fp32(v);
}

}  // namespace tensor_gguf
