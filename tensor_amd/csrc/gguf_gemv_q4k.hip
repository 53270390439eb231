// Q4_K decode GEMV fast paths (gfx950), out[m, n] = sum_k x[m, k] * W[n, k].
//
// Two kernels replace the generic VALU GEMV for Q4_K:
//
//  * M = 1, K a multiple of 4096: gemv_q4k_m1.  A workgroup of 4 or 8 waves owns
//    as many rows, one per wave, of one matrix of a group of up to three matrices
//    that share x (gate + up, q + k + v).  It loads x first, then all of its
//    weight bytes, and stages x once in LDS together with the per-sub-block
//    sums of x.  Lane = (super-block slot 0..15, quant pair j 0..3): each lane
//    decodes 64 codes per row and 4096-column step, widens them to subnormal
//    fp16 codes with bit masks only, accumulates with v_dot2_f32_f16 and
//    applies d * sc once per sub-block and dmin * m with the sum of x.
//
//  * 2 <= M <= 8: gemv_q4k_mfma.  A wave computes a 16-row tile with
//    v_mfma_f32_16x16x32_f16: the weights are the B operand (lane l holds row
//    l % 16, k-group l / 16), x the A operand.  Each lane widens its 64 codes
//    to fp16 "1024 + q" and folds the sub-block scale with one v_pk_fma_f16
//    per two codes, giving the exact integers sc * q (<= 945), so one MFMA
//    chain covers the whole super-block and d is applied once per super-block.
//    The min term  sum_s dmin * m_s * sum(x over s)  is a second, fp32
//    product (v_mfma_f32_16x16x4f32) whose A operand is the per-sub-block
//    activation sums and whose B operand is dmin * m.  The K range is split
//    across the waves of a workgroup and the partial tiles meet in LDS.
//    gemv_q4k_sec is the same arithmetic with the weights read as whole
//    64-byte sectors of 16 rows per load (wide matrices, long rows).
//
// Block format and element formula: benchmarks/kernels/showcase/triton_kernels.py:143-162.
#include <algorithm>

#include "gguf_common.h"
#include "gguf_launch.h"

namespace tensor_gguf {

typedef float float4v_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------- shared ---

// Scale and min codes of sub-blocks 2j (bits 0-7) and 2j+1 (bits 8-15) of a
// super-block header, with the lane-constant selectors of pair j.
struct PairSelect {
  int shift;
  bool low;
  uint32_t lowmask, highmask;
  __device__ __forceinline__ explicit PairSelect(int j)
      : shift(16 * (j & 1)), low(j < 2), lowmask(j < 2 ? 0x3F3Fu : 0x0F0Fu), highmask(j < 2 ? 0u : 0x3030u) {}
  __device__ __forceinline__ void codes(const uint4& hd, uint32_t& scs, uint32_t& mns) const {
    const uint32_t b0 = hd.y >> shift, b1 = hd.z >> shift, b2 = hd.w >> shift;
    scs = ((low ? b0 : b2) & lowmask) | ((b0 >> 2) & highmask);
    mns = ((low ? b1 : (b2 >> 4)) & lowmask) | ((b1 >> 2) & highmask);
  }
};

// ------------------------------------------------------- M = 1, LDS x ---

// Widening by bit masks alone: q & 0x000F000F is the fp16 pair (q0 * 2^-24,
// q2 * 2^-24) -- subnormal fp16 values are exact and v_dot2_f32_f16 multiplies
// them exactly -- and q & 0x00F000F0 the pair (16 q0, 16 q2) * 2^-24 of the high
// nibbles.  Codes of bytes 0 and 2 pair with x[4u] and x[4u+2], so x is staged
// in LDS with the halves of every 4-element group reordered (x0, x2, x1, x3).
constexpr float kTwo24 = 16777216.0f, kTwo20 = 1048576.0f;

// One wave = one weight row; the WAVES waves of a workgroup = WAVES
// consecutive rows of one matrix of the group.  The activation vector is
// loaded first, then every weight load of the wave, so that on each CU the
// small x load is not queued behind weight traffic; a compiler barrier keeps
// the weight loads from sinking below the x staging, and the workgroup
// barrier fences LDS only, so decoding starts as soon as this wave's own
// bytes have arrived.
//
// SWIGLU = true (MATS = 2: gate, up): waves 0 .. WAVES/2-1 take rows r .. of
// the gate matrix and the other half the same rows of the up matrix; the up
// waves hand their sums over in LDS and the gate waves store silu(gate) * up
// to out0, so the pair's products never leave the workgroup.
//
// TYPE = kQ5_K runs Q5_K rows through the same kernel: its super-block is Q4_K's header and
// nibbles (at byte 48) plus 32 bytes of fifth bits, bit sub of byte l for element 32 sub + l.
// Byte l of a lane's quant chunks pairs with byte l of the qh run, so the fifth bit of each
// code is OR-ed into its fp16 subnormal (bit 4 for the low nibble, bit 8 for the high nibble's
// 16 q): every code stays below 1024 and exact.
//
// The arguments are plain scalars, x, the weights and the row counts first: the library is
// built with kernel-argument preloading, so the dispatcher places them in SGPRs and the first
// loads of a wave leave without waiting on scalar loads of the argument block (the selection
// of the matrix is scalar arithmetic on them; only the output pointers, needed at the store,
// are read from memory).  Matrix i takes ceil(n_i / rows-per-workgroup) consecutive
// workgroups.
//
// ONE_ROUND (grids of at most four waves per SIMD, all resident from the start): each wave
// raises its issue priority until its loads are out, then drops back (down 4096 x 12288 in a
// timing harness: 6.45 against 6.61 us).  Grids that run in rounds keep the default: there a
// raised start delays the resident waves' decode (gate + up: 11.8 against 10.3 us).
template <int STEPS, int WAVES, int MATS, typename OutT, bool SWIGLU = false, int TYPE = kQ4_K, bool ONE_ROUND = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_q4k_m1(const _Float16* __restrict__ x, const uint8_t* w0,
                                                          const uint8_t* w1, const uint8_t* w2, int n0, int n1, int n2,
                                                          OutT* out0, OutT* out1, OutT* out2) {
  if constexpr (ONE_ROUND) __builtin_amdgcn_s_setprio(3);
  constexpr bool Q5 = TYPE == kQ5_K;
  constexpr int BLOCK = Q5 ? 176 : 144, QOFF = Q5 ? 48 : 16, SB = 16 * BLOCK;  // SB: one 4096-column step
  constexpr int K = STEPS * 4096, ROW_BYTES = STEPS * SB, T = WAVES * 64;
  constexpr int XC = (K / 8 + T - 1) / T;  // 16-byte x chunks per thread
  constexpr int PAIRS = WAVES / 2;
  static_assert(!SWIGLU || MATS == 2, "the SwiGLU pairing takes a gate and an up matrix");
  static_assert(MATS >= 1 && MATS <= kGemvGroupMax, "one to three matrices per launch");
  __shared__ __attribute__((aligned(16))) uint8_t xlds[K * 2 + K / 4];
  __shared__ __attribute__((aligned(16))) float sxl[K / 32];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;

  // chunk c of x is in range for every thread when the workgroup divides K / 8 (no exec-mask
  // branch ahead of the first load)
  constexpr bool XALL = (K / 8) % T == 0;
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (XALL || c < K / 8) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * c);
  }
  int mat = 0, block = blockIdx.x;
  if constexpr (SWIGLU) {
    mat = wv >= PAIRS ? 1 : 0;
  } else {
    const int b0 = (n0 + WAVES - 1) / WAVES, b1 = (n1 + WAVES - 1) / WAVES;
    if (MATS > 1 && block >= b0) {
      block -= b0;
      mat = 1;
      if (MATS > 2 && block >= b1) {
        block -= b1;
        mat = 2;
      }
    }
  }
  const uint8_t* const wm = mat == 0 ? w0 : mat == 1 ? w1 : w2;
  const int n_rows = mat == 0 ? n0 : mat == 1 ? n1 : n2;
  const int row = SWIGLU ? block * PAIRS + wv - mat * PAIRS : block * WAVES + wv;
  const int slot = lane >> 2, j = lane & 3;
  // One 4096-column step: 32-bit byte offsets from the matrix's scalar base (the host keeps every
  // matrix under 4 GiB), so the loads take the scalar-base form with no 64-bit address arithmetic
  // per lane (single gate 6.20 -> 6.08 us, Q5_K 7.78 -> 7.55 us, A/B on one box).  Longer rows
  // keep 64-bit addresses: the same form made the 4096 x 12288 down 2% slower.
  const uint8_t* wl;
  const uint8_t* wq;
  if constexpr (STEPS == 1) {
    const uint32_t off = (uint32_t)min(row, n_rows - 1) * (uint32_t)ROW_BYTES + (uint32_t)(slot * BLOCK);
    wl = wm + off;
    wq = wm + (off + 32u * j);
  } else {
    wl = wm + (size_t)min(row, n_rows - 1) * ROW_BYTES + slot * BLOCK;
    wq = wl + 32 * j;
  }
  uint4 hd[STEPS], q0[STEPS], q1[STEPS];
  uint4 h0[Q5 ? STEPS : 1], h1[Q5 ? STEPS : 1];  // Q5_K: the 32 fifth-bit bytes of the super-block
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    hd[s] = load16(wl + s * SB);
    q0[s] = load16(wq + s * SB + QOFF);
    q1[s] = load16(wq + s * SB + QOFF + 16);
    if constexpr (Q5) {
      h0[s] = load16(wl + s * SB + 16);
      h1[s] = load16(wl + s * SB + 32);
    }
  }
  asm volatile("" ::: "memory");
  if constexpr (ONE_ROUND) __builtin_amdgcn_s_setprio(0);
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (XALL || c < K / 8) {
      const uint4 v = xr[i];
      // sum of the 32 x of sub-block c / 4 over the four chunks c = 4 s' .. 4 s' + 3 (one quad
      // of lanes; K / 8 is a multiple of 4, so a quad is wholly inside or outside the range).
      // All four lanes of the quad hold the same sum; they all store it, to the same word, which
      // saves the masking (except for the SwiGLU pairs, measured 1.4% faster with one store)
      const float p = quad_sum(sum8(v));
      if (!SWIGLU || (c & 3) == 0) sxl[c >> 2] = p;
      // chunk c (16 B) -> LDS byte 16 c + 16 (c / 8): padding keeps the b128 reads conflict-free
      *reinterpret_cast<uint4*>(xlds + 16 * c + 16 * (c >> 3)) =
          make_uint4(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                     __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u));
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  // (a SwiGLU pair past the last row still decodes the clamped row: it meets the barrier below)
  if (!SWIGLU && row >= n_rows) return;

  const PairSelect sel(j);
  float total = 0.f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int c0 = ((s * 16 + slot) * 256 + 64 * j) >> 3;
    const float2 sx = *reinterpret_cast<const float2*>(&sxl[(s * 16 + slot) * 8 + 2 * j]);
    // the two sub-blocks one after the other, so that only four x chunks are live at a time
    float acc2[2] = {0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint4 xs[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = c0 + 4 * h + i;
        xs[i] = *reinterpret_cast<const uint4*>(xlds + 16 * c + 16 * (c >> 3));
      }
      const uint32_t mask = h == 0 ? 0x000F000Fu : 0x00F000F0u;
      float a = 0.f;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t q = word(u < 4 ? q0[s] : q1[s], u & 3), t = q >> 8;
        uint32_t cq = q & mask, ct = t & mask;
        if constexpr (Q5) {
          // fifth bit of sub-block 2j + h: bit 4 (low nibble) or bit 8 (16 x high nibble) of the half
          const uint32_t hq = word(u < 4 ? h0[s] : h1[s], u & 3) >> (2 * j + h);
          cq |= (hq & 0x00010001u) << (4 + 4 * h);
          ct |= ((hq >> 8) & 0x00010001u) << (4 + 4 * h);
        }
        a = dot2(cq, word(xs[u >> 1], 2 * (u & 1)), a);
        a = dot2(ct, word(xs[u >> 1], 2 * (u & 1) + 1), a);
      }
      acc2[h] = a;
      __builtin_amdgcn_sched_barrier(0);
    }
    uint32_t scs, mns;
    sel.codes(hd[s], scs, mns);
    const float dd = half_bits_to_float(hd[s].x), dmin = half_bits_to_float(hd[s].x >> 16);
    // acc2[0] = 2^-24 sum x q (sub-block 2j), acc2[1] = 2^-20 sum x q (sub-block 2j+1)
    total = fmaf(dd * (float)(scs & 0xFF) * kTwo24, acc2[0], total);
    total = fmaf(dd * (float)(scs >> 8) * kTwo20, acc2[1], total);
    total = fmaf(-dmin * (float)(mns & 0xFF), sx.x, total);
    total = fmaf(-dmin * (float)(mns >> 8), sx.y, total);
  }
  const float v = wave_sum(total);
  if constexpr (SWIGLU) {
    __shared__ float up_sum[PAIRS];
    const int pair = wv - mat * PAIRS;
    if (mat == 1 && lane == 0) up_sum[pair] = v;
    __syncthreads();
    if (mat == 0 && lane == 0 && row < n_rows) store_out<OutT>(out0, (uint32_t)row, swiglu(v, up_sum[pair]));
  } else {
    if (lane == 0) store_out<OutT>(mat == 0 ? out0 : mat == 1 ? out1 : out2, (uint32_t)row, v);
  }
}

// ------------------------------------------------------ M = 1, fp32 x ---

// fp32 activations at M = 1 (the showcase's packed call form, benchmark.py:460-464): the lane
// plan and loads of gemv_q4k_m1 (one row per wave, lane = super-block slot x quant pair j, x
// staged once per workgroup), with each 4-bit code converted to fp32 and multiplied by the fp32
// activation, so the products are the reference's decode numerics (fp32 operands,
// benchmark.py:466-472) up to summation order: d * sc once per sub-block, dmin * m with the
// sub-block's fp32 sum of x.  x sits in LDS as fp32 chunks of 4 with 16 bytes of padding per
// 256, so the sixteen (slot, j) start offsets of one b128 read fall in distinct banks.
__device__ __forceinline__ int f32_chunk(int c) { return 4 * c + 4 * (c >> 4); }

template <int STEPS, int WAVES, typename OutT, int TYPE>
__global__ __launch_bounds__(WAVES * 64) void gemv_q4k_m1_f32(const float* __restrict__ x, const uint8_t* __restrict__ w,
                                                              OutT* __restrict__ out, int n_rows) {
  constexpr bool Q5 = TYPE == kQ5_K;
  constexpr int BLOCK = Q5 ? 176 : 144, QOFF = Q5 ? 48 : 16, SB = 16 * BLOCK;  // SB: one 4096-column step
  constexpr int K = STEPS * 4096, ROW_BYTES = STEPS * SB, T = WAVES * 64;
  constexpr int XC = K / 4 / T;  // 16-byte x chunks (4 floats) per thread
  static_assert(XC * T * 4 == K, "every thread stages whole chunks");
  __shared__ __attribute__((aligned(16))) float xlds[K + K / 16];
  __shared__ float sxl[K / 32];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * (threadIdx.x + i * T));
  const int row = blockIdx.x * WAVES + wv, slot = lane >> 2, j = lane & 3;
  const uint8_t* wl = w + (size_t)min(row, n_rows - 1) * ROW_BYTES + slot * BLOCK;
  const uint8_t* wq = wl + 32 * j;
  uint4 hd[STEPS], q0[STEPS], q1[STEPS];
  uint4 h0[Q5 ? STEPS : 1], h1[Q5 ? STEPS : 1];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    hd[s] = load16(wl + s * SB);
    q0[s] = load16(wq + s * SB + QOFF);
    q1[s] = load16(wq + s * SB + QOFF + 16);
    if constexpr (Q5) {
      h0[s] = load16(wl + s * SB + 16);
      h1[s] = load16(wl + s * SB + 32);
    }
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    const uint4 v = xr[i];
    *reinterpret_cast<uint4*>(&xlds[f32_chunk(c)]) = v;
    // a sub-block is 8 consecutive chunks, held by 8 consecutive lanes: their sum in all 8
    const float part = (__uint_as_float(v.x) + __uint_as_float(v.y)) + (__uint_as_float(v.z) + __uint_as_float(v.w));
    const float sum = dpp_add<0x141>(quad_sum(part));
    if ((c & 7) == 0) sxl[c >> 3] = sum;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (row >= n_rows) return;

  const PairSelect sel(j);
  float total = 0.f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int sub = (s * 16 + slot) * 8 + 2 * j;  // sub-block 2j of the super-block
    const float2 sx = *reinterpret_cast<const float2*>(&sxl[sub]);
    float acc2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c0 = 8 * (sub + h);  // first x chunk of sub-block 2j + h
      float a = 0.f;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        uint32_t codes = (word(u < 4 ? q0[s] : q1[s], u & 3) >> (4 * h)) & 0x0F0F0F0Fu;
        if constexpr (Q5) codes |= ((word(u < 4 ? h0[s] : h1[s], u & 3) >> (2 * j + h)) & 0x01010101u) << 4;
        const float4 xv = *reinterpret_cast<const float4*>(&xlds[f32_chunk(c0 + u)]);
        a = fmaf((float)(codes & 0xFF), xv.x, a);
        a = fmaf((float)((codes >> 8) & 0xFF), xv.y, a);
        a = fmaf((float)((codes >> 16) & 0xFF), xv.z, a);
        a = fmaf((float)(codes >> 24), xv.w, a);
      }
      acc2[h] = a;
    }
    uint32_t scs, mns;
    sel.codes(hd[s], scs, mns);
    const float dd = half_bits_to_float(hd[s].x), dmin = half_bits_to_float(hd[s].x >> 16);
    total = fmaf(dd * (float)(scs & 0xFF), acc2[0], total);
    total = fmaf(dd * (float)(scs >> 8), acc2[1], total);
    total = fmaf(-dmin * (float)(mns & 0xFF), sx.x, total);
    total = fmaf(-dmin * (float)(mns >> 8), sx.y, total);
  }
  const float v = wave_sum(total);
  if (lane == 0) store_out<OutT>(out, (size_t)row, v);
}

template <int STEPS, typename OutT, int TYPE>
static void launch_m1_f32_steps(const GemvArgs& a, hipStream_t stream) {
  constexpr int WAVES = 8;
  hipLaunchKernelGGL((gemv_q4k_m1_f32<STEPS, WAVES, OutT, TYPE>), dim3((a.n + WAVES - 1) / WAVES), dim3(WAVES * 64),
                     0, stream, static_cast<const float*>(a.x), static_cast<const uint8_t*>(a.w),
                     static_cast<OutT*>(a.out), a.n);
}

template <typename OutT, int TYPE>
static hipError_t launch_m1_f32(const GemvArgs& a, hipStream_t stream) {
  switch (a.k / 4096) {
    case 1: launch_m1_f32_steps<1, OutT, TYPE>(a, stream); break;
    case 2: launch_m1_f32_steps<2, OutT, TYPE>(a, stream); break;
    case 3: launch_m1_f32_steps<3, OutT, TYPE>(a, stream); break;
    case 4: launch_m1_f32_steps<4, OutT, TYPE>(a, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Q4_K and Q5_K with fp32 x at M = 1, K a multiple of 4096 up to 16384.
hipError_t launch_gemv_q4k_f32x(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = (a.type == kQ4_K || a.type == kQ5_K) && a.x_f32 && gemv_q4k_group_supported(a.m, a.k, a.n);
  if (!*handled) return hipSuccess;
  if (a.type == kQ5_K)
    return a.out_half ? launch_m1_f32<_Float16, kQ5_K>(a, stream) : launch_m1_f32<float, kQ5_K>(a, stream);
  return a.out_half ? launch_m1_f32<_Float16, kQ4_K>(a, stream) : launch_m1_f32<float, kQ4_K>(a, stream);
}

// ------------------------------------------------------- 2 <= M, MFMA ---

__device__ __forceinline__ uint32_t pk_fma(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(as_half2(a), as_half2(b), as_half2(c)));
}

__device__ __forceinline__ uint32_t half2_splat(float a) {
  const uint32_t b = __builtin_bit_cast(uint16_t, (_Float16)a);
  return b | (b << 16);
}

template <int M, int SPLIT, typename OutT>
__global__ __launch_bounds__(SPLIT * 64) void gemv_q4k_mfma(const _Float16* __restrict__ x,
                                                            const uint8_t* __restrict__ w,
                                                            OutT* __restrict__ out, int n_rows, int k) {
  __shared__ float partial[SPLIT > 1 ? SPLIT : 1][64][4];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int blocks = k >> 8;
  const uint8_t* wrow = w + (size_t)min(n0 + n, n_rows - 1) * (size_t)blocks * 144;
  const bool xrow = n < M;  // as the A operand this lane holds activation row m = n
  const uint8_t* xr = reinterpret_cast<const uint8_t*>(x + (size_t)(xrow ? n : 0) * k + 64 * g);
  const PairSelect sel(g);
  float4v_t acc = {0.f, 0.f, 0.f, 0.f}, accmin = {0.f, 0.f, 0.f, 0.f};
  for (int b = wv; b < blocks; b += SPLIT) {
    const uint8_t* blk = wrow + (size_t)b * 144;
    const uint4 hd = load16(blk);
    const uint4 q0 = load16(blk + 16 + 32 * g);
    const uint4 q1 = load16(blk + 32 + 32 * g);
    uint4 xa[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xa[i] = xrow ? load16(xr + b * 512 + 16 * i) : make_uint4(0, 0, 0, 0);
    uint32_t scs, mns;
    sel.codes(hd, scs, mns);
    const float sc_lo = (float)(scs & 0xFF), sc_hi = (float)(scs >> 8);
    // low: (1024 + q) sc - 1024 sc = sc q;  high: (1024 + 16 q) sc / 16 - 64 sc = sc q  (exact)
    const uint32_t mul_lo = half2_splat(sc_lo), add_lo = half2_splat(-1024.0f * sc_lo);
    const uint32_t mul_hi = half2_splat(sc_hi * 0.0625f), add_hi = half2_splat(-64.0f * sc_hi);
    float4v_t cs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      // MFMA t: codes of dwords 2(t%4), 2(t%4)+1 -- low nibbles for t < 4, high for t >= 4;
      // elements 8t .. 8t+7 of the lane's 64, matching x chunk t
      const int u = 2 * (t & 3);
      const uint32_t wa = word(u < 4 ? q0 : q1, u & 3), wb = word(u < 4 ? q0 : q1, (u & 3) + 1);
      const uint32_t mask = t < 4 ? 0x0F0F0F0Fu : 0xF0F0F0F0u;
      const uint32_t mul = t < 4 ? mul_lo : mul_hi, add = t < 4 ? add_lo : add_hi;
      const uint32_t ca = wa & mask, cb = wb & mask;
      const uint4 bv = make_uint4(pk_fma(magic01(ca), mul, add), pk_fma(magic23(ca), mul, add),
                                  pk_fma(magic01(cb), mul, add), pk_fma(magic23(cb), mul, add));
      cs = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, xa[t]),
                                                  __builtin_bit_cast(half8_t, bv), cs, 0, 0, 0);
    }
    const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
    acc += d * cs;
    const float sx_lo = sum16(xa[0], xa[1]) + sum16(xa[2], xa[3]);
    const float sx_hi = sum16(xa[4], xa[5]) + sum16(xa[6], xa[7]);
    accmin = __builtin_amdgcn_mfma_f32_16x16x4f32(sx_lo, dmin * (float)(mns & 0xFF), accmin, 0, 0, 0);
    accmin = __builtin_amdgcn_mfma_f32_16x16x4f32(sx_hi, dmin * (float)(mns >> 8), accmin, 0, 0, 0);
  }
  const float4v_t total = acc - accmin;
  if (SPLIT > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) partial[wv][lane][i] = total[i];
    __syncthreads();
    if (wv != 0) return;
  }
  // result tile: lane holds rows m = 4g + i of column n
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = total[i];
    if (SPLIT > 1)
#pragma unroll
      for (int p = 1; p < SPLIT; ++p) v += partial[p][lane][i];
    const int m = 4 * g + i;
    if (m < M && n0 + n < n_rows) store_out<OutT>(out, (size_t)m * n_rows + n0 + n, v);
  }
}

// Sector-aligned variant for 2 <= M <= 8 and K a multiple of 1024 (wide matrices and long
// rows).  Wave (t, q) of a workgroup owns 16-row tile t and the 576-byte range of four
// super-blocks 4q .. 4q+3 of every row; a workgroup holds TILES tiles x K/1024 waves.
// Load c (0..8) of a lane (n, g) reads the 16-byte chunk 4c + g of row n's range, so each
// load instruction covers whole 64-byte sectors of 16 rows.  Chunk 9b of the range is the
// header of super-block b; it lands in load 2b of lane g = b, so every lane holds exactly one
// header.  Quant chunk r (1..8) of a super-block is bytes 16(r-1) .. of its 128 quant bytes:
// pair j = (r-1)/2, low nibbles of sub-block 2j and high nibbles of 2j+1, elements
// 16((r-1) % 2) ..  Lane g's two quant chunks of super-block b are r and r + 4 (pairs j and
// j + 2) with r - 1 = (g - b - 1) mod 4, in loads 2b+1, 2b+2 when g <= b, else 2b, 2b+1.
//
// Each lane decodes its own header once, into a per-wave LDS table of pair entries
// {half2(sc_lo, sc_hi / 16), half2(-1024 sc_lo, -64 sc_hi), dmin m_lo, dmin m_hi} and d.  A
// code widened to fp16 "1024 + q" (low nibble) or "1024 + 16 q" (high nibble) times the
// entry's first half plus its second (each broadcast through op_sel) is the exact integer
// sc * q, so a super-block's MFMA chain takes d once at its end.  The min term is a 16x16x4
// fp32 MFMA of 16-element x sums (staged with x, a chunk's low- and high-nibble runs side by
// side) and dmin * m.  Activation rows past M read row M - 1: they reach only output rows
// that are never stored.
//
// Issue order (per-wave s_memrealtime stamps on MI355X, M = 4, 12288 x 4096).  XFIRST: x alone,
// then every weight load after the barrier that publishes x.  x then reaches LDS 1.6 us after
// launch; with the four header loads issued ahead of the barrier it took 3.3 us, with all nine
// 4.8 us (the weight bytes in flight delay it), and every wave waits for x before it computes
// (10.7 against 11.7 and 11.2 us per launch).  That holds for a grid of one workgroup per CU;
// where workgroups come in several rounds a late one would stream nothing while its x arrives,
// so those grids (!XFIRST) put all nine loads in flight behind x (grouped pair at M = 4:
// 17.2 us against 18.2 x-first).
constexpr int kSecXPad = 16;               // bytes after each LDS row of x
constexpr size_t kSecMaxLds = 160 * 1024;  // LDS of one gfx950 workgroup
constexpr int kSecTableBytes = 64 * 4 * 16 + 64 * 4;  // per wave: 4 pair entries per lane, then d per lane

// Floats per LDS row of x sums: one per 16 elements and 16 bytes of padding, so that the rows of
// one read fall in different banks.
__host__ __device__ constexpr int sec_sum_row(int k) { return (k >> 4) + 4; }

__device__ __forceinline__ uint4 select4(bool c, const uint4& a, const uint4& b) {
  return make_uint4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

// Slot of 16-element run 16 s + 4 j + 2 nib + h of a row (elements 256 s + 64 j + 32 nib + 16 h)
// in the sum table: 16 s + 4 j + 2 h + nib, the low- and high-nibble runs of a chunk side by side.
__device__ __forceinline__ int sum_slot(int run) { return (run & ~3) | ((run & 1) << 1) | ((run >> 1) & 1); }

__device__ __forceinline__ uint32_t half2_bits(half2_t v) { return __builtin_bit_cast(uint32_t, v); }

// PAIR = 1 (SwiGLU) or 2 (two outputs): the workgroup's two tile slots are tile blockIdx.x of w
// and the same tile of w2, a second matrix of the same shape. PAIR = 1: the wave that sums the w
// (gate) tile also sums the w2 (up) tile's partials and stores silu(gate) * up to out. PAIR = 2:
// each tile is stored, to out and out2 (the grouped GEMV of two equal matrices in one launch).
//
// SPLITS > 1 (x of the whole row does not fit in LDS): K is cut into SPLITS equal ranges, and
// workgroup SPLITS g + s takes range s of tile group g, staging only that range of x.  Its
// reduced tiles are fp32 partial sums, stored to part[s][m][n]; gemv_q4k_sec_reduce adds the
// ranges in order.
template <int M, typename OutT, int PAIR = 0, bool XFIRST = true, int SPLITS = 1>
__global__ __launch_bounds__(1024) void gemv_q4k_sec(const _Float16* __restrict__ x, const uint8_t* __restrict__ w,
                                                     OutT* __restrict__ out, int n_rows, int k, int tiles,
                                                     const uint8_t* __restrict__ w2 = nullptr,
                                                     OutT* __restrict__ out2 = nullptr,
                                                     float* __restrict__ part = nullptr) {
  constexpr bool SWIGLU = PAIR == 1;
  static_assert(SPLITS == 1 || PAIR == 0, "K ranges split across workgroups store one matrix's partials");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int XCH = 8;  // x chunks per thread (the host checks M * K / 8 <= XCH * threads)
  const int row_bytes = (k >> 8) * 144;  // the whole row
  const int split = SPLITS > 1 ? (int)blockIdx.x % SPLITS : 0;
  const int group = SPLITS > 1 ? (int)blockIdx.x / SPLITS : (int)blockIdx.x;
  const int kfull = k;
  if constexpr (SPLITS > 1) k /= SPLITS;  // from here on: this workgroup's K range
  const int KW = k >> 10;
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int t = wv / KW, q = wv - t * KW;
  const int threads = blockDim.x;
  const int xrow = 2 * k + kSecXPad, cpr = k >> 3, srow = sec_sum_row(k);
  uint8_t* xl = lds;                                                       // M rows of x
  float* s16 = reinterpret_cast<float*>(lds + M * xrow);                   // [M][K/16 + pad] run sums
  uint8_t* tab = lds + M * xrow + M * srow * 4 + wv * kSecTableBytes;      // this wave's header table:
  float* dtab = reinterpret_cast<float*>(tab + 64 * 4 * 16);               // entry (b, j, n), then d (b, n)

  // x chunk c = 64 wv + lane + i * threads: the 64 chunks of a wave lie in one row (K / 8 is a
  // multiple of 128), so row and bounds are wave-uniform
  uint4 xr[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int cw = wv * 64 + i * threads;
    if (cw < M * cpr) {
      if constexpr (SPLITS > 1) {
        const int m = cw / cpr;
        xr[i] = load16(reinterpret_cast<const uint8_t*>(x + (size_t)m * kfull + (size_t)split * k) +
                       16 * (size_t)(cw - m * cpr + lane));
      } else {
        xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * (size_t)(cw + lane));
      }
    }
  }
  const int tile = PAIR ? group : group * tiles + t;
  const uint8_t* base = (PAIR && t == 1 ? w2 : w) + (size_t)min(tile * 16 + n, n_rows - 1) * row_bytes +
                        (split * KW + q) * 576 + 16 * g;
  uint4 v[9];
  auto load_weights = [&]() {
#pragma unroll
    for (int c = 0; c < 8; c += 2) v[c] = load16(base + 64 * c);  // the headers first: they are decoded first
#pragma unroll
    for (int c = 1; c < 9; c += 2) v[c] = load16(base + 64 * c);
    v[8] = load16(base + 512);
  };
  if constexpr (!XFIRST) {
    // every wave's x requests enter the CU's memory pipeline ahead of its weight requests (the
    // barrier orders issue only), and the weights stream while x is staged
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    load_weights();
    asm volatile("" ::: "memory");
  }
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int cw = wv * 64 + i * threads;
    if (cw < M * cpr) {
      const int m = cw / cpr, cc = cw - m * cpr + lane;
      *reinterpret_cast<uint4*>(xl + m * xrow + 16 * cc) = xr[i];
      const uint32_t one = 0x3C003C00u;
      float s = dot2(xr[i].w, one, dot2(xr[i].z, one, dot2(xr[i].y, one, dot2(xr[i].x, one, 0.f))));
      s = dpp_add<0xB1>(s);  // + the neighbouring chunk (lane ^ 1)
      if ((lane & 1) == 0) s16[m * srow + sum_slot(cc >> 1)] = s;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if constexpr (XFIRST) {
    asm volatile("" ::: "memory");
    load_weights();
  }

  // this lane's header: row n, super-block g, in load 2g.  The selector is opaque to the
  // compiler past the barrier, so the decode cannot be hoisted above it.
  {
    int hb = g;
    asm volatile("" : "+v"(hb));
    const uint4 h = select4(hb < 2, select4(hb == 0, v[0], v[2]), select4(hb == 2, v[4], v[6]));
    const uint32_t s03 = h.y & 0x3F3F3F3Fu, m03 = h.z & 0x3F3F3F3Fu;
    const uint32_t s47 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t m47 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    const float dmin = half_bits_to_float(h.x >> 16);
    // entry (b, j, n) at 16 ((4 b + j) 16 + n): the 16 rows of one (b, j) fill all LDS banks once
    uint8_t* entry = tab + (4 * g * 16 + n) * 16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t sc = j < 2 ? s03 : s47, mn = j < 2 ? m03 : m47;
      const int shift = 16 * (j & 1);
      // fp16 1024 + sc of sub-blocks 2j and 2j + 1, then exactly (sc_lo, sc_hi / 16)
      const half2_t wide = as_half2(__builtin_amdgcn_perm(kMagic, sc, (j & 1) ? 0x04030402u : 0x04010400u));
      const half2_t mul = __builtin_elementwise_fma(wide, (half2_t){(_Float16)1.0f, (_Float16)0.0625f},
                                                    (half2_t){(_Float16)-1024.0f, (_Float16)-64.0f});
      const half2_t add = mul * (half2_t){(_Float16)-1024.0f, (_Float16)-1024.0f};
      const float mlo = dmin * (float)((mn >> shift) & 0xFF), mhi = dmin * (float)((mn >> (shift + 8)) & 0xFF);
      *reinterpret_cast<uint4*>(entry + 256 * j) =
          make_uint4(half2_bits(mul), half2_bits(add), __float_as_uint(mlo), __float_as_uint(mhi));
    }
    dtab[g * 16 + n] = half_bits_to_float(h.x);
  }
  // the table is this wave's own: LDS accesses of one wave complete in order
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");

  const int xm = min(n, M - 1);  // the activation row this lane supplies as the A operand
  const uint8_t* xn = xl + xm * xrow;
  const float* sn = s16 + xm * srow;
  float4v_t acc = {0.f, 0.f, 0.f, 0.f}, accmin = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int u = (g - b - 1) & 3;  // r - 1 of the lane's first quant chunk
    const int jf = u >> 1, h = u & 1;
    const uint4 F = select4(g <= b, v[2 * b + 1], v[2 * b]);
    const uint4 S = select4(g <= b, v[2 * b + 2], v[2 * b + 1]);
    const int sb = 4 * q + b;                    // super-block of the row
    const int e = 256 * sb + 64 * jf + 16 * h;  // first element of chunk F's low-nibble run
    const uint8_t* entries = tab + ((4 * b + jf) * 16 + n) * 16;
    const float* sums = sn + 16 * sb + 4 * jf + 2 * h;
    float4v_t cs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 2; ++c) {  // chunk F (pair jf), then S (pair jf + 2: 128 elements on)
      const uint4 C = c == 0 ? F : S;
      const uint4 E = *reinterpret_cast<const uint4*>(entries + 512 * c);
      const float2 sx = *reinterpret_cast<const float2*>(sums + 8 * c);
      const half2_t mul = as_half2(E.x), add = as_half2(E.y);
#pragma unroll
      for (int nib = 0; nib < 2; ++nib) {
        // low: (1024 + q) sc - 1024 sc = sc q;  high: (1024 + 16 q) sc / 16 - 64 sc = sc q  (exact)
        const uint32_t mask = nib == 0 ? 0x0F0F0F0Fu : 0xF0F0F0F0u;
        const half2_t m2 = nib == 0 ? mul.xx : mul.yy, a2 = nib == 0 ? add.xx : add.yy;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const uint32_t ca = word(C, 2 * p) & mask, cb = word(C, 2 * p + 1) & mask;
          const uint4 bv = make_uint4(half2_bits(__builtin_elementwise_fma(as_half2(magic01(ca)), m2, a2)),
                                      half2_bits(__builtin_elementwise_fma(as_half2(magic23(ca)), m2, a2)),
                                      half2_bits(__builtin_elementwise_fma(as_half2(magic01(cb)), m2, a2)),
                                      half2_bits(__builtin_elementwise_fma(as_half2(magic23(cb)), m2, a2)));
          const uint4 xa = *reinterpret_cast<const uint4*>(xn + 2 * (e + 128 * c + 32 * nib + 8 * p));
          cs = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, xa),
                                                      __builtin_bit_cast(half8_t, bv), cs, 0, 0, 0);
        }
        accmin = __builtin_amdgcn_mfma_f32_16x16x4f32(nib == 0 ? sx.x : sx.y, __uint_as_float(nib == 0 ? E.z : E.w),
                                                      accmin, 0, 0, 0);
      }
    }
    acc += dtab[b * 16 + n] * cs;
  }
  const float4v_t total = acc - accmin;
  __syncthreads();  // every wave is done with x: the partial tiles go over it
  float4v_t* partial = reinterpret_cast<float4v_t*>(lds);
  partial[wv * 64 + lane] = total;
  __syncthreads();
  if (q != 0 || tile * 16 >= n_rows || (SWIGLU && t != 0)) return;
  // wave (t, 0) sums its tile's K ranges in order and stores it
  float4v_t sum = partial[t * KW * 64 + lane];
  for (int p = 1; p < KW; ++p) sum += partial[(t * KW + p) * 64 + lane];
  if constexpr (SWIGLU) {
    float4v_t up = partial[KW * 64 + lane];
    for (int p = 1; p < KW; ++p) up += partial[(KW + p) * 64 + lane];
#pragma unroll
    for (int i = 0; i < 4; ++i) sum[i] = swiglu(sum[i], up[i]);
  }
  OutT* dst = PAIR == 2 && t == 1 ? out2 : out;
  const int col = tile * 16 + n;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * g + i;
    if (m < M && col < n_rows) {
      if constexpr (SPLITS > 1)
        part[((size_t)split * M + m) * n_rows + col] = sum[i];
      else
        store_out<OutT>(dst, (size_t)m * n_rows + col, sum[i]);
    }
  }
}

// out[m][c] = part[0][m][c] + .. + part[SPLITS-1][m][c], added in range order; one thread per
// output, grid (ceil(n / 256), M).
template <int SPLITS, typename OutT>
__global__ __launch_bounds__(256) void gemv_q4k_sec_reduce(const float* __restrict__ part, OutT* __restrict__ out,
                                                           int n_rows, int m_rows) {
  const int c = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
  if (c >= n_rows) return;
  const size_t plane = (size_t)m_rows * n_rows, at = (size_t)m * n_rows + c;
  float v = part[at];
#pragma unroll
  for (int s = 1; s < SPLITS; ++s) v += part[at + s * plane];
  store_out<OutT>(out, at, v);
}

// Multi-tile variant for 2 <= M <= 8 when x fits in LDS (M * K <= kMtMaxMK).
// A workgroup of W waves owns TILES 16-row tiles; wave w takes the S
// super-blocks [w S, w S + S) of every tile.  The workgroup first loads all of
// x, then every weight byte of every wave (pinned above a compiler barrier),
// and only then stages x in LDS, so the activations are not queued behind the
// weight stream on the CU.  Per super-block a wave reads its x operands from
// LDS once and reuses them for all TILES tiles; the K-split partial tiles meet
// in LDS and are summed in a fixed order.
constexpr int kMtMaxMK = 65536;     // x of up to 128 KiB in LDS
constexpr int kMtRowPad = 16;       // bytes after each LDS row of x: rows start in different banks

template <int M, int TILES, int S, typename OutT>
__global__ __launch_bounds__(1024) void gemv_q4k_mt(const _Float16* __restrict__ x, const uint8_t* __restrict__ w,
                                                    OutT* __restrict__ out, int n_rows, int k) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int W = blockDim.x >> 6;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int blocks = k >> 8;
  const size_t row_bytes = (size_t)blocks * 144;
  const int xrow_bytes = 2 * k + kMtRowPad;
  float* partial = reinterpret_cast<float*>(lds);  // [W][TILES][64][4], over x once every wave is done with it
  constexpr int XCH = 8;  // 16-byte x chunks per thread (M * K / 8 chunks over >= 512 threads)
  const int chunks = M * k / 8;

  uint4 xr[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int c = threadIdx.x + i * (int)blockDim.x;
    if (c < chunks) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * (size_t)c);
  }
  uint4 hd[TILES][S], q0[TILES][S], q1[TILES][S];
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const int row = min((blockIdx.x * TILES + t) * 16 + n, n_rows - 1);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int b = min(wv * S + s, blocks - 1);
      const uint8_t* blk = w + (size_t)row * row_bytes + (size_t)b * 144;
      hd[t][s] = load16(blk);
      q0[t][s] = load16(blk + 16 + 32 * g);
      q1[t][s] = load16(blk + 32 + 32 * g);
    }
  }
  asm volatile("" ::: "memory");
  const int chunks_per_row = k / 8;
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int c = threadIdx.x + i * (int)blockDim.x;
    if (c < chunks) {
      const int m = c / chunks_per_row, cc = c - m * chunks_per_row;
      *reinterpret_cast<uint4*>(lds + m * xrow_bytes + 16 * cc) = xr[i];
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");

  const PairSelect sel(g);
  const bool xrow = n < M;  // as the A operand this lane holds activation row m = n
  const uint8_t* xl = lds + (xrow ? n : 0) * xrow_bytes + 128 * g;
  float4v_t acc[TILES], accmin[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) acc[t] = accmin[t] = float4v_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int b = wv * S + s;
    if (b >= blocks) break;
    uint4 xa[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      xa[i] = xrow ? *reinterpret_cast<const uint4*>(xl + 512 * b + 16 * i) : make_uint4(0, 0, 0, 0);
    const float sx_lo = sum16(xa[0], xa[1]) + sum16(xa[2], xa[3]);
    const float sx_hi = sum16(xa[4], xa[5]) + sum16(xa[6], xa[7]);
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      uint32_t scs, mns;
      sel.codes(hd[t][s], scs, mns);
      const float sc_lo = (float)(scs & 0xFF), sc_hi = (float)(scs >> 8);
      // low: (1024 + q) sc - 1024 sc = sc q;  high: (1024 + 16 q) sc / 16 - 64 sc = sc q  (exact)
      const uint32_t mul_lo = half2_splat(sc_lo), add_lo = half2_splat(-1024.0f * sc_lo);
      const uint32_t mul_hi = half2_splat(sc_hi * 0.0625f), add_hi = half2_splat(-64.0f * sc_hi);
      float4v_t cs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int v = 2 * (u & 3);
        const uint32_t wa = word(v < 4 ? q0[t][s] : q1[t][s], v & 3), wb = word(v < 4 ? q0[t][s] : q1[t][s], (v & 3) + 1);
        const uint32_t mask = u < 4 ? 0x0F0F0F0Fu : 0xF0F0F0F0u;
        const uint32_t mul = u < 4 ? mul_lo : mul_hi, add = u < 4 ? add_lo : add_hi;
        const uint32_t ca = wa & mask, cb = wb & mask;
        const uint4 bv = make_uint4(pk_fma(magic01(ca), mul, add), pk_fma(magic23(ca), mul, add),
                                    pk_fma(magic01(cb), mul, add), pk_fma(magic23(cb), mul, add));
        cs = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, xa[u]),
                                                    __builtin_bit_cast(half8_t, bv), cs, 0, 0, 0);
      }
      const float d = half_bits_to_float(hd[t][s].x), dmin = half_bits_to_float(hd[t][s].x >> 16);
      acc[t] += d * cs;
      accmin[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(sx_lo, dmin * (float)(mns & 0xFF), accmin[t], 0, 0, 0);
      accmin[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(sx_hi, dmin * (float)(mns >> 8), accmin[t], 0, 0, 0);
    }
  }
  __syncthreads();  // every wave has read its last x operands
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const float4v_t total = acc[t] - accmin[t];
#pragma unroll
    for (int i = 0; i < 4; ++i) partial[((wv * TILES + t) * 64 + lane) * 4 + i] = total[i];
  }
  __syncthreads();
  // wave t sums tile t over the W K-slices in order and stores it
  for (int t = wv; t < TILES; t += W) {
    const int col = (blockIdx.x * TILES + t) * 16 + n;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = 0.f;
      for (int p = 0; p < W; ++p) v += partial[((p * TILES + t) * 64 + lane) * 4 + i];
      const int m = 4 * g + i;
      if (m < M && col < n_rows) store_out<OutT>(out, (size_t)m * n_rows + col, v);
    }
  }
}

// ---------------------------------------------------------------- launch ---

// Arguments of one M = 1 launch: up to three matrices sharing x (unused slots repeat matrix 0,
// which the kernel never selects).
template <typename OutT>
struct M1Launch {
  const _Float16* x;
  const uint8_t* w[kGemvGroupMax];
  int n[kGemvGroupMax];
  OutT* out[kGemvGroupMax];
};

// Grids of at most this many waves are resident at once (four per SIMD on 256 CUs).
constexpr unsigned kOneRoundWaves = 256 * 16;

template <int STEPS, int WAVES, int MATS, typename OutT, bool SWIGLU, int TYPE>
static void launch_m1_kernel(const M1Launch<OutT>& l, dim3 grid, hipStream_t stream) {
  if (!SWIGLU && grid.x * WAVES <= kOneRoundWaves)
    hipLaunchKernelGGL((gemv_q4k_m1<STEPS, WAVES, MATS, OutT, SWIGLU, TYPE, !SWIGLU>), grid, dim3(WAVES * 64), 0, stream,
                       l.x, l.w[0], l.w[1], l.w[2], l.n[0], l.n[1], l.n[2], l.out[0], l.out[1], l.out[2]);
  else
    hipLaunchKernelGGL((gemv_q4k_m1<STEPS, WAVES, MATS, OutT, SWIGLU, TYPE>), grid, dim3(WAVES * 64), 0, stream, l.x,
                       l.w[0], l.w[1], l.w[2], l.n[0], l.n[1], l.n[2], l.out[0], l.out[1], l.out[2]);
}

template <int WAVES, int MATS, typename OutT, bool SWIGLU, int TYPE>
static hipError_t launch_m1(const M1Launch<OutT>& l, int k, dim3 grid, hipStream_t stream) {
  switch (k / 4096) {
    case 1: launch_m1_kernel<1, WAVES, MATS, OutT, SWIGLU, TYPE>(l, grid, stream); break;
    case 2: launch_m1_kernel<2, WAVES, MATS, OutT, SWIGLU, TYPE>(l, grid, stream); break;
    case 3: launch_m1_kernel<3, WAVES, MATS, OutT, SWIGLU, TYPE>(l, grid, stream); break;
    case 4: launch_m1_kernel<4, WAVES, MATS, OutT, SWIGLU, TYPE>(l, grid, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int WAVES, typename OutT, int TYPE = kQ4_K>
static hipError_t launch_m1_waves(const GemvArgs* a, int count, hipStream_t stream) {
  if (count < 1 || count > kGemvGroupMax) return hipErrorInvalidValue;
  M1Launch<OutT> l{};
  l.x = static_cast<const _Float16*>(a[0].x);
  unsigned blocks = 0;
  for (int i = 0; i < kGemvGroupMax; ++i) {
    const GemvArgs& m = a[i < count ? i : 0];
    l.w[i] = static_cast<const uint8_t*>(m.w);
    l.out[i] = static_cast<OutT*>(m.out);
    l.n[i] = m.n;
    if (i < count) blocks += (unsigned)((m.n + WAVES - 1) / WAVES);
  }
  const dim3 grid(blocks);
  switch (count) {
    case 1: return launch_m1<WAVES, 1, OutT, false, TYPE>(l, a[0].k, grid, stream);
    case 2: return launch_m1<WAVES, 2, OutT, false, TYPE>(l, a[0].k, grid, stream);
    default: return launch_m1<WAVES, 3, OutT, false, TYPE>(l, a[0].k, grid, stream);
  }
}

// Rows per workgroup (measured on MI355X, M = 1, back-to-back launches on rotated weights):
// 4 for K = 4096 groups of 8193..16384 rows (12288 rows: 6.21 us at 4, 6.38 at 8 and 16;
// 16384: 7.64 at 4, 7.70 at 8, 8.37 at 16), else 8 (4096 rows: 3.30 at 8, 3.29 at 16, 3.63
// at 4; 6144: 4.09 at 8, 4.20 at 16; gate + up 24576: 10.33 at 8, 10.41 at 4, 11.6 at 16;
// down 4096 x 12288: 6.63 at 8, 7.00 at 4, 7.37 at 16).
static int m1_waves(const GemvArgs* a, int count) {
  long rows = 0;
  for (int i = 0; i < count; ++i) rows += a[i].n;
  return a[0].k == 4096 && rows > 8192 && rows <= 16384 ? 4 : 8;
}

template <typename OutT, int TYPE = kQ4_K>
static hipError_t launch_m1_group(const GemvArgs* a, int count, hipStream_t stream, int waves = 0) {
  switch (waves > 0 ? waves : m1_waves(a, count)) {
    case 4: return launch_m1_waves<4, OutT, TYPE>(a, count, stream);
    case 8: return launch_m1_waves<8, OutT, TYPE>(a, count, stream);
    case 16: return launch_m1_waves<16, OutT, TYPE>(a, count, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int M, typename OutT>
static hipError_t launch_mfma(const GemvArgs& a, hipStream_t stream, int waves) {
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const int tiles = (a.n + 15) / 16;
  if (waves == 8)
    hipLaunchKernelGGL((gemv_q4k_mfma<M, 8, OutT>), dim3(tiles), dim3(8 * 64), 0, stream, x, w, out, a.n, a.k);
  else
    hipLaunchKernelGGL((gemv_q4k_mfma<M, 4, OutT>), dim3(tiles), dim3(4 * 64), 0, stream, x, w, out, a.n, a.k);
  return hipGetLastError();
}

template <int M, int TILES, int S, typename OutT>
static hipError_t launch_mt_cfg(const GemvArgs& a, hipStream_t stream) {
  const int blocks = a.k / 256, waves = (blocks + S - 1) / S;
  const int tiles = (a.n + 16 * TILES - 1) / (16 * TILES);
  const size_t lds = std::max((size_t)M * (2 * a.k + kMtRowPad), (size_t)waves * TILES * 64 * 4 * sizeof(float));
  hipLaunchKernelGGL((gemv_q4k_mt<M, TILES, S, OutT>), dim3(tiles), dim3(waves * 64), lds, stream,
                     static_cast<const _Float16*>(a.x), static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out),
                     a.n, a.k);
  return hipGetLastError();
}

template <int M, typename OutT>
static hipError_t launch_mt(const GemvArgs& a, hipStream_t stream, int tiles, int s) {
  if (s == 2) return tiles == 2 ? launch_mt_cfg<M, 2, 2, OutT>(a, stream) : launch_mt_cfg<M, 1, 2, OutT>(a, stream);
  return tiles == 2 ? launch_mt_cfg<M, 2, 3, OutT>(a, stream) : launch_mt_cfg<M, 1, 3, OutT>(a, stream);
}

// x rows, the 16-element x sums and one header table per wave; the partial tiles of the
// epilogue go over x.
static size_t sec_lds_bytes(int m, int k, int waves) {
  const size_t staged = (size_t)m * (2 * k + kSecXPad) + (size_t)m * sec_sum_row(k) * sizeof(float) +
                        (size_t)waves * kSecTableBytes;
  return std::max(staged, (size_t)waves * 64 * sizeof(float4v_t));
}

template <int M, typename OutT>
static hipError_t launch_sec(const GemvArgs& a, hipStream_t stream, int per, bool xfirst) {
  const int kw = a.k / 1024, tiles = (a.n + 15) / 16, threads = per * kw * 64;
  const size_t lds = sec_lds_bytes(M, a.k, per * kw);
  const int grid = (tiles + per - 1) / per;
  if (xfirst)
    hipLaunchKernelGGL((gemv_q4k_sec<M, OutT, 0, true>), dim3(grid), dim3(threads), lds, stream,
                       static_cast<const _Float16*>(a.x), static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out),
                       a.n, a.k, per);
  else
    hipLaunchKernelGGL((gemv_q4k_sec<M, OutT, 0, false>), dim3(grid), dim3(threads), lds, stream,
                       static_cast<const _Float16*>(a.x), static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out),
                       a.n, a.k, per);
  return hipGetLastError();
}

// Bytes of fp32 partial sums a K split into `splits` ranges stores.
static size_t sec_split_bytes(const GemvArgs& a, int splits) { return (size_t)splits * a.m * a.n * sizeof(float); }

// K cut into `splits` ranges across workgroups (per tiles each), then the ranges added in order.
template <int M, int SPLITS, typename OutT>
static hipError_t launch_sec_split_cfg(const GemvArgs& a, hipStream_t stream, int per) {
  const int ks = a.k / SPLITS, kw = ks / 1024, tiles = (a.n + 15) / 16, threads = per * kw * 64;
  const size_t lds = sec_lds_bytes(M, ks, per * kw);
  const int groups = (tiles + per - 1) / per;
  float* part = static_cast<float*>(a.workspace);
  hipLaunchKernelGGL((gemv_q4k_sec<M, OutT, 0, true, SPLITS>), dim3(groups * SPLITS), dim3(threads), lds, stream,
                     static_cast<const _Float16*>(a.x), static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out),
                     a.n, a.k, per, nullptr, nullptr, part);
  hipError_t status = hipGetLastError();
  if (status != hipSuccess) return status;
  hipLaunchKernelGGL((gemv_q4k_sec_reduce<SPLITS, OutT>), dim3((a.n + 255) / 256, M), dim3(256), 0, stream, part,
                     static_cast<OutT*>(a.out), a.n, M);
  return hipGetLastError();
}

template <int M, typename OutT>
static hipError_t launch_sec_split(const GemvArgs& a, hipStream_t stream, int per, int splits) {
  if constexpr (M < 4) {
    return hipErrorInvalidValue;  // x of M <= 3 rows fits without a split
  } else {
    if (!a.workspace || a.workspace_bytes < sec_split_bytes(a, splits)) return hipErrorInvalidValue;
    return splits == 2 ? launch_sec_split_cfg<M, 2, OutT>(a, stream, per)
                       : launch_sec_split_cfg<M, 4, OutT>(a, stream, per);
  }
}

// SwiGLU pairs at 2 <= M <= 8 on the sector-aligned kernel: one gate tile and the same up tile
// per workgroup (2 x K/1024 waves, so K <= 8192), x in LDS.
template <int M, typename OutT, int PAIR>
static hipError_t launch_sec_pair(const GemvArgs& a, const void* w2, void* out2, hipStream_t stream, bool* handled) {
  *handled = false;
  const int kw = a.k / 1024, tiles = (a.n + 15) / 16, threads = 2 * kw * 64;
  if (a.k % 1024 != 0 || kw > 8) return hipSuccess;
  const size_t lds = sec_lds_bytes(M, a.k, 2 * kw);
  if ((long)M * a.k / 8 > 8L * threads || lds > kSecMaxLds) return hipSuccess;
  *handled = true;
  hipLaunchKernelGGL((gemv_q4k_sec<M, OutT, PAIR, false>), dim3(tiles), dim3(threads), lds, stream,
                     static_cast<const _Float16*>(a.x), static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out),
                     a.n, a.k, 2, static_cast<const uint8_t*>(w2), static_cast<OutT*>(out2));
  return hipGetLastError();
}

template <typename OutT, int PAIR>
static hipError_t launch_pair_multirow(const GemvArgs& a, const void* w2, void* out2, hipStream_t stream,
                                       bool* handled) {
  switch (a.m) {
    case 2: return launch_sec_pair<2, OutT, PAIR>(a, w2, out2, stream, handled);
    case 3: return launch_sec_pair<3, OutT, PAIR>(a, w2, out2, stream, handled);
    case 4: return launch_sec_pair<4, OutT, PAIR>(a, w2, out2, stream, handled);
    case 5: return launch_sec_pair<5, OutT, PAIR>(a, w2, out2, stream, handled);
    case 6: return launch_sec_pair<6, OutT, PAIR>(a, w2, out2, stream, handled);
    case 7: return launch_sec_pair<7, OutT, PAIR>(a, w2, out2, stream, handled);
    case 8: return launch_sec_pair<8, OutT, PAIR>(a, w2, out2, stream, handled);
    default: *handled = false; return hipSuccess;
  }
}

template <int M, typename OutT>
static hipError_t launch_plan_typed(const GemvArgs& a, const GemvPlan& plan, hipStream_t stream) {
  switch (plan.kernel) {
    case kGemvSec: return launch_sec<M, OutT>(a, stream, plan.a, plan.b != 0);
    case kGemvMt: return launch_mt<M, OutT>(a, stream, plan.a, plan.b);
    case kGemvSecSplit: return launch_sec_split<M, OutT>(a, stream, plan.a, plan.b);
    default: return launch_mfma<M, OutT>(a, stream, plan.a);
  }
}

template <typename OutT>
static hipError_t launch_plan_m(const GemvArgs& a, const GemvPlan& plan, hipStream_t stream) {
  switch (a.m) {
    case 2: return launch_plan_typed<2, OutT>(a, plan, stream);
    case 3: return launch_plan_typed<3, OutT>(a, plan, stream);
    case 4: return launch_plan_typed<4, OutT>(a, plan, stream);
    case 5: return launch_plan_typed<5, OutT>(a, plan, stream);
    case 6: return launch_plan_typed<6, OutT>(a, plan, stream);
    case 7: return launch_plan_typed<7, OutT>(a, plan, stream);
    default: return launch_plan_typed<8, OutT>(a, plan, stream);
  }
}

// Launch limits of each multi-row kernel (what its indexing and LDS layout assume).
static bool sec_fits(const GemvArgs& a, int per) {
  const int kw = a.k / 1024;
  if (a.k % 1024 != 0 || kw < 1 || kw > 16 || per < 1 || per > 3 || per * kw > 16) return false;
  const int threads = per * kw * 64;
  // x is staged with eight 16-byte chunks per thread at most, and must fit in LDS with its sums
  return (long)a.m * a.k / 8 <= 8L * threads && sec_lds_bytes(a.m, a.k, per * kw) <= kSecMaxLds;
}

// The K-split form: M >= 4 (the instantiated range), 2 or 4 ranges of whole 1024-column
// sectors, at most 16 waves, x of one range staged like the unsplit kernel's, and partial sums
// within 32-bit offsets.
static bool sec_split_fits(const GemvArgs& a, int per, int splits) {
  if (a.m < 4 || (splits != 2 && splits != 4) || a.k % (1024 * splits) != 0) return false;
  const int ks = a.k / splits, kw = ks / 1024;
  if (per < 1 || per * kw > 16 || sec_split_bytes(a, splits) >= (1ull << 31)) return false;
  const int threads = per * kw * 64;
  return (long)a.m * ks / 8 <= 8L * threads && sec_lds_bytes(a.m, ks, per * kw) <= kSecMaxLds;
}

static bool mt_fits(const GemvArgs& a, int tiles, int s) {
  if (a.k % 256 != 0 || (tiles != 1 && tiles != 2) || (s != 2 && s != 3)) return false;
  const int waves = (a.k / 256 + s - 1) / s;
  // at most 16 waves and at most 8 x chunks per thread; x in LDS
  return waves <= 16 && (long)a.m * a.k <= kMtMaxMK && (long)a.m * a.k / 8 <= (long)waves * 64 * 8;
}

bool gemv_q4k_plan_fits(const GemvArgs& a, const GemvPlan& plan) {
  if (a.type != kQ4_K || a.x_f32 || a.m < 2 || a.m > 8 || a.k % 256 != 0 || a.n < 1) return false;
  switch (plan.kernel) {
    case kGemvSec: return (plan.b == 0 || plan.b == 1) && sec_fits(a, plan.a);
    case kGemvMt: return mt_fits(a, plan.a, plan.b);
    case kGemvMfma: return (plan.a == 4 || plan.a == 8) && plan.b == 0;
    case kGemvSecSplit: return sec_split_fits(a, plan.a, plan.b);
    default: return false;
  }
}

size_t gemv_q4k_plan_workspace(const GemvArgs& a, const GemvPlan& plan) {
  return plan.kernel == kGemvSecSplit ? sec_split_bytes(a, plan.b) : 0;
}

// The library's multi-row plan.  Sector-aligned kernel for matrices of at least 512 tiles
// (gate / up, 12288 x 4096: 11.0 us at M = 4 against 12.8 us for gemv_q4k_mt) and rows of at
// least 8192 columns (down, 4096 x 12288: 12.5 against 14.5 us), three tiles per workgroup when
// that still gives 256 workgroups (so every CU holds one), x first only where every workgroup
// starts at once (at most one per CU of the 256) and x is at most 32 KB (M = 4 gate: 10.4 against
// 10.7-11.0 us; with 64 KB at the M = 8 gate or 96 KB at the M = 4 down, the weights issued behind x
// run 1-3% faster in the plan sweep and a timing harness); shorter and narrower shapes take
// gemv_q4k_mt (4096 x 4096: 6.1 us both) with x in LDS, 2 super-blocks per wave up to K = 8192
// and 3 up to 12288, two tiles per workgroup from 8192 rows.  Long rows whose x does not fit in
// LDS (M = 8 down, 4096 x 12288: 196 KB of x) split K across workgroups when that gives one round
// of 128 to 256 workgroups, the most workgroups first, then the shorter ranges of x (M = 8 down: 4 ranges
// of 3 sectors, 4 tiles per workgroup, 256 workgroups; 13.2 against 16.5 us for gemv_q4k_mfma
// with the reduce, in a timing harness); it needs a workspace, which the entry points give from
// the library's scratch.  Else gemv_q4k_mfma, K split over 8 waves up to 512 tiles (about 12
// waves per CU on 256 CUs), else over 4.
bool gemv_q4k_plan(const GemvArgs& a, GemvPlan* plan) {
  if (a.type != kQ4_K || a.x_f32 || a.m < 2 || a.m > 8 || a.k % 256 != 0) return false;
  const int kw = a.k / 1024, tiles = (a.n + 15) / 16, blocks = a.k / 256;
  if (a.k % 1024 == 0 && (tiles >= 512 || kw >= 8)) {
    const int per = tiles >= 768 && 3 * kw <= 16 ? 3 : tiles >= 512 && 2 * kw <= 16 ? 2 : 1;
    if (sec_fits(a, per)) {
      const bool xfirst = (tiles + per - 1) / per <= 256 && (long)a.m * a.k * 2 <= 32 * 1024;
      *plan = GemvPlan{kGemvSec, per, xfirst ? 1 : 0};
      return true;
    }
    if (kw >= 8) {
      GemvPlan best{-1, 0, 0};
      int best_grid = 127;
      for (int splits = 4; splits >= 2; splits -= 2)
        for (int p = 1; p <= 16; ++p) {
          const long grid = (long)((tiles + p - 1) / p) * splits;
          if (grid > 256 || grid <= best_grid || !sec_split_fits(a, p, splits)) continue;
          best = GemvPlan{kGemvSecSplit, p, splits};
          best_grid = (int)grid;
        }
      if (best.kernel == kGemvSecSplit) {
        *plan = best;
        return true;
      }
    }
  }
  const GemvPlan mt{kGemvMt, a.n >= 8192 ? 2 : 1, blocks <= 32 ? 2 : 3};
  if (mt_fits(a, mt.a, mt.b)) {
    *plan = mt;
    return true;
  }
  *plan = GemvPlan{kGemvMfma, tiles <= 512 ? 8 : 4, 0};
  return true;
}

hipError_t launch_gemv_q4k_plan(const GemvArgs& a, const GemvPlan& plan, hipStream_t stream) {
  if (!gemv_q4k_plan_fits(a, plan)) return hipErrorInvalidValue;
  return a.out_half ? launch_plan_m<_Float16>(a, plan, stream) : launch_plan_m<float>(a, plan, stream);
}

template <typename OutT>
static hipError_t launch_typed(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = true;
  if (gemv_q4k_group_supported(a.m, a.k, a.n)) return launch_m1_group<OutT>(&a, 1, stream);
  GemvPlan plan;
  if (!gemv_q4k_plan(a, &plan)) {
    *handled = false;
    return hipSuccess;
  }
  // a call without a workspace runs the plan that reads x per wave
  if (plan.kernel == kGemvSecSplit && (!a.workspace || a.workspace_bytes < gemv_q4k_plan_workspace(a, plan)))
    plan = GemvPlan{kGemvMfma, (a.n + 15) / 16 <= 512 ? 8 : 4, 0};
  return launch_plan_m<OutT>(a, plan, stream);
}

// Q5_K at M = 1 (K a multiple of 4096, at most 16384): the M = 1 kernel with the fifth bits.
hipError_t launch_gemv_q5k_fast(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = gemv_q4k_group_supported(a.m, a.k, a.n);
  if (!*handled) return hipSuccess;
  return a.out_half ? launch_m1_group<_Float16, kQ5_K>(&a, 1, stream) : launch_m1_group<float, kQ5_K>(&a, 1, stream);
}

hipError_t launch_gemv_q4k_fast(const GemvArgs& a, hipStream_t stream, bool* handled) {
  return a.out_half ? launch_typed<_Float16>(a, stream, handled) : launch_typed<float>(a, stream, handled);
}

// The kernel addresses a matrix with 32-bit byte offsets: n rows of K / 256 blocks of at most 176
// bytes (Q5_K) must stay below 4 GiB.
bool gemv_q4k_group_supported(int m, int k, int n) {
  return m == 1 && k % 4096 == 0 && k <= 4 * 4096 && (uint64_t)n * (uint64_t)(k / 256) * 176u < (1ull << 32);
}

// Up to M = 4 (gate + up 2 x 12288 x 4096 at M = 4: 17.4 us against 21.4 us for two launches; at
// M = 8 the 64 KB of x staged for two tiles per workgroup makes the pair slower, 24.6 against 23.1).
bool gemv_q4k_pair_supported(const GemvArgs* a, int count) {
  return count == 2 && a[0].type == kQ4_K && a[0].m >= 2 && a[0].m <= 4 && a[1].n == a[0].n &&
         a[0].k % 1024 == 0 && a[0].k <= 8192;
}

hipError_t launch_gemv_q4k_pair(const GemvArgs* a, hipStream_t stream, bool* handled) {
  return a[0].out_half ? launch_pair_multirow<_Float16, 2>(a[0], a[1].w, a[1].out, stream, handled)
                       : launch_pair_multirow<float, 2>(a[0], a[1].w, a[1].out, stream, handled);
}

hipError_t launch_gemv_q4k_group(const GemvArgs* a, int count, hipStream_t stream, int waves) {
  if (a[0].type == kQ5_K)
    return a[0].out_half ? launch_m1_group<_Float16, kQ5_K>(a, count, stream, waves)
                         : launch_m1_group<float, kQ5_K>(a, count, stream, waves);
  return a[0].out_half ? launch_m1_group<_Float16>(a, count, stream, waves) : launch_m1_group<float>(a, count, stream, waves);
}

// M = 1 SwiGLU pairs: WAVES / 2 gate rows and the same up rows per workgroup.
template <int WAVES, typename OutT, int TYPE>
static hipError_t launch_m1_swiglu(const GemvArgs& a, const void* w_up, hipStream_t stream) {
  M1Launch<OutT> l{};
  l.x = static_cast<const _Float16*>(a.x);
  l.w[0] = static_cast<const uint8_t*>(a.w);
  l.w[1] = l.w[2] = static_cast<const uint8_t*>(w_up);
  l.out[0] = l.out[1] = l.out[2] = static_cast<OutT*>(a.out);
  l.n[0] = l.n[1] = l.n[2] = a.n;
  const dim3 grid((unsigned)((a.n + WAVES / 2 - 1) / (WAVES / 2)));
  return launch_m1<WAVES, 2, OutT, true, TYPE>(l, a.k, grid, stream);
}

template <typename OutT, int TYPE>
static hipError_t launch_m1_swiglu_waves(const GemvArgs& a, const void* w_up, hipStream_t stream, int waves) {
  switch (waves > 0 ? waves : 8) {
    case 8: return launch_m1_swiglu<8, OutT, TYPE>(a, w_up, stream);
    case 16: return launch_m1_swiglu<16, OutT, TYPE>(a, w_up, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv_q4k_swiglu_fast(const GemvArgs& a, const void* w_up, hipStream_t stream, bool* handled,
                                       int waves) {
  if (a.type == kQ4_K && a.m >= 2)
    return a.out_half ? launch_pair_multirow<_Float16, 1>(a, w_up, nullptr, stream, handled)
                      : launch_pair_multirow<float, 1>(a, w_up, nullptr, stream, handled);
  *handled = gemv_q4k_group_supported(a.m, a.k, a.n);
  if (!*handled) return hipSuccess;
  if (a.type == kQ5_K)
    return a.out_half ? launch_m1_swiglu_waves<_Float16, kQ5_K>(a, w_up, stream, waves)
                      : launch_m1_swiglu_waves<float, kQ5_K>(a, w_up, stream, waves);
  return a.out_half ? launch_m1_swiglu_waves<_Float16, kQ4_K>(a, w_up, stream, waves)
                    : launch_m1_swiglu_waves<float, kQ4_K>(a, w_up, stream, waves);
}

}  // namespace tensor_gguf
