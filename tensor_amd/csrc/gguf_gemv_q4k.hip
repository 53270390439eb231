// Q4_K decode GEMV fast paths (gfx950), out[m, n] = sum_k x[m, k] * W[n, k].
//
// Two kernels replace the generic VALU GEMV for Q4_K:
//
//  * M = 1, K a multiple of 4096: gemv_q4k_lds.  A 512-thread workgroup stages
//    x once in LDS (padded 16 B per 128 B so the wave's b128 reads are
//    conflict-free) while the weight loads of its 16 rows are already in
//    flight.  Lane = (super-block slot 0..15, quant pair j 0..3): each lane
//    decodes 64 codes per row and super-block, unpacks its two sub-blocks'
//    6-bit scale/min pairs once, and accumulates with v_dot2_f32_f16 on
//    "1024 + q" (low nibbles) and "1024 + 16 q" (high nibbles, left in place)
//    fp16 codes; the bias is removed per sub-block with the sum of x.
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
//
// Block format and element formula: benchmarks/kernels/showcase/triton_kernels.py:143-162.
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

__device__ __forceinline__ float dpp_row_sum(float v) {
  // within each 16-lane row: xor 1, xor 2, half mirror, mirror
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
  return v;
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_row_sum(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// ------------------------------------------------------- M = 1, LDS x ---

template <int STEPS>
struct Q4KRow {
  uint4 hd[STEPS], q0[STEPS], q1[STEPS];
};

template <int STEPS>
__device__ __forceinline__ float q4k_row_dot(const Q4KRow<STEPS>& d, const uint4 (&xs)[STEPS][8],
                                             const float (&sx)[STEPS][2], const PairSelect& sel) {
  float total = 0.f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    float al = 0.f, ah = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const uint32_t q = word(u < 4 ? d.q0[s] : d.q1[s], u & 3);
      const uint32_t lo = q & 0x0F0F0F0Fu, hi = q & 0xF0F0F0F0u;
      al = dot2(magic01(lo), word(xs[s][u >> 1], 2 * (u & 1)), al);
      al = dot2(magic23(lo), word(xs[s][u >> 1], 2 * (u & 1) + 1), al);
      ah = dot2(magic01(hi), word(xs[s][4 + (u >> 1)], 2 * (u & 1)), ah);
      ah = dot2(magic23(hi), word(xs[s][4 + (u >> 1)], 2 * (u & 1) + 1), ah);
    }
    uint32_t scs, mns;
    sel.codes(d.hd[s], scs, mns);
    const float dd = half_bits_to_float(d.hd[s].x), dmin = half_bits_to_float(d.hd[s].x >> 16);
    const float ds_lo = dd * (float)(scs & 0xFF), ds_hi = dd * (float)(scs >> 8) * 0.0625f;
    const float dm_lo = dmin * (float)(mns & 0xFF), dm_hi = dmin * (float)(mns >> 8);
    // al = sum x (1024 + q), ah = sum x (1024 + 16 q)
    total = fmaf(ds_lo, al - 1024.0f * sx[s][0], total);
    total = fmaf(-dm_lo, sx[s][0], total);
    total = fmaf(ds_hi, ah - 1024.0f * sx[s][1], total);
    total = fmaf(-dm_hi, sx[s][1], total);
  }
  return total;
}

constexpr int kLdsWaves = 8, kLdsRows = 2;

template <int STEPS, typename OutT>
__global__ __launch_bounds__(kLdsWaves * 64) void gemv_q4k_lds(const _Float16* __restrict__ x,
                                                               const uint8_t* __restrict__ w,
                                                               OutT* __restrict__ out, int n_rows) {
  constexpr int K = STEPS * 4096;
  constexpr int ROW_BYTES = STEPS * 16 * 144;
  __shared__ __attribute__((aligned(16))) uint8_t xlds[K * 2 + K / 4];
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * kLdsWaves + (threadIdx.x >> 6)) * kLdsRows;
  const int slot = lane >> 2, j = lane & 3;
  const uint8_t* wl = w + slot * 144;  // super-block start
  const uint8_t* wq = wl + 32 * j;     // this lane's 32 quant bytes at +16
  Q4KRow<STEPS> rd[kLdsRows];
#pragma unroll
  for (int r = 0; r < kLdsRows; ++r) {
    const size_t base = (size_t)min(row0 + r, n_rows - 1) * ROW_BYTES;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      rd[r].hd[s] = load16(wl + base + s * 2304);
      rd[r].q0[s] = load16(wq + base + s * 2304 + 16);
      rd[r].q1[s] = load16(wq + base + s * 2304 + 32);
    }
  }
  // x chunk c (16 B) -> LDS byte 16 c + 16 (c / 8)
  for (int c = threadIdx.x; c < K / 8; c += kLdsWaves * 64)
    *reinterpret_cast<uint4*>(xlds + 16 * c + 16 * (c >> 3)) = load16(reinterpret_cast<const uint8_t*>(x) + 16 * c);
  __syncthreads();
  if (row0 >= n_rows) return;
  uint4 xs[STEPS][8];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int c0 = ((s * 16 + slot) * 256 + 64 * j) >> 3;
#pragma unroll
    for (int i = 0; i < 8; ++i) xs[s][i] = *reinterpret_cast<const uint4*>(xlds + 16 * (c0 + i) + 16 * ((c0 + i) >> 3));
  }
  float sx[STEPS][2];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    sx[s][0] = sum16(xs[s][0], xs[s][1]) + sum16(xs[s][2], xs[s][3]);
    sx[s][1] = sum16(xs[s][4], xs[s][5]) + sum16(xs[s][6], xs[s][7]);
  }
  const PairSelect sel(j);
#pragma unroll
  for (int r = 0; r < kLdsRows; ++r) {
    const float v = wave_sum_dpp(q4k_row_dot<STEPS>(rd[r], xs, sx, sel));
    if (lane == 0 && row0 + r < n_rows) store_out<OutT>(out, (size_t)(row0 + r), v);
  }
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

// ---------------------------------------------------------------- launch ---

template <typename OutT>
static hipError_t launch_lds(const GemvArgs& a, hipStream_t stream) {
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const dim3 grid((a.n + kLdsWaves * kLdsRows - 1) / (kLdsWaves * kLdsRows)), block(kLdsWaves * 64);
  switch (a.k / 4096) {
    case 1: hipLaunchKernelGGL((gemv_q4k_lds<1, OutT>), grid, block, 0, stream, x, w, out, a.n); break;
    case 2: hipLaunchKernelGGL((gemv_q4k_lds<2, OutT>), grid, block, 0, stream, x, w, out, a.n); break;
    case 3: hipLaunchKernelGGL((gemv_q4k_lds<3, OutT>), grid, block, 0, stream, x, w, out, a.n); break;
    case 4: hipLaunchKernelGGL((gemv_q4k_lds<4, OutT>), grid, block, 0, stream, x, w, out, a.n); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int M, typename OutT>
static hipError_t launch_mfma(const GemvArgs& a, hipStream_t stream) {
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const int tiles = (a.n + 15) / 16;
  // split K so the grid holds roughly 12 waves per CU on a 256-CU part
  if (tiles <= 512)
    hipLaunchKernelGGL((gemv_q4k_mfma<M, 8, OutT>), dim3(tiles), dim3(8 * 64), 0, stream, x, w, out, a.n, a.k);
  else
    hipLaunchKernelGGL((gemv_q4k_mfma<M, 4, OutT>), dim3(tiles), dim3(4 * 64), 0, stream, x, w, out, a.n, a.k);
  return hipGetLastError();
}

template <typename OutT>
static hipError_t launch_typed(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = true;
  if (a.m == 1 && a.k % 4096 == 0 && a.k <= 4 * 4096) return launch_lds<OutT>(a, stream);
  switch (a.m) {
    case 2: return launch_mfma<2, OutT>(a, stream);
    case 3: return launch_mfma<3, OutT>(a, stream);
    case 4: return launch_mfma<4, OutT>(a, stream);
    case 5: return launch_mfma<5, OutT>(a, stream);
    case 6: return launch_mfma<6, OutT>(a, stream);
    case 7: return launch_mfma<7, OutT>(a, stream);
    case 8: return launch_mfma<8, OutT>(a, stream);
    default: *handled = false; return hipSuccess;
  }
}

hipError_t launch_gemv_q4k_fast(const GemvArgs& a, hipStream_t stream, bool* handled) {
  return a.out_half ? launch_typed<_Float16>(a, stream, handled) : launch_typed<float>(a, stream, handled);
}

}  // namespace tensor_gguf
