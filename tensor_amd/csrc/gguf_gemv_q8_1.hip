// Q8_1-activation integer-dot decode GEMV (gfx950), GGML's path for quantized
// matrix-vector products, which the reference benchmarks as its external GGML baseline
// (benchmarks/kernels/showcase/external_baselines.py:24-58, qualified at relative L2 <= 0.02
// against the fp32 oracle): out[m, n] = sum over 32-element blocks of x[m] (quantized to Q8_1)
// and W[n] of an integer dot product of their codes, scaled in fp32.
//
// The grid is one round of resident workgroups of 8 waves.  Each first quantizes all of x
// (M <= 8 rows) into LDS: per 32-element block d = max|x| / 127, q = roundf(x * (1 / d)) (0 for
// an all-zero block), and the block's d and s = d * sum(q), both rounded to fp16 as ggml's
// block_q8_1 stores them; 8 lanes per block, 4 elements each, the loads of 8 blocks per lane
// issued together; a lane's first weight bytes are requested before that, so they arrive
// meanwhile.  Then each wave takes the rows r, r + S, r + 2S, ... (S waves in the grid), so x is
// quantized once per workgroup however many rows there are, and its lanes take a row's units
// in turn (Q4_K: 64-element quant pairs, two Q8_1 blocks; Q6_K: 32-element runs; Q8_0 / Q4_0:
// whole blocks), each meeting the M activation blocks through v_dot4_i32_i8:
//
//   Q8_0  (d_w d_x) sum(q_w q_x)
//   Q4_0  d_w (d_x sum(q_w q_x) - 8 s_x)               q_w in 0..15
//   Q4_K  (d sc_j)(d_x sum(q q_x)) - (dmin m_j) s_x      per 32-element sub-block j
//   Q6_K  (d d_x)(sc_0 sum_0((q - 32) q_x) + sc_1 sum_1(...))   two 16-element scale groups
//
// The lanes' fp32 partial sums meet in a butterfly reduction, so the order of the block
// contributions differs from a sequential sum only by fp32 rounding.
//
// Block formats: benchmarks/kernels/showcase/triton_kernels.py:135-180 (Q4_0, Q4_K, Q6_K) and
// the public GGML block_q8_0.
#include <algorithm>

#include "gguf_common.h"
#include "gguf_launch.h"

namespace tensor_gguf {
namespace {

constexpr int kQ81Waves = 8, kQ81Threads = kQ81Waves * 64;
constexpr int kQ81MaxMK = 98304;  // int8 x codes plus two floats per block within LDS

// LDS layout of the activation codes: 32-byte blocks with 16 bytes of padding after every 8, so
// the 16 lanes of a b128 read that take consecutive blocks (or block pairs) meet 16 distinct
// 16-byte bank groups.
__host__ __device__ constexpr int q81_row_bytes(int nb) { return 32 * nb + 16 * ((nb + 7) >> 3); }
__device__ __forceinline__ int q81_block(int b) { return 32 * b + 16 * (b >> 3); }

__device__ __forceinline__ float group8_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  return fmaxf(v, __shfl_xor(v, 4));
}

__device__ __forceinline__ int group8_sum(int v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  return v + __shfl_xor(v, 4);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// (q - 32) of four 6-bit codes as signed bytes: flipping bit 5 gives q - 32 for q >= 32 and
// q + 32 for q < 32, whose bytes then also take bits 6 and 7 (the subtraction of 64).
__device__ __forceinline__ uint32_t minus32(uint32_t q) {
  const uint32_t low = ~q & 0x20202020u;
  return (q ^ 0x20202020u) | (low << 1) | (low << 2);
}

template <typename XT>
__device__ __forceinline__ void load4x(const XT* p, float v[4]) {
  if constexpr (sizeof(XT) == 4) {
    const float4 f = *reinterpret_cast<const float4*>(p);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    const uint2 h = *reinterpret_cast<const uint2*>(p);
    v[0] = half_bits_to_float(h.x); v[1] = half_bits_to_float(h.x >> 16);
    v[2] = half_bits_to_float(h.y); v[3] = half_bits_to_float(h.y >> 16);
  }
}

// One lane's unit of a weight row, loaded into registers and then met with the activation
// blocks: Q8_0 / Q4_0 a whole block, Q4_K a 64-element quant pair (two Q8_1 blocks), Q6_K a
// 32-element run.
template <int TYPE>
struct Unit;

template <>
struct Unit<kQ8_0> {
  static constexpr int BYTES = 34;
  uint32_t head;  // fp16 d in the low half
  uint4 lo, hi;
  static __device__ int count(int k) { return k >> 5; }
  __device__ void load(const uint8_t* wr, int b) {
    const uint8_t* blk = wr + (size_t)b * BYTES;
    head = load4(blk);
    lo = load16(blk + 2);
    hi = load16(blk + 18);
  }
};

template <>
struct Unit<kQ4_0> {
  static constexpr int BYTES = 18;
  uint32_t head;
  uint4 quants;
  static __device__ int count(int k) { return k >> 5; }
  __device__ void load(const uint8_t* wr, int b) {
    const uint8_t* blk = wr + (size_t)b * BYTES;
    head = load4(blk);
    quants = load16(blk + 2);
  }
};

template <>
struct Unit<kQ4_K> {  // quant pair u % 4 of super-block u / 4
  uint4 hd, qa, qb;
  static __device__ int count(int k) { return k >> 6; }
  __device__ void load(const uint8_t* wr, int u) {
    const uint8_t* sb = wr + (size_t)(u >> 2) * 144;
    hd = load16(sb);
    qa = load16(sb + 16 + 32 * (u & 3));
    qb = load16(sb + 32 + 32 * (u & 3));
  }
};

template <>
struct Unit<kQ6_K> {  // run j = b % 8 of super-block b / 8: elements 128 h + 32 c + l, h = j / 4, c = j % 4
  uint4 l0, l1, h0, h1;
  uint32_t scales, dword;
  static __device__ int count(int k) { return k >> 5; }
  __device__ void load(const uint8_t* wr, int b) {
    const uint8_t* sb = wr + (size_t)(b >> 3) * 210;
    const int j = b & 7, h = j >> 2, c = j & 3;
    l0 = load16(sb + 64 * h + 32 * (c & 1));
    l1 = load16(sb + 64 * h + 32 * (c & 1) + 16);
    h0 = load16(sb + 128 + 32 * h);
    h1 = load16(sb + 128 + 32 * h + 16);
    scales = load4(sb + 192 + 8 * h + 2 * c);  // bytes 0, 1: the scales of the two 16-element groups
    dword = load4(sb + 206);                   // high half: d
  }
};

template <int TYPE, int M, typename XT, typename OutT>
__global__ __launch_bounds__(kQ81Threads) void gemv_q8_1(const XT* __restrict__ x, const uint8_t* __restrict__ w,
                                                         OutT* __restrict__ out, int n, int k) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nb = k >> 5;                            // Q8_1 blocks per activation row
  int8_t* const qx = reinterpret_cast<int8_t*>(lds);  // [M] rows of padded code blocks
  const int xrow = q81_row_bytes(nb);
  float* const dx = reinterpret_cast<float*>(lds + M * xrow);
  float* const sx = dx + M * nb;
  constexpr int ROW_BLOCK = TYPE == kQ8_0 ? 34 : TYPE == kQ4_0 ? 18 : 0;
  constexpr int ROW_SUPER = TYPE == kQ4_K ? 144 : TYPE == kQ6_K ? 210 : 0;
  const size_t row_bytes = ROW_BLOCK ? (size_t)nb * ROW_BLOCK : (size_t)(k >> 8) * ROW_SUPER;
  const int lane = threadIdx.x & 63, stride = gridDim.x * kQ81Waves;
  const int row0 = blockIdx.x * kQ81Waves + (threadIdx.x >> 6);  // the wave's rows: row0, row0 + stride, ...
  const int units = Unit<TYPE>::count(k);
  // A lane's items, in order: for each row of the wave, its units lane, lane + 64, ...  One
  // item at a time is held in registers: the waves resident on a CU keep the weight stream
  // busy, and a second item's registers would cost resident waves.
  const int per_row = (units + 63) >> 6;
  const int total = row0 < n ? ((n - 1 - row0) / stride + 1) * per_row : 0;
  int load_row = row0, load_j = 0;
  auto load_next = [&](Unit<TYPE>& t) {
    const int u = lane + 64 * load_j;
    if (load_row < n && u < units) t.load(w + (size_t)load_row * row_bytes, u);
    if (++load_j == per_row) {
      load_j = 0;
      load_row += stride;
    }
  };
  // the first item is requested before x is quantized: its bytes arrive meanwhile
  Unit<TYPE> cur;
  load_next(cur);
  asm volatile("" ::: "memory");

  // quantize x: 8 lanes per block, blocks in turn over the workgroup, the loads of up to
  // kQ81Batch blocks per lane in flight together
  constexpr int kQ81Batch = 8;
  for (int base = threadIdx.x >> 3; base < M * nb; base += kQ81Batch * (kQ81Threads / 8)) {
    const int part = threadIdx.x & 7;
    float v[kQ81Batch][4];
#pragma unroll
    for (int i = 0; i < kQ81Batch; ++i) {
      const int blk = base + i * (kQ81Threads / 8);
      if (blk < M * nb) load4x<XT>(x + (size_t)blk * 32 + 4 * part, v[i]);
    }
#pragma unroll
    for (int i = 0; i < kQ81Batch; ++i) {
      const int blk = base + i * (kQ81Threads / 8);
      if (blk >= M * nb) break;
      const int m = blk / nb, b = blk - m * nb;
      float amax = fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3])));
      amax = group8_max(amax);
      const float d = amax / 127.0f;
      const float inv = d != 0.0f ? 1.0f / d : 0.0f;
      int q[4], sum = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        q[j] = (int)roundf(v[i][j] * inv);
        sum += q[j];
      }
      sum = group8_sum(sum);
      *reinterpret_cast<uint32_t*>(qx + m * xrow + q81_block(b) + 4 * part) =
          (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) | ((uint32_t)(q[2] & 0xFF) << 16) |
          ((uint32_t)(q[3] & 0xFF) << 24);
      if (part == 0) {
        dx[blk] = (float)fp16_of_fp32(d);
        sx[blk] = (float)fp16_of_fp32((float)sum * d);
      }
    }
  }
  __syncthreads();

  float acc[M];
  auto xwords = [&](int m, int b, uint32_t xw[8]) {
    const uint4 a = *reinterpret_cast<const uint4*>(qx + m * xrow + q81_block(b));
    const uint4 c = *reinterpret_cast<const uint4*>(qx + m * xrow + q81_block(b) + 16);
    xw[0] = a.x; xw[1] = a.y; xw[2] = a.z; xw[3] = a.w;
    xw[4] = c.x; xw[5] = c.y; xw[6] = c.z; xw[7] = c.w;
  };
  auto dot = [&](const Unit<TYPE>& t, int u) {
    if constexpr (TYPE == kQ8_0 || TYPE == kQ4_0) {
      const float dw = half_bits_to_float(t.head);
      uint32_t wq[8];
      if constexpr (TYPE == kQ8_0) {
        wq[0] = t.lo.x; wq[1] = t.lo.y; wq[2] = t.lo.z; wq[3] = t.lo.w;
        wq[4] = t.hi.x; wq[5] = t.hi.y; wq[6] = t.hi.z; wq[7] = t.hi.w;
      } else {
        // byte i: element i (low nibble) and element i + 16 (high nibble)
        const uint32_t words[4] = {t.quants.x, t.quants.y, t.quants.z, t.quants.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          wq[i] = words[i] & 0x0F0F0F0Fu;
          wq[4 + i] = (words[i] >> 4) & 0x0F0F0F0Fu;
        }
      }
#pragma unroll
      for (int m = 0; m < M; ++m) {
        uint32_t xw[8];
        xwords(m, u, xw);
        int isum = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) isum = dot4(wq[i], xw[i], isum);
        const float d8 = dx[m * nb + u];
        if constexpr (TYPE == kQ8_0)
          acc[m] += (dw * d8) * (float)isum;
        else
          acc[m] += dw * (d8 * (float)isum - 8.0f * sx[m * nb + u]);
      }
    } else if constexpr (TYPE == kQ4_K) {
      int sc_lo, mn_lo, sc_hi, mn_hi;
      q4k_scale_pair(t.hd.y, t.hd.z, t.hd.w, u & 3, sc_lo, mn_lo, sc_hi, mn_hi);
      const float d = half_bits_to_float(t.hd.x), dmin = half_bits_to_float(t.hd.x >> 16);
      const float s_lo = d * (float)sc_lo, s_hi = d * (float)sc_hi;
      const float o_lo = dmin * (float)mn_lo, o_hi = dmin * (float)mn_hi;
      const uint32_t words[8] = {t.qa.x, t.qa.y, t.qa.z, t.qa.w, t.qb.x, t.qb.y, t.qb.z, t.qb.w};
      const int b0 = 2 * u;  // low nibbles: sub-block 2 (u % 4), the Q8_1 block 2u; high: 2u + 1
#pragma unroll
      for (int m = 0; m < M; ++m) {
        uint32_t x0[8], x1[8];
        xwords(m, b0, x0);
        xwords(m, b0 + 1, x1);
        int i0 = 0, i1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          i0 = dot4(words[i] & 0x0F0F0F0Fu, x0[i], i0);
          i1 = dot4((words[i] >> 4) & 0x0F0F0F0Fu, x1[i], i1);
        }
        acc[m] += s_lo * (dx[m * nb + b0] * (float)i0) - o_lo * sx[m * nb + b0];
        acc[m] += s_hi * (dx[m * nb + b0 + 1] * (float)i1) - o_hi * sx[m * nb + b0 + 1];
      }
    } else {
      const int c = u & 3;
      const uint32_t lw[8] = {t.l0.x, t.l0.y, t.l0.z, t.l0.w, t.l1.x, t.l1.y, t.l1.z, t.l1.w};
      const uint32_t hw[8] = {t.h0.x, t.h0.y, t.h0.z, t.h0.w, t.h1.x, t.h1.y, t.h1.z, t.h1.w};
      const int sc0 = (int)(int8_t)(t.scales & 0xFF), sc1 = (int)(int8_t)((t.scales >> 8) & 0xFF);
      const float d = half_bits_to_float(t.dword >> 16);
      uint32_t wq[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        wq[i] = minus32(((lw[i] >> (4 * (c >> 1))) & 0x0F0F0F0Fu) | (((hw[i] >> (2 * c)) & 0x03030303u) << 4));
#pragma unroll
      for (int m = 0; m < M; ++m) {
        uint32_t xw[8];
        xwords(m, u, xw);
        int g0 = 0, g1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          g0 = dot4(wq[i], xw[i], g0);
          g1 = dot4(wq[4 + i], xw[4 + i], g1);
        }
        acc[m] += (d * dx[m * nb + u]) * (float)(sc0 * g0 + sc1 * g1);
      }
    }
  };
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.0f;
  int row = row0, j = 0;
  for (int t = 0; t < total; ++t) {
    const int u = lane + 64 * j;
    if (u < units) dot(cur, u);
    load_next(cur);
    if (++j == per_row) {  // the row is complete
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const float v = wave_sum(acc[m]);
        if (lane == 0) store_out<OutT>(out, (size_t)m * n + row, v);
        acc[m] = 0.0f;
      }
      j = 0;
      row += stride;
    }
  }
}

// Grid: as many workgroups as are resident at once on the 256 CUs (registers and LDS
// permitting), each wave taking ceil(rows / waves) rows, so every workgroup quantizes x once
// and the weight stream of its waves follows without a second round of workgroups.
template <int TYPE, int M, typename XT, typename OutT>
hipError_t launch_typed(const GemvArgs& a, hipStream_t stream) {
  constexpr int kCUs = 256, kLdsPerCU = 160 * 1024;
  const size_t lds = (size_t)M * q81_row_bytes(a.k >> 5) + 2 * sizeof(float) * (size_t)M * (a.k >> 5);
  static const int by_regs = [] {
    int blocks = 0;
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &blocks, reinterpret_cast<const void*>(gemv_q8_1<TYPE, M, XT, OutT>), kQ81Threads, 0);
    return e == hipSuccess && blocks > 0 ? blocks : 1;
  }();
  const int per_cu = std::max(1, std::min(by_regs, (int)(kLdsPerCU / std::max<size_t>(lds, 1))));
  const long waves = (long)kCUs * per_cu * kQ81Waves;
  const long rows_per_wave = (a.n + waves - 1) / waves;
  const int grid = (int)((a.n + rows_per_wave * kQ81Waves - 1) / (rows_per_wave * kQ81Waves));
  hipLaunchKernelGGL((gemv_q8_1<TYPE, M, XT, OutT>), dim3(grid), dim3(kQ81Threads), lds, stream,
                     static_cast<const XT*>(a.x), static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out), a.n,
                     a.k);
  return hipGetLastError();
}

template <int TYPE, int M>
hipError_t launch_m(const GemvArgs& a, hipStream_t stream) {
  if (a.x_f32)
    return a.out_half ? launch_typed<TYPE, M, float, _Float16>(a, stream) : launch_typed<TYPE, M, float, float>(a, stream);
  return a.out_half ? launch_typed<TYPE, M, _Float16, _Float16>(a, stream)
                    : launch_typed<TYPE, M, _Float16, float>(a, stream);
}

template <int TYPE>
hipError_t launch_type(const GemvArgs& a, hipStream_t stream) {
  switch (a.m) {
    case 1: return launch_m<TYPE, 1>(a, stream);
    case 2: return launch_m<TYPE, 2>(a, stream);
    case 3: return launch_m<TYPE, 3>(a, stream);
    case 4: return launch_m<TYPE, 4>(a, stream);
    case 5: return launch_m<TYPE, 5>(a, stream);
    case 6: return launch_m<TYPE, 6>(a, stream);
    case 7: return launch_m<TYPE, 7>(a, stream);
    default: return launch_m<TYPE, 8>(a, stream);
  }
}

}  // namespace

bool gemv_q8_1_supported(const GemvArgs& a) {
  const bool kquant = a.type == kQ4_K || a.type == kQ6_K;
  return (kquant || a.type == kQ8_0 || a.type == kQ4_0) && a.m >= 1 && a.m <= kGemvMaxM && a.n >= 1 &&
         a.k >= 32 && a.k % (kquant ? 256 : 32) == 0 && (long)a.m * a.k <= kQ81MaxMK;
}

hipError_t launch_gemv_q8_1(const GemvArgs& a, hipStream_t stream) {
  if (!gemv_q8_1_supported(a)) return hipErrorInvalidValue;
  switch (a.type) {
    case kQ8_0: return launch_type<kQ8_0>(a, stream);
    case kQ4_0: return launch_type<kQ4_0>(a, stream);
    case kQ4_K: return launch_type<kQ4_K>(a, stream);
    default: return launch_type<kQ6_K>(a, stream);
  }
}

}  // namespace tensor_gguf
