// Prefill fused dequant-GEMM: out[m, n] = sum_k fp16(x[m, k]) * fp16(W[n, k]),
// fp32 accumulation (reference kernel: AKAS _packed at
// benchmarks/kernels/showcase/kernels.py:114-119; restated by the Triton
// gguf kernel at triton_kernels.py:185-211).
//
// gfx950 design: a 256-thread workgroup owns a BM x BN output tile.  Per K
// step it stages the fp16 activation tile and the weight tile, decoded from
// raw GGUF blocks straight into LDS as fp16 (same arithmetic as the
// dequantizer, so the staged weights are bit-exact fp16(dequant(W))), then
// each wave runs v_mfma_f32_16x16x32_f16 over its sub-tile with fp32
// accumulators held in registers.
#include "gguf_decode.h"
#include "gguf_launch.h"

namespace tensor_gguf {

namespace gemm {
constexpr int BM = 128, BN = 128, BK = 128;
constexpr int LDS_STRIDE = BK + 8;  // halves; 16-byte skew between rows
constexpr int THREADS = 256;
}  // namespace gemm

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  const _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// MFMA 16x16x32 fp16 operand layout (wave64): lane l supplies row/column
// l % 16 and the 8 consecutive k values 8*(l/16) .. 8*(l/16)+7; the 16x16 fp32
// result gives lane l rows 4*(l/16) .. +3 of column l % 16.
template <int TYPE, typename OutT>
__global__ __launch_bounds__(256) void gemm_kernel(const _Float16* __restrict__ x,
                                                   const uint8_t* __restrict__ w,
                                                   OutT* __restrict__ out, int M, int N, int K) {
  using namespace gemm;
  constexpr int QK = (TYPE == kQ4_K || TYPE == kQ6_K) ? 256 : 32;
  constexpr int BYTES = TYPE == kQ4_K ? 144 : TYPE == kQ6_K ? 210 : TYPE == kQ8_0 ? 34 : 18;
  __shared__ __attribute__((aligned(16))) _Float16 xs[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) _Float16 ws[BN * LDS_STRIDE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;  // 2 x 2 waves of 64 x 64
  const size_t row_bytes = (size_t)(K / QK) * BYTES;

  float4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += BK) {
    // activation tile: BM rows x BK halves, 16 B per thread-iteration
#pragma unroll
    for (int it = 0; it < (BM * BK / 8) / THREADS; ++it) {
      const int idx = it * THREADS + tid;
      const int r = idx / (BK / 8), c8 = (idx % (BK / 8)) * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m0 + r < M && k0 + c8 < K)
        v = *reinterpret_cast<const uint4*>(x + (size_t)(m0 + r) * K + k0 + c8);
      *reinterpret_cast<uint4*>(&xs[r * LDS_STRIDE + c8]) = v;
    }
    // weight tile: BN rows x BK elements decoded to fp16
#pragma unroll
    for (int it = 0; it < (BN * BK / 8) / THREADS; ++it) {
      const int idx = it * THREADS + tid;
      const int r = idx / (BK / 8), c8 = (idx % (BK / 8)) * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      const int kk = k0 + c8;
      if (n0 + r < N && kk < K) {
        const uint8_t* block = w + (size_t)(n0 + r) * row_bytes + (size_t)(kk / QK) * BYTES;
        float f[8];
        decode8<TYPE>(block, kk % QK, f);
        v = make_uint4(pack_half2(f[0], f[1]), pack_half2(f[2], f[3]), pack_half2(f[4], f[5]),
                       pack_half2(f[6], f[7]));
      }
      *reinterpret_cast<uint4*>(&ws[r * LDS_STRIDE + c8]) = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      half8_t a[4], b[4];
      const int koff = kk + 8 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const half8_t*>(&xs[(wm + 16 * i + (lane & 15)) * LDS_STRIDE + koff]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const half8_t*>(&ws[(wn + 16 * j + (lane & 15)) * LDS_STRIDE + koff]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  // D layout: lane holds rows 4*(lane/16)+e of column lane%16 of each 16x16 tile
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wm + 16 * i + 4 * (lane >> 4) + e;
        if (row < M && col < N) store_out<OutT>(out, (size_t)row * N + col, acc[i][j][e]);
      }
    }
}

template <typename OutT>
static hipError_t launch_typed(const GemvArgs& a, hipStream_t stream) {
  using namespace gemm;
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const dim3 grid((a.n + BN - 1) / BN, (a.m + BM - 1) / BM), block(THREADS);
  switch (a.type) {
    case kQ4_K:
      hipLaunchKernelGGL((gemm_kernel<kQ4_K, OutT>), grid, block, 0, stream, x, w, out, a.m, a.n, a.k);
      break;
    case kQ6_K:
      hipLaunchKernelGGL((gemm_kernel<kQ6_K, OutT>), grid, block, 0, stream, x, w, out, a.m, a.n, a.k);
      break;
    case kQ8_0:
      hipLaunchKernelGGL((gemm_kernel<kQ8_0, OutT>), grid, block, 0, stream, x, w, out, a.m, a.n, a.k);
      break;
    case kQ4_0:
      hipLaunchKernelGGL((gemm_kernel<kQ4_0, OutT>), grid, block, 0, stream, x, w, out, a.m, a.n, a.k);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemm(const GemvArgs& a, hipStream_t stream) {
  return a.out_half ? launch_typed<_Float16>(a, stream) : launch_typed<float>(a, stream);
}

}  // namespace tensor_gguf
