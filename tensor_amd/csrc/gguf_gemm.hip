// Prefill fused dequant-GEMM: out[m, n] = sum_k fp16(x[m, k]) * fp16(W[n, k]),
// fp32 accumulation (reference kernel: AKAS _packed at
// benchmarks/kernels/showcase/kernels.py:114-119; restated by the Triton
// gguf kernel at triton_kernels.py:185-211).
//
// gfx950 design.  A workgroup of WM x WN waves owns a BM x BN output tile and
// walks K in steps of BK = 64 elements:
//
//   * The next step's activation tile and raw GGUF bytes are prefetched into
//     registers while the current step's MFMAs run.
//   * Weights are dequantized straight from those registers into fp16 LDS
//     tiles with the reference's fp32 arithmetic (every product exact, one
//     rounding), so the staged weights are bit-exact fp16(dequant(W)).
//   * LDS tiles are double-buffered: one barrier per K step.  Rows are padded
//     by 16 bytes so the b128 fragment reads of a wave spread over the banks.
//   * Each wave computes a 64 x (16 NT) sub-tile with v_mfma_f32_16x16x32_f16
//     (lane l supplies row/column l % 16 and k = 8 (l / 16) .. + 7; the 16 x 16
//     result gives lane l rows 4 (l / 16) .. + 3 of column l % 16).
//
// Q4_K weights take a dedicated path (header and quant bytes prefetched, two
// to four threads per weight row); the other encodings decode 8-element
// groups with the shared per-element decoder.
#include "gguf_decode.h"
#include "gguf_launch.h"

namespace tensor_gguf {

namespace gemm {
constexpr int BK = 64;
constexpr int PAD = 8;  // halves of padding per LDS row
constexpr int LDS_ROW = BK + PAD;
}  // namespace gemm

__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  return half2_from_fp32(a, b);
}

// Exact Q4_K dequantization of four codes held in the bytes of one dword
// (each byte's nibble already isolated in its low four bits).
__device__ __forceinline__ void q4k_dequant4(uint32_t codes, float ds, float dm, uint32_t& lo_pair, uint32_t& hi_pair) {
  const float a = ds * (float)(codes & 0xFFu) - dm;
  const float b = ds * (float)((codes >> 8) & 0xFFu) - dm;
  const float c = ds * (float)((codes >> 16) & 0xFFu) - dm;
  const float d = ds * (float)(codes >> 24) - dm;
  lo_pair = pack_half2(a, b);
  hi_pair = pack_half2(c, d);
}

// XT = float: fp32 activations (the packed call form), rounded to fp16 as they are loaded.
template <int TYPE, int BM, int BN, int WM, int WN, typename OutT, typename XT = _Float16>
__global__ __launch_bounds__(WM * WN * 64) void gemm_v2(const XT* __restrict__ x,
                                                        const uint8_t* __restrict__ w,
                                                        OutT* __restrict__ out, int M, int N, int K) {
  using namespace gemm;
  constexpr int THREADS = WM * WN * 64;
  constexpr int NT = BN / WN / 16;             // 16-column MFMA tiles per wave
  static_assert(BM / WM == 64, "each wave covers 64 rows of M");
  static_assert(NT * 16 * WN == BN, "BN must split into 16-column tiles per wave");
  constexpr int QK = Block<TYPE>::QK;
  constexpr int BYTES = Block<TYPE>::BYTES;
  // activation tile: BM rows x BK halves = BM * 8 chunks of 16 bytes
  constexpr int X_LOADS = BM * 8 / THREADS;
  static_assert(X_LOADS * THREADS == BM * 8, "activation tile must split evenly");
  // Q4_K: TPR threads per weight row, each owning 32 / TPR quant bytes of the step's pair
  constexpr int TPR = THREADS / BN;
  static_assert(TYPE != kQ4_K || (TPR * BN == THREADS && (TPR == 1 || TPR == 2 || TPR == 4)),
                "Q4_K tiles need 1, 2 or 4 threads per weight row");
  constexpr int QBYTES = TYPE == kQ4_K ? 32 / TPR : 16;
  // generic decoder: BN rows x 8 groups of 8 elements
  constexpr int G_LOADS = (BN * 8 + THREADS - 1) / THREADS;

  __shared__ __attribute__((aligned(16))) _Float16 xs[2][BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) _Float16 ws[2][BN * LDS_ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = (wave / WN) * 64, wn = (wave % WN) * (16 * NT);
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const size_t row_bytes = (size_t)(K / QK) * BYTES;
  const int steps = (K + BK - 1) / BK;

  // ---- prefetch registers
  uint4 xr[X_LOADS];
  uint4 hd;                       // Q4_K header of this thread's weight row
  uint32_t qw[QBYTES / 4];        // Q4_K quant bytes of this thread's slice
  const int wrow = tid / (TYPE == kQ4_K ? TPR : 1), wpart = tid % (TYPE == kQ4_K ? TPR : 1);
  const uint8_t* wbase = w + (size_t)min(n0 + wrow, N - 1) * row_bytes;

  auto prefetch = [&](int step) {
    const int k0 = step * BK;
#pragma unroll
    for (int i = 0; i < X_LOADS; ++i) {
      const int c = i * THREADS + tid, r = c >> 3, c8 = (c & 7) * 8;
      if (m0 + r < M && k0 + c8 < K) {
        const XT* src = x + (size_t)(m0 + r) * K + k0 + c8;
        if constexpr (sizeof(XT) == 4) {
          const uint4 lo = load16(reinterpret_cast<const uint8_t*>(src));
          const uint4 hi = load16(reinterpret_cast<const uint8_t*>(src + 4));
          xr[i] = make_uint4(half2_from_fp32(__builtin_bit_cast(float, lo.x), __builtin_bit_cast(float, lo.y)),
                             half2_from_fp32(__builtin_bit_cast(float, lo.z), __builtin_bit_cast(float, lo.w)),
                             half2_from_fp32(__builtin_bit_cast(float, hi.x), __builtin_bit_cast(float, hi.y)),
                             half2_from_fp32(__builtin_bit_cast(float, hi.z), __builtin_bit_cast(float, hi.w)));
        } else {
          xr[i] = *reinterpret_cast<const uint4*>(src);
        }
      } else {
        xr[i] = make_uint4(0, 0, 0, 0);
      }
    }
    if (TYPE == kQ4_K && wrow < BN) {
      const uint8_t* blk = wbase + (size_t)(k0 >> 8) * 144;
      hd = load16(blk);
      const uint8_t* q = blk + 16 + 32 * ((k0 >> 6) & 3) + QBYTES * wpart;
#pragma unroll
      for (int i = 0; i < QBYTES / 4; ++i) qw[i] = load4(q + 4 * i);
    }
  };

  auto stage = [&](int step, int buf) {
    const int k0 = step * BK;
#pragma unroll
    for (int i = 0; i < X_LOADS; ++i) {
      const int c = i * THREADS + tid, r = c >> 3, c8 = (c & 7) * 8;
      *reinterpret_cast<uint4*>(&xs[buf][r * LDS_ROW + c8]) = xr[i];
    }
    if (TYPE == kQ4_K) {
      if (wrow < BN) {
        // pair j = step % 4: low nibbles are sub-block 2j, high nibbles 2j+1
        const int j = (k0 >> 6) & 3;
        int sc_lo, mn_lo, sc_hi, mn_hi;
        q4k_scale_pair(hd.y, hd.z, hd.w, j, sc_lo, mn_lo, sc_hi, mn_hi);
        const float d = half_bits_to_float(hd.x), dmin = half_bits_to_float(hd.x >> 16);
        const float ds_lo = d * (float)sc_lo, dm_lo = dmin * (float)mn_lo;
        const float ds_hi = d * (float)sc_hi, dm_hi = dmin * (float)mn_hi;
        _Float16* dst = &ws[buf][wrow * LDS_ROW + QBYTES * wpart];
#pragma unroll
        for (int i = 0; i < QBYTES / 4; ++i) {
          uint32_t l0, l1, h0, h1;
          q4k_dequant4(qw[i] & 0x0F0F0F0Fu, ds_lo, dm_lo, l0, l1);
          q4k_dequant4((qw[i] >> 4) & 0x0F0F0F0Fu, ds_hi, dm_hi, h0, h1);
          *reinterpret_cast<uint2*>(dst + 4 * i) = make_uint2(l0, l1);
          *reinterpret_cast<uint2*>(dst + 32 + 4 * i) = make_uint2(h0, h1);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < G_LOADS; ++i) {
        const int c = i * THREADS + tid;
        if (c < BN * 8) {
          const int r = c >> 3, c8 = (c & 7) * 8, kk = k0 + c8;
          uint4 v = make_uint4(0, 0, 0, 0);  // a K tail shorter than BK reads as zeros
          if (kk < K) {
            const uint8_t* blk = w + (size_t)min(n0 + r, N - 1) * row_bytes + (size_t)(kk / QK) * BYTES;
            float f[8];
            decode8<TYPE>(blk, kk % QK, f);
            v = make_uint4(pack_half2(f[0], f[1]), pack_half2(f[2], f[3]), pack_half2(f[4], f[5]),
                           pack_half2(f[6], f[7]));
          }
          *reinterpret_cast<uint4*>(&ws[buf][r * LDS_ROW + c8]) = v;
        }
      }
    }
  };

  float4_t acc[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  prefetch(0);
  stage(0, 0);
  __syncthreads();
  for (int step = 0; step < steps; ++step) {
    const int buf = step & 1;
    if (step + 1 < steps) prefetch(step + 1);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      const int koff = kk + 8 * (lane >> 4);
      half8_t a[4], b[NT];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const half8_t*>(&xs[buf][(wm + 16 * i + (lane & 15)) * LDS_ROW + koff]);
#pragma unroll
      for (int j = 0; j < NT; ++j)
        b[j] = *reinterpret_cast<const half8_t*>(&ws[buf][(wn + 16 * j + (lane & 15)) * LDS_ROW + koff]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (step + 1 < steps) stage(step + 1, buf ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int col = n0 + wn + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wm + 16 * i + 4 * (lane >> 4) + e;
        if (row < M && col < N) store_out<OutT>(out, (size_t)row * N + col, acc[i][j][e]);
      }
    }
}

template <int TYPE, int BM, int BN, int WM, int WN, typename OutT, typename XT>
static hipError_t launch_tile(const GemvArgs& a, hipStream_t stream) {
  const dim3 grid((a.n + BN - 1) / BN, (a.m + BM - 1) / BM), block(WM * WN * 64);
  hipLaunchKernelGGL((gemm_v2<TYPE, BM, BN, WM, WN, OutT, XT>), grid, block, 0, stream,
                     static_cast<const XT*>(a.x), static_cast<const uint8_t*>(a.w),
                     static_cast<OutT*>(a.out), a.m, a.n, a.k);
  return hipGetLastError();
}

// The small-M kernel where the tiled kernels leave most CUs idle: M <= 64 for shapes on the
// generic tiles, and for shapes the pipelined tiles take also N <= 4096 (at N = 12288 those are
// faster from M = 16: Q4_K M = 32, K = 4096: 33.6 against 38.4 us, Q4_0 with fp16 x 23.4
// against 40.9; at N = K = 1024, M = 32 the small-M kernel takes 5.3 against 10.4 us, Q4_0
// 4.9 against 30.6).  Q8_0 with fp32 x keeps it to M = 16 (33.7 against 42.8 us at N = 12288).
bool gemm_small_m(const GemvArgs& a) {
  if (!gemm_skinny_supported(a)) return false;
  return !gemm_pipe_supported(a) || a.n <= 4096 || (a.type == kQ8_0 && a.x_f32 && a.m <= 16);
}

template <int TYPE, typename OutT>
static hipError_t launch_type(const GemvArgs& a, hipStream_t stream) {
  if (gemm_small_m(a)) return launch_gemm_skinny(a, stream);
  bool handled = false;
  const hipError_t status = launch_gemm_pipe(a, stream, &handled);
  if (handled) return status;
  // 128 x 128 tiles; 256 x 128 once M is large enough to fill the chip with them
  if (a.x_f32) return launch_tile<TYPE, 128, 128, 2, 2, OutT, float>(a, stream);
  if (a.m >= 1024) return launch_tile<TYPE, 256, 128, 4, 2, OutT, _Float16>(a, stream);
  return launch_tile<TYPE, 128, 128, 2, 2, OutT, _Float16>(a, stream);
}

template <typename OutT>
static hipError_t launch_typed(const GemvArgs& a, hipStream_t stream) {
  switch (a.type) {
    case kQ4_K: return launch_type<kQ4_K, OutT>(a, stream);
    case kQ6_K: return launch_type<kQ6_K, OutT>(a, stream);
    case kQ8_0: return launch_type<kQ8_0, OutT>(a, stream);
    case kQ4_0: return launch_type<kQ4_0, OutT>(a, stream);
    case kQ4_1: return launch_type<kQ4_1, OutT>(a, stream);
    case kQ5_0: return launch_type<kQ5_0, OutT>(a, stream);
    case kQ5_1: return launch_type<kQ5_1, OutT>(a, stream);
    case kQ2_K: return launch_type<kQ2_K, OutT>(a, stream);
    case kQ3_K: return launch_type<kQ3_K, OutT>(a, stream);
    case kQ5_K: return launch_type<kQ5_K, OutT>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm(const GemvArgs& a, hipStream_t stream) {
  return a.out_half ? launch_typed<_Float16>(a, stream) : launch_typed<float>(a, stream);
}

}  // namespace tensor_gguf
