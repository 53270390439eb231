// Small-M prefill dequant-GEMM (gfx950), every encoding: out[m, n] = sum_k fp16(x[m, k]) *
// fp16(W[n, k]) with fp32 accumulation, for M <= 64 (the showcase's M = 32 prefill at
// N = K = 1024 among them: benchmarks/kernels/showcase/benchmark.py:122-126, :460-464).
//
// At these shapes the tiled GEMM has few output tiles (8-16 workgroups of 128 or 64 columns for
// N = 1024) and each walks the whole of K, so its time is the latency of one long K loop.  Here
// a workgroup owns 16 NT weight rows and 16 MT activation rows, and its SPLIT waves take
// interleaved 64-element chunks of K (wave v: chunks v, v + SPLIT, ..), so the K loop is SPLIT
// times shorter and N / (16 NT) x M / (16 MT) workgroups run at once.  No LDS tile of weights:
// in each 32-element step lane l
//   * dequantizes the 8 elements 8 (l / 16) .. + 7 of weight row l % 16 of every 16-row tile
//     with the shared per-element decoder (the reference's fp32 arithmetic, then one cast to
//     fp16) straight into the B operand of v_mfma_f32_16x16x32_f16, and
//   * takes the same 8 elements of activation row 16 i + l % 16 as the A operand of tile i
//     (fp32 activations rounded to fp16 on the way through a wave-private LDS tile),
// so each dequantized weight feeds MT MFMAs.  The waves' fp32 tiles meet in LDS, summed in
// wave order by all threads.  The operands are the ones the tiled GEMM stages (fp16(x),
// fp16(dequant(W))); only the order of the fp32 additions differs.
#include "gguf_common.h"
#include "gguf_decode.h"
#include "gguf_launch.h"

namespace tensor_gguf {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

template <int TYPE, int MT, int NT, int SPLIT, typename OutT, typename XT>
__global__ __launch_bounds__(SPLIT * 64) void gemm_skinny(const XT* __restrict__ x, const uint8_t* __restrict__ w,
                                                          OutT* __restrict__ out, int M, int N, int K) {
  constexpr int QK = Block<TYPE>::QK, BYTES = Block<TYPE>::BYTES;
  __shared__ float red[SPLIT][MT * NT][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int n0 = blockIdx.x * 16 * NT, m0 = blockIdx.y * 16 * MT;  // this workgroup's rows of W and x
  const size_t row_bytes = (size_t)(K / QK) * BYTES;
  const uint8_t* wr[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) wr[j] = w + (size_t)min(n0 + 16 * j + r, N - 1) * row_bytes;
  float4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  // The waves take interleaved 64-element chunks of K (wave v: chunks v, v + SPLIT, ..), U
  // chunks per pass with no branch between their loads: a chunk past the end reloads the last
  // chunk (in bounds) and its A operands are zeroed.  All loads of a pass (activations, then
  // the fp32 decodes) come before the first fp16 cast of a weight, whose register pin would
  // otherwise keep the scheduler from moving later loads above it.
  //
  // Activations are loaded row-contiguous (fp16: 8 rows of a chunk's 128 bytes per load
  // instruction, fp32: 4 rows of 256 bytes), cast to fp16 and passed through a wave-private
  // LDS tile into the MFMA layout.  Loaded in that layout directly, each instruction would
  // touch 16 rows (lane l holds row l % 16), and measured slower for both widths.  Rows past M
  // reload row M - 1; they only reach result rows that are never stored.
  constexpr int U = MT * NT <= 2 ? 2 : 1;
  constexpr int XE = 16 / sizeof(XT);       // activations per 16-byte load
  constexpr int RPL = 64 / (64 / XE);       // rows per load instruction (8 or 4)
  constexpr int TROW = 72;                  // halves per staged row: 64 + 8 of padding
  __shared__ __attribute__((aligned(16))) _Float16 xt[SPLIT][U * MT][16 * TROW];
  const int chunks = K >> 6, tail = K & 63;  // a last half chunk when K % 64 == 32
  const int xrow = lane / (64 / XE), xcol = XE * (lane % (64 / XE));
  for (int c0 = wave; c0 < chunks + (tail ? 1 : 0); c0 += U * SPLIT) {
    uint4 xw[U][MT][16 / RPL];
    float f[U][2][NT][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int cl = min(c0 + u * SPLIT, chunks + (tail ? 1 : 0) - 1);
      // a half chunk (K % 64 == 32) reads its 32 elements twice; its second step is zeroed
      const int kc = 64 * cl, second = cl == chunks ? 0 : 32;
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int h = 0; h < 16 / RPL; ++h)
          xw[u][i][h] = load16(reinterpret_cast<const uint8_t*>(
              x + (size_t)min(m0 + 16 * i + RPL * h + xrow, M - 1) * K + kc + (xcol & (second ? 63 : 31))));
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int k = kc + (t ? second : 0) + 8 * g;  // this lane's first element of step t
#pragma unroll
        for (int j = 0; j < NT; ++j) decode8<TYPE>(wr[j] + (size_t)(k / QK) * BYTES, k % QK, f[u][t][j]);
      }
    }
    // rows RPL h + lane / (64 / XE), elements XE (lane % (64 / XE)) .. -> the wave's tile of (u, i)
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int h = 0; h < 16 / RPL; ++h) {
          _Float16* dst = &xt[wave][u * MT + i][(RPL * h + xrow) * TROW + xcol];
          if constexpr (sizeof(XT) == 4) {
            const float4_t v = __builtin_bit_cast(float4_t, xw[u][i][h]);
            *reinterpret_cast<uint2*>(dst) = __builtin_bit_cast(uint2, __builtin_convertvector(v, half4_t));
          } else {
            *reinterpret_cast<uint4*>(dst) = xw[u][i][h];
          }
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u * SPLIT;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bool in = c < chunks || (t == 0 && c == chunks && tail);
        half8_t a[MT], b[NT];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          a[i] = *reinterpret_cast<const half8_t*>(&xt[wave][u * MT + i][r * TROW + 32 * t + 8 * g]);
          if (!in) a[i] = half8_t{};
        }
#pragma unroll
        for (int j = 0; j < NT; ++j)
          b[j] = __builtin_bit_cast(half8_t, make_uint4(half2_from_fp32(f[u][t][j][0], f[u][t][j][1]),
                                                        half2_from_fp32(f[u][t][j][2], f[u][t][j][3]),
                                                        half2_from_fp32(f[u][t][j][4], f[u][t][j][5]),
                                                        half2_from_fp32(f[u][t][j][6], f[u][t][j][7])));
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
          for (int j = 0; j < NT; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
      }
    }
    __builtin_amdgcn_wave_barrier();  // the next pass rewrites the wave's tiles
  }

  // Every wave's fp32 tiles go to LDS, row-major per 16 x 16 tile; then each thread sums
  // outputs over the SPLIT partials in wave order (so the result does not depend on which wave
  // finished first) and stores them: a wave instruction covers 4 rows x 16 columns.  (Wave 0
  // alone summing all partials in the MFMA layout took ~0.5 us at M = 32.)
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave][i * NT + j][(4 * g + e) * 16 + r] = acc[i][j][e];
  __syncthreads();
  for (int f = threadIdx.x; f < MT * NT * 256; f += SPLIT * 64) {
    const int tile = f >> 8, pos = f & 255;
    float v = red[0][tile][pos];
#pragma unroll
    for (int p = 1; p < SPLIT; ++p) v += red[p][tile][pos];
    const int row = m0 + 16 * (tile / NT) + (pos >> 4), col = n0 + 16 * (tile % NT) + (pos & 15);
    if (row < M && col < N) store_out<OutT>(out, (size_t)row * N + col, v);
  }
}

namespace {

template <int TYPE, int MT, int NT, int SPLIT, typename OutT, typename XT>
hipError_t launch_shape(const GemvArgs& a, hipStream_t stream) {
  const dim3 grid((a.n + 16 * NT - 1) / (16 * NT), (a.m + 16 * MT - 1) / (16 * MT)), block(SPLIT * 64);
  hipLaunchKernelGGL((gemm_skinny<TYPE, MT, NT, SPLIT, OutT, XT>), grid, block, 0, stream,
                     static_cast<const XT*>(a.x), static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out), a.m,
                     a.n, a.k);
  return hipGetLastError();
}

// MT x NT <= 8 tiles per wave: 4 x 4 spills (its accumulators, operands and decoder state pass
// 256 VGPRs), 2 x 4 and 4 x 2 take ~236 without spilling.
template <int TYPE, int MT, typename OutT, typename XT>
hipError_t launch_nt(const GemvArgs& a, int nt, hipStream_t stream) {
  switch (nt) {
    case 1: return launch_shape<TYPE, MT, 1, 8, OutT, XT>(a, stream);
    case 2: return launch_shape<TYPE, MT, 2, 8, OutT, XT>(a, stream);
    case 4: return launch_shape<TYPE, MT, MT <= 2 ? 4 : 2, 8, OutT, XT>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

// mt: 16-row M tiles per workgroup (1, 2 or 4); the M tiles beyond it go to further rows of
// workgroups (grid y)
template <int TYPE, typename OutT, typename XT>
hipError_t launch_mt(const GemvArgs& a, int nt, int mt, hipStream_t stream) {
  switch (mt) {
    case 1: return launch_nt<TYPE, 1, OutT, XT>(a, nt, stream);
    case 2: return launch_nt<TYPE, 2, OutT, XT>(a, nt, stream);
    case 4: return launch_nt<TYPE, 4, OutT, XT>(a, nt, stream);
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE>
hipError_t launch_io(const GemvArgs& a, int nt, int mt, hipStream_t stream) {
  if (a.x_f32)
    return a.out_half ? launch_mt<TYPE, _Float16, float>(a, nt, mt, stream)
                      : launch_mt<TYPE, float, float>(a, nt, mt, stream);
  return a.out_half ? launch_mt<TYPE, _Float16, _Float16>(a, nt, mt, stream)
                    : launch_mt<TYPE, float, _Float16>(a, nt, mt, stream);
}

}  // namespace

bool gemm_skinny_supported(const GemvArgs& a) { return a.m >= 1 && a.m <= kSkinnyMaxM && a.k % 32 == 0; }

hipError_t launch_gemm_skinny(const GemvArgs& a, hipStream_t stream, int nt, int mt) {
  if (!gemm_skinny_supported(a)) return hipErrorInvalidValue;
  // one 16-row tile of W per workgroup unless N is wide enough to fill the CUs with pairs (M =
  // 64, N = 12288: 58 against 64 us; at M <= 16 the single tiles stay ahead)
  if (nt == 0) nt = a.n >= 8192 && a.m > 16 ? 2 : 1;
  // one 16-row tile of x per workgroup while that keeps the grid within one round of 256
  // workgroups (each then reads a quarter or half of x and decodes its weights again from L2:
  // N = K = 1024, M = 64: Q4_0 6.4 -> 4.2 us, M = 32: 4.6 -> 4.0 us), else all of them
  const int mtiles = (a.m + 15) / 16, ntiles = (a.n + 16 * nt - 1) / (16 * nt);
  if (mt == 0) mt = (long)ntiles * mtiles <= 256 ? 1 : mtiles <= 1 ? 1 : mtiles <= 2 ? 2 : 4;
  switch (a.type) {
    case kQ4_0: return launch_io<kQ4_0>(a, nt, mt, stream);
    case kQ4_1: return launch_io<kQ4_1>(a, nt, mt, stream);
    case kQ5_0: return launch_io<kQ5_0>(a, nt, mt, stream);
    case kQ5_1: return launch_io<kQ5_1>(a, nt, mt, stream);
    case kQ8_0: return launch_io<kQ8_0>(a, nt, mt, stream);
    case kQ2_K: return launch_io<kQ2_K>(a, nt, mt, stream);
    case kQ3_K: return launch_io<kQ3_K>(a, nt, mt, stream);
    case kQ4_K: return launch_io<kQ4_K>(a, nt, mt, stream);
    case kQ5_K: return launch_io<kQ5_K>(a, nt, mt, stream);
    case kQ6_K: return launch_io<kQ6_K>(a, nt, mt, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace tensor_gguf
