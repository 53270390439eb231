// Q2_K and Q3_K decode GEMV fast path (gfx950) for M = 1 and K a multiple of 4096 up to
// 16384: out[n] = sum_k x[k] * W[n, k].
//
// The workgroup plan of the Q6_K kernel: 8 waves of R rows each; the activation vector loaded
// first, then every weight byte of the wave, x staged once in LDS (padded 16 B per 128 B,
// conflict-free b128 reads) with the sums of its 16-element runs, behind one LDS-only barrier.
// Four lanes per super-block and sixteen super-blocks per 4096-column step; lane (slot, part)
// takes half h = part >> 1 and offset 16 j (j = part & 1) of its super-block, which is the
// four runs e = 128 h + 32 p + 16 j .. + 15 of the four 2-bit planes p, one 16-element scale
// group each (sub-block 8 h + 2 p + j).
//
// Codes are rebuilt four at a time from a dword of plane bytes with byte masks, each left at
// the bit offset where its plane lies when that saves a shift (a power-of-two factor 4^t taken
// out once per run), widened by v_perm_b32 into fp16 subnormal pairs (code * 4^t * 2^-24, all
// below 1024 * 2^-24, so exact) and multiplied with x by v_dot2_f32_f16 (exact products, fp32
// sums): no magic bias to cancel.  Q3_K's "- 4" (its third bit cleared) comes off once per run
// with the run's sum of x, which the staging writes pre-multiplied by -4.
//
// Block formats (public GGML layouts, the same as the dequantizer's decode8):
//   Q2_K, 84 B: scales[16] (low nibble scale, high nibble min), qs[64], fp16 d, fp16 dmin;
//     element 128 h + 32 p + l: (qs[32 h + l] >> 2 p) & 3, value d * sc * q - dmin * m.
//   Q3_K, 110 B: hmask[32], qs[64], 12 bytes of 6-bit scales, fp16 d; element
//     128 h + 32 p + l: q = (qs[32 h + l] >> 2 p) & 3 | bit (4 h + p) of hmask[l] << 2,
//     value d * (scale - 32) * (q - 4).
#include "gguf_common.h"
#include "gguf_launch.h"

namespace tensor_gguf {

// Slot of run r = e / 16 of a row (e = 256 b + 128 h + 32 p + 16 j) in the table of run sums:
// 16 b + 8 h + 4 j + p, so the four runs of one lane (fixed b, h, j) are adjacent.
__device__ __forceinline__ int q23k_run_slot(int r) {
  return (r & ~15) | (r & 8) | ((r & 1) << 2) | ((r >> 1) & 3);
}

// Q3_K's 110-byte blocks start at 2 mod 4 bytes in odd slots, and loads that are not 4-byte
// aligned cost the kernel about a fifth of its time (loads alone at 12288 x 4096: 5.9 against
// 4.8 us aligned).  So every Q3_K load is 4-aligned: a 16-byte window that starts sh = 0 or 2
// bytes before the piece it is for, and the dword after it for the piece's last sh bytes.
// The 16 bytes at byte sh (0..3) of the window w followed by the dword next.
__device__ __forceinline__ uint4 realign(const uint4& w, uint32_t next, uint32_t sh) {
  return make_uint4(__builtin_amdgcn_alignbyte(w.y, w.x, sh), __builtin_amdgcn_alignbyte(w.z, w.y, sh),
                    __builtin_amdgcn_alignbyte(w.w, w.z, sh), __builtin_amdgcn_alignbyte(next, w.w, sh));
}

// Bytes 0 and 1 of c as the fp16 subnormal pair (c0, c1) * 2^-24; bytes 2 and 3 likewise.
__device__ __forceinline__ uint32_t sub01(uint32_t c) { return __builtin_amdgcn_perm(0u, c, 0x0C010C00u); }
__device__ __forceinline__ uint32_t sub23(uint32_t c) { return __builtin_amdgcn_perm(0u, c, 0x0C030C02u); }

template <int TYPE, int R, int STEPS, int WAVES, typename OutT>
__global__ __launch_bounds__(WAVES * 64) void gemv_q23k(const _Float16* __restrict__ x, const uint8_t* __restrict__ w,
                                                        OutT* __restrict__ out, int n_rows) {
  constexpr bool Q3 = TYPE == kQ3_K;
  constexpr int BLOCK = Q3 ? 110 : 84;
  constexpr int K = STEPS * 4096, ROW_BYTES = STEPS * 16 * BLOCK;
  constexpr int T = WAVES * 64, XC = (K / 8 + T - 1) / T;  // 16-byte x chunks per thread
  __shared__ __attribute__((aligned(16))) uint8_t xlds[K * 2 + K / 4];
  __shared__ __attribute__((aligned(16))) float sxl[K / 16];  // run sums (Q3_K: times -4), q23k_run_slot order
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * WAVES + (threadIdx.x >> 6)) * R;
  const int slot = lane >> 2, part = lane & 3, h = part >> 1, j = part & 1;
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (c < K / 8) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * c);
  }
  // per step: the lane's 16 plane bytes; Q3_K: its 16 hmask bytes and the 14 bytes of scales
  // and d (as the windows described above); Q2_K: its 8 scale bytes (8 h ..) and d, dmin
  uint4 qs[R][STEPS], hm[R][STEPS], hd[R][STEPS];
  uint32_t qn[R][STEPS], hn[R][STEPS];
  uint2 sa[R][STEPS];
  uint32_t dd[R][STEPS];
  // Q3_K: block address mod 4 (w is 4-aligned and rows and steps are whole dwords)
  const uint32_t sh = 2 * (slot & 1);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint8_t* wr = w + (size_t)min(row0 + r, n_rows - 1) * ROW_BYTES + slot * BLOCK;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const uint8_t* block = wr + s * 16 * BLOCK;
      if constexpr (Q3) {
        // windows at block - sh + ...: the hmask window of an odd slot starts in the block
        // before it, and the header window of an even slot ends 2 bytes into the one after
        const uint8_t* win = block - sh;
        qs[r][s] = load16(win + 32 + 16 * part);
        qn[r][s] = load4(win + 48 + 16 * part);
        hm[r][s] = load16(win + 16 * j);
        hn[r][s] = load4(win + 16 + 16 * j);
        hd[r][s] = load16(win + 96);
      } else {
        qs[r][s] = load16(block + 16 + 32 * h + 16 * j);
        sa[r][s] = load8(block + 8 * h);
        dd[r][s] = load4(block + 80);
      }
    }
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (c < K / 8) {
      *reinterpret_cast<uint4*>(xlds + 16 * c + 16 * (c >> 3)) = xr[i];
      // chunks c and c ^ 1 make one run (K / 8 is even: both lanes are in range)
      const float sum = dpp_add<0xB1>(sum8(xr[i]));
      if ((c & 1) == 0) sxl[q23k_run_slot(c >> 1)] = Q3 ? -4.0f * sum : sum;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (row0 >= n_rows) return;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    // one step at a time: without this fence every step's x reads move up to the barrier
    // and stay live together (160 against 61 VGPRs at three steps)
    if (s) asm volatile("" ::: "memory");
    const int sb_index = s * 16 + slot;
    uint4 xs[4][2];
    const float4 s4 = *reinterpret_cast<const float4*>(&sxl[sb_index * 16 + 8 * h + 4 * j]);
    const float sx[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int ch = (sb_index * 256 + 128 * h + 32 * p + 16 * j) >> 3;
      xs[p][0] = *reinterpret_cast<const uint4*>(xlds + 16 * ch + 16 * (ch >> 3));
      xs[p][1] = *reinterpret_cast<const uint4*>(xlds + 16 * (ch + 1) + 16 * ((ch + 1) >> 3));
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint4 qv = qs[r][s], hv = hm[r][s];
      if constexpr (Q3) {
        qv = realign(qv, qn[r][s], sh);
        hv = realign(hv, hn[r][s], sh);
      }
      float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t Q = word(qv, u);
        uint32_t c[4];
        if constexpr (Q3) {
          // plane p's two bits and its third bit (bit 4 h + p of the hmask byte) side by side:
          // planes 0 and 2 at bits 0-2 (factor 1), planes 1 and 3 at bits 2-4 (factor 4)
          const uint32_t H = word(hv, u) >> (4 * h), Q4 = Q >> 4;
          c[0] = (Q & 0x03030303u) | ((H << 2) & 0x04040404u);
          c[1] = (Q & 0x0C0C0C0Cu) | ((H << 3) & 0x10101010u);
          c[2] = (Q4 & 0x03030303u) | (H & 0x04040404u);
          c[3] = (Q4 & 0x0C0C0C0Cu) | ((H << 1) & 0x10101010u);
        } else {
          // plane p in place: factor 4^p
          c[0] = Q & 0x03030303u;
          c[1] = Q & 0x0C0C0C0Cu;
          c[2] = Q & 0x30303030u;
          c[3] = Q & 0xC0C0C0C0u;
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          a[p] = dot2(sub01(c[p]), word(xs[p][u >> 1], 2 * (u & 1)), a[p]);
          a[p] = dot2(sub23(c[p]), word(xs[p][u >> 1], 2 * (u & 1) + 1), a[p]);
        }
      }
      if constexpr (Q3) {
        // the lane's scales: sub-blocks 8 h + 2 p + j, bytes 0 and 2 of the 6-bit scale dwords
        // of sub-blocks 8 h .. 8 h + 3 (Sa) and 8 h + 4 .. (Sb) after a shift by 8 j
        const uint4 hw = hd[r][s];  // scale bytes 0-11 and d at byte sh
        const int shs = 4 * h + 8 * j;
        const uint32_t hs = __builtin_amdgcn_alignbyte(hw.w, hw.z, sh) >> shs;  // scale bytes 8-11
        const uint32_t Sa = ((__builtin_amdgcn_alignbyte(hw.y, hw.x, sh) >> shs) & 0x0F0F0F0Fu) | ((hs << 4) & 0x30303030u);
        const uint32_t Sb = ((__builtin_amdgcn_alignbyte(hw.z, hw.y, sh) >> shs) & 0x0F0F0F0Fu) | ((hs << 2) & 0x30303030u);
        const float d = half_bits_to_float(hw.w >> (8 * sh));
        const float sc[4] = {(float)(Sa & 0xFFu), (float)((Sa >> 16) & 0xFFu), (float)(Sb & 0xFFu),
                             (float)((Sb >> 16) & 0xFFu)};
        float v = 0.f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          // sum over the run of (q - 4) x = a * 2^24 / factor - 4 * (sum of x)
          const float t = fmaf(a[p], (p & 1) ? 4194304.0f : 16777216.0f, sx[p]);
          v = fmaf(sc[p] - 32.0f, t, v);
        }
        acc[r] = fmaf(d, v, acc[r]);
      } else {
        const uint32_t S0 = sa[r][s].x >> (8 * j), S1 = sa[r][s].y >> (8 * j);
        const uint32_t lo0 = S0 & 0x0F0F0F0Fu, lo1 = S1 & 0x0F0F0F0Fu;
        const uint32_t hi0 = (S0 >> 4) & 0x0F0F0F0Fu, hi1 = (S1 >> 4) & 0x0F0F0F0Fu;
        const float sc[4] = {(float)(lo0 & 0xFFu), (float)((lo0 >> 16) & 0xFFu), (float)(lo1 & 0xFFu),
                             (float)((lo1 >> 16) & 0xFFu)};
        const float mn[4] = {(float)(hi0 & 0xFFu), (float)((hi0 >> 16) & 0xFFu), (float)(hi1 & 0xFFu),
                             (float)((hi1 >> 16) & 0xFFu)};
        float vd = 0.f, vm = 0.f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          // sum over the run of q x = a * 2^24 / 4^p
          vd = fmaf(sc[p], a[p] * (float)(16777216 >> (2 * p)), vd);
          vm = fmaf(mn[p], sx[p], vm);
        }
        acc[r] = fmaf(half_bits_to_float(dd[r][s]), vd, acc[r]);
        acc[r] = fmaf(-half_bits_to_float(dd[r][s] >> 16), vm, acc[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < n_rows) store_out<OutT>(out, (size_t)(row0 + r), v);
  }
}

// R = 2 rows per wave where one row per wave would take more than one round of 8 waves per
// SIMD (K = 4096 and more than 8192 rows): then every wave is resident from the start.
template <int TYPE, int STEPS, typename OutT>
static hipError_t launch_q23k(const GemvArgs& a, hipStream_t stream) {
  constexpr int WAVES = 8;
  if constexpr (STEPS == 1) {
    if (a.n > 8192) {
      hipLaunchKernelGGL((gemv_q23k<TYPE, 2, STEPS, WAVES, OutT>), dim3((a.n + 2 * WAVES - 1) / (2 * WAVES)),
                         dim3(WAVES * 64), 0, stream, static_cast<const _Float16*>(a.x),
                         static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out), a.n);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv_q23k<TYPE, 1, STEPS, WAVES, OutT>), dim3((a.n + WAVES - 1) / WAVES), dim3(WAVES * 64), 0,
                     stream, static_cast<const _Float16*>(a.x), static_cast<const uint8_t*>(a.w),
                     static_cast<OutT*>(a.out), a.n);
  return hipGetLastError();
}

template <int TYPE, typename OutT>
static hipError_t launch_q23k_typed(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = true;
  switch (a.k) {
    case 4096: return launch_q23k<TYPE, 1, OutT>(a, stream);
    case 8192: return launch_q23k<TYPE, 2, OutT>(a, stream);
    case 12288: return launch_q23k<TYPE, 3, OutT>(a, stream);
    case 16384: return launch_q23k<TYPE, 4, OutT>(a, stream);
    default: *handled = false; return hipSuccess;
  }
}

hipError_t launch_gemv_q23k_fast(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = false;
  if (a.m != 1 || a.n <= 0) return hipSuccess;
  // Q3_K's windows assume 4-byte aligned weights (the entry points accept 16-byte aligned buffers only)
  if (a.type == kQ3_K && (reinterpret_cast<uintptr_t>(a.w) & 3) == 0)
    return a.out_half ? launch_q23k_typed<kQ3_K, _Float16>(a, stream, handled)
                      : launch_q23k_typed<kQ3_K, float>(a, stream, handled);
  if (a.type == kQ2_K)
    return a.out_half ? launch_q23k_typed<kQ2_K, _Float16>(a, stream, handled)
                      : launch_q23k_typed<kQ2_K, float>(a, stream, handled);
  return hipSuccess;
}

}  // namespace tensor_gguf
