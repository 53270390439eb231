// Q6_K decode GEMV fast path (gfx950) for M = 1 and K a multiple of 4096,
// the LM-head and down-projection shapes: out[n] = sum_k x[k] * W[n, k].
//
// A workgroup of 8 waves, one row each, loads the activation vector first, then
// every weight byte of its rows, and stages x once in LDS (padded 16 B per
// 128 B, conflict-free b128 reads) behind a single LDS-only barrier, so the
// activation vector is read from L2 once per 8 rows instead of once per wave.  Lane plan as the generic kernel: four lanes
// per 210-byte super-block (half hh, 16-element offset l0), sixteen
// super-blocks per step; each lane rebuilds its 64 six-bit codes with byte
// masks and multiplies "1024 + q" fp16 codes with v_dot2_f32_f16, removing
// the 1056 bias (1024 + 32) once per 16-element scale group.
//
// Block format: benchmarks/kernels/showcase/triton_kernels.py:163-180.
#include "gguf_common.h"
#include "gguf_launch.h"

namespace tensor_gguf {

// ALIGNED (w 4-byte aligned; used at K = 4096): the 210-byte blocks of odd slots start at 2 mod
// 4, and loads that are not 4-byte aligned cost the LM head about 7% (151936 x 4096 in a timing
// harness: 83.5 against 90.1 us, identical outputs).  Each piece is then read as the 16-byte
// window sh = block mod 4 bytes before it, and its last sh bytes come from the first dword of
// the window after it, which a neighbouring lane of the quad holds (a DPP quad permute); the
// scale bytes as a 12-byte window and d from the dword at byte 208 - sh.
__device__ __forceinline__ uint4 q6k_realign(const uint4& w, uint32_t next, uint32_t sh) {
  return make_uint4(__builtin_amdgcn_alignbyte(w.y, w.x, sh), __builtin_amdgcn_alignbyte(w.z, w.y, sh),
                    __builtin_amdgcn_alignbyte(w.w, w.z, sh), __builtin_amdgcn_alignbyte(next, w.w, sh));
}
template <int CONTROL>
__device__ __forceinline__ uint32_t q6k_quad_mov(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CONTROL, 0xF, 0xF, true);
}

// Slot of run r = e / 16 of a row (e = 256 b + 128 hh + 32 c + 16 p) in the table of run sums:
// 16 b + 8 hh + 4 p + c, so the runs c = 0..3 that one lane reads (fixed b, hh, p) are adjacent.
__device__ __forceinline__ int run_slot(int r) { return (r & ~15) | (r & 8) | ((r & 1) << 2) | ((r >> 1) & 3); }

//
// KSPLIT (R = 1): the STEPS steps of a row go to STEPS waves of the workgroup, WAVES / STEPS rows
// per workgroup, each wave one step (so three times the waves of a one-row-per-wave grid, and
// the aligned one-step loads); the waves' totals meet in LDS and are added in step order.
template <int R, int STEPS, int WAVES, typename OutT, bool ALIGNED = false, bool KSPLIT = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_q6k_lds(const _Float16* __restrict__ x,
                                                           const uint8_t* __restrict__ w,
                                                           OutT* __restrict__ out, int n_rows) {
  static_assert(!KSPLIT || (R == 1 && WAVES % STEPS == 0), "one step per wave");
  constexpr int LS = KSPLIT ? 1 : STEPS;            // steps per wave
  constexpr int ROWS = KSPLIT ? WAVES / STEPS : 0;  // KSPLIT: rows per workgroup
  constexpr int K = STEPS * 4096;
  constexpr int ROW_BYTES = STEPS * 16 * 210;
  constexpr int T = WAVES * 64, XC = (K / 8 + T - 1) / T;  // 16-byte x chunks per thread
  __shared__ __attribute__((aligned(16))) uint8_t xlds[K * 2 + K / 4];
  // sums of the K / 16 runs of 16 x, super-block by super-block in the order the lanes read
  // them (see run_slot), staged with x so that no wave sums x itself
  __shared__ __attribute__((aligned(16))) float sxl[K / 16];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = KSPLIT ? blockIdx.x * ROWS + wave % (KSPLIT ? ROWS : 1) : (blockIdx.x * WAVES + wave) * R;
  const int s0 = KSPLIT ? wave / (KSPLIT ? ROWS : 1) : 0;  // the wave's first step
  const int slot = lane >> 2, part = lane & 3, hh = part >> 1, l0 = 16 * (part & 1);
  // x first, then every weight load of the wave, pinned above a compiler barrier: on each CU
  // the small x load is not queued behind weight traffic, and the workgroup barrier below
  // fences LDS only, so decoding starts as soon as this wave's own bytes have arrived
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (c < K / 8) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * c);
  }
  uint4 qa[R][LS], qb[R][LS], qh[R][LS];
  uint2 sc8[R][LS];
  uint32_t sc_next[R][LS];  // ALIGNED: the dword after the 8 scale bytes' window
  uint32_t dw[R][LS];
  const uint32_t sh = ALIGNED ? 2 * (slot & 1) : 0;  // block address mod 4
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint8_t* wr = w + (size_t)min(row0 + r, n_rows - 1) * ROW_BYTES + slot * 210;
#pragma unroll
    for (int s = 0; s < LS; ++s) {
      const uint8_t* block = wr + (s0 + s) * 16 * 210;
      if constexpr (ALIGNED) {
        // windows at block - sh: those of an odd slot start in the even block before it, and the
        // last ones of an even slot end 2 bytes into the odd block after it
        const uint8_t* win = block - sh;
        qa[r][s] = load16(win + 64 * hh + l0);
        qb[r][s] = load16(win + 64 * hh + 32 + l0);
        qh[r][s] = load16(win + 128 + 32 * hh + l0);
        uint3 t;
        __builtin_memcpy(&t, win + 192 + 8 * hh, 12);
        sc8[r][s] = make_uint2(t.x, t.y);
        sc_next[r][s] = t.z;
        dw[r][s] = load4(win + 208);  // d at byte sh
      } else {
        qa[r][s] = load16(block + 64 * hh + l0);
        qb[r][s] = load16(block + 64 * hh + 32 + l0);
        qh[r][s] = load16(block + 128 + 32 * hh + l0);
        sc8[r][s] = load8(block + 192 + 8 * hh);
        dw[r][s] = load4(block + 206);  // high half: d
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
      const float s = dpp_add<0xB1>(sum8(xr[i]));
      if ((c & 1) == 0) sxl[run_slot(c >> 1)] = s;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (!KSPLIT && row0 >= n_rows) return;  // KSPLIT: every wave meets the second barrier
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
#pragma unroll
  for (int s = 0; s < LS; ++s) {
    // the four 16-element runs 128 hh + 32 c + l0 (c = 0..3), one scale group each; their
    // sums of x are four consecutive slots
    uint4 xs[4][2];
    const int sb = (s0 + s) * 16 + slot;  // super-block index in the row
    const float4 s4 = *reinterpret_cast<const float4*>(&sxl[sb * 16 + 8 * hh + 4 * (part & 1)]);
    const float sx[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int ch = (sb * 256 + 128 * hh + 32 * c + l0) >> 3;
      xs[c][0] = *reinterpret_cast<const uint4*>(xlds + 16 * ch + 16 * (ch >> 3));
      xs[c][1] = *reinterpret_cast<const uint4*>(xlds + 16 * (ch + 1) + 16 * ((ch + 1) >> 3));
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      uint4 QA = qa[r][s], QB = qb[r][s], QH = qh[r][s];
      uint2 SC = sc8[r][s];
      float d;
      if constexpr (ALIGNED) {
        // the first dword of the window after each piece: for qa of part 0..3 part 1's qa,
        // part 0's qb, part 3's qa, part 2's qb; for qb part 1's qb, part 2's qa, part 3's qb,
        // part 0's qh; for qh parts 1, 2, 3's qh and part 0's scale window
        const uint32_t send_a = (part & 1) ? QA.x : QB.x;
        const uint32_t send_b = part == 0 ? QH.x : (part == 2 ? QA.x : QB.x);
        const uint32_t send_h = part == 0 ? SC.x : QH.x;
        const uint32_t next_a = q6k_quad_mov<0xB1>(send_a);  // quad_perm [1, 0, 3, 2]
        const uint32_t next_b = q6k_quad_mov<0x39>(send_b);  // quad_perm [1, 2, 3, 0]
        const uint32_t next_h = q6k_quad_mov<0x39>(send_h);
        QA = q6k_realign(QA, next_a, sh);
        QB = q6k_realign(QB, next_b, sh);
        QH = q6k_realign(QH, next_h, sh);
        SC = make_uint2(__builtin_amdgcn_alignbyte(SC.y, SC.x, sh), __builtin_amdgcn_alignbyte(sc_next[r][s], SC.y, sh));
        d = half_bits_to_float(dw[r][s] >> (8 * sh));
      } else {
        d = half_bits_to_float(dw[r][s] >> 16);
      }
      float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t A = word(QA, u), B = word(QB, u), H = word(QH, u);
        uint32_t q[4];
        q[0] = (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
        q[1] = (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
        q[2] = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
        q[3] = ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          a[c] = dot2(magic01(q[c]), word(xs[c][u >> 1], 2 * (u & 1)), a[c]);
          a[c] = dot2(magic23(q[c]), word(xs[c][u >> 1], 2 * (u & 1) + 1), a[c]);
        }
      }
      // scale of run c: byte 2c + l0/16 of the 8 scale bytes of this half
      const int p = part & 1;
      const float ds0 = d * (float)(int8_t)(SC.x >> (8 * p));
      const float ds1 = d * (float)(int8_t)(SC.x >> (8 * (2 + p)));
      const float ds2 = d * (float)(int8_t)(SC.y >> (8 * p));
      const float ds3 = d * (float)(int8_t)(SC.y >> (8 * (2 + p)));
      float v = acc[r];
      v = fmaf(ds0, a[0] - 1056.0f * sx[0], v);
      v = fmaf(ds1, a[1] - 1056.0f * sx[1], v);
      v = fmaf(ds2, a[2] - 1056.0f * sx[2], v);
      v = fmaf(ds3, a[3] - 1056.0f * sx[3], v);
      acc[r] = v;
    }
  }
  if constexpr (KSPLIT) {
    __shared__ float red[WAVES];  // wave totals, wave = step * ROWS + row in the workgroup
    const float v = wave_sum(acc[0]);
    if (lane == 0) red[wave] = v;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (wave < ROWS && lane == 0 && row0 < n_rows) {
      float total = red[wave];
#pragma unroll
      for (int s = 1; s < STEPS; ++s) total += red[s * ROWS + wave];
      store_out<OutT>(out, (size_t)row0, total);
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(acc[r]);
      if (lane == 0 && row0 + r < n_rows) store_out<OutT>(out, (size_t)(row0 + r), v);
    }
  }
}

// fp32 activations at M = 1 (the packed call form): gemv_q6k_lds's lane plan and loads, each
// six-bit code converted to fp32 and multiplied by the fp32 activation (the reference's decode
// numerics, fp32 operands, benchmark.py:466-472, up to summation order), d * scale and the bias
// 32 applied once per 16-element run with the run's fp32 sum of x.  x sits in LDS as 16-byte
// chunks of 4 floats, chunk c at a swizzled position: the lanes of one b128 read (slot s, part p)
// read chunks 64 s + 32 (p >> 1) + 4 (p & 1) + 8 run + u, which differ only in bits 2, 5, 6 and
// 7; XOR-ing bits 5-7 into bits 0-3 spreads 16 of them over all 64 banks.
__device__ __forceinline__ int q6k_f32_chunk(int c) { return 4 * (c ^ ((((c >> 5) & 1) << 3) | ((c >> 6) & 3))); }

template <int STEPS, int WAVES, typename OutT>
__global__ __launch_bounds__(WAVES * 64) void gemv_q6k_f32(const float* __restrict__ x, const uint8_t* __restrict__ w,
                                                           OutT* __restrict__ out, int n_rows) {
  constexpr int K = STEPS * 4096, ROW_BYTES = STEPS * 16 * 210, T = WAVES * 64, XC = K / 4 / T;
  static_assert(XC * T * 4 == K, "every thread stages whole chunks");
  __shared__ __attribute__((aligned(16))) float xlds[K];
  __shared__ __attribute__((aligned(16))) float sxl[K / 16];  // run sums, in run_slot order
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * WAVES + (threadIdx.x >> 6);
  const int slot = lane >> 2, part = lane & 3, hh = part >> 1, l0 = 16 * (part & 1);
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * (threadIdx.x + i * T));
  uint4 qa[STEPS], qb[STEPS], qh[STEPS];
  uint2 sc8[STEPS];
  uint32_t dw[STEPS];
  const uint8_t* wr = w + (size_t)min(row, n_rows - 1) * ROW_BYTES + slot * 210;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const uint8_t* block = wr + s * 16 * 210;
    qa[s] = load16(block + 64 * hh + l0);
    qb[s] = load16(block + 64 * hh + 32 + l0);
    qh[s] = load16(block + 128 + 32 * hh + l0);
    sc8[s] = load8(block + 192 + 8 * hh);
    dw[s] = load4(block + 206);  // high half: d
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    const uint4 v = xr[i];
    *reinterpret_cast<uint4*>(&xlds[q6k_f32_chunk(c)]) = v;
    // a 16-element run is 4 consecutive chunks, held by one quad of lanes
    const float sum = quad_sum((__uint_as_float(v.x) + __uint_as_float(v.y)) + (__uint_as_float(v.z) + __uint_as_float(v.w)));
    if ((c & 3) == 0) sxl[run_slot(c >> 2)] = sum;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (row >= n_rows) return;
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const float4 s4 = *reinterpret_cast<const float4*>(&sxl[(s * 16 + slot) * 16 + 8 * hh + 4 * (part & 1)]);
    const float sx[4] = {s4.x, s4.y, s4.z, s4.w};
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t A = word(qa[s], u), B = word(qb[s], u), H = word(qh[s], u);
      uint32_t q[4];
      q[0] = (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
      q[1] = (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
      q[2] = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
      q[3] = ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        // run c: elements 256 sb + 128 hh + 32 c + l0 + 4 u .. + 3
        const int chunk = ((s * 16 + slot) * 256 + 128 * hh + 32 * c + l0 + 4 * u) >> 2;
        const float4 xv = *reinterpret_cast<const float4*>(&xlds[q6k_f32_chunk(chunk)]);
        a[c] = fmaf((float)(q[c] & 0xFF), xv.x, a[c]);
        a[c] = fmaf((float)((q[c] >> 8) & 0xFF), xv.y, a[c]);
        a[c] = fmaf((float)((q[c] >> 16) & 0xFF), xv.z, a[c]);
        a[c] = fmaf((float)(q[c] >> 24), xv.w, a[c]);
      }
    }
    const float d = half_bits_to_float(dw[s] >> 16);
    const int p = part & 1;
    acc = fmaf(d * (float)(int8_t)(sc8[s].x >> (8 * p)), a[0] - 32.0f * sx[0], acc);
    acc = fmaf(d * (float)(int8_t)(sc8[s].x >> (8 * (2 + p))), a[1] - 32.0f * sx[1], acc);
    acc = fmaf(d * (float)(int8_t)(sc8[s].y >> (8 * p)), a[2] - 32.0f * sx[2], acc);
    acc = fmaf(d * (float)(int8_t)(sc8[s].y >> (8 * (2 + p))), a[3] - 32.0f * sx[3], acc);
  }
  const float v = wave_sum(acc);
  if (lane == 0) store_out<OutT>(out, (size_t)row, v);
}

template <int STEPS, typename OutT>
static hipError_t launch_q6k_f32(const GemvArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((gemv_q6k_f32<STEPS, 8, OutT>), dim3((a.n + 7) / 8), dim3(512), 0, stream,
                     static_cast<const float*>(a.x), static_cast<const uint8_t*>(a.w), static_cast<OutT*>(a.out), a.n);
  return hipGetLastError();
}

template <typename OutT>
static hipError_t launch_q6k_f32_typed(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = true;
  switch (a.k) {
    case 4096: return launch_q6k_f32<1, OutT>(a, stream);
    case 8192: return launch_q6k_f32<2, OutT>(a, stream);
    case 12288: return launch_q6k_f32<3, OutT>(a, stream);
    default: *handled = false; return hipSuccess;
  }
}

hipError_t launch_gemv_q6k_f32x(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = false;
  if (a.m != 1 || a.type != kQ6_K || !a.x_f32) return hipSuccess;
  return a.out_half ? launch_q6k_f32_typed<_Float16>(a, stream, handled) : launch_q6k_f32_typed<float>(a, stream, handled);
}

// The aligned loads at K = 4096 (one step), and at K = 12288 in the K-split form (three waves
// per row, four rows per 12-wave workgroup, one aligned step per wave): in a timing harness
// 10.05 against 10.19 us at 4096 x 12288 and 4.58 against 5.75 us at 1001 x 12288, where one
// row per wave leaves most of the GPU idle.  Aligned loads with all three steps in one wave
// measured level or slower (10.24-12.3 against 10.19-10.3 us at 4096 x 12288).
template <int R, int STEPS, int WAVES, typename OutT>
static hipError_t launch_q6k(const GemvArgs& a, hipStream_t stream) {
  constexpr int per_block = WAVES * R;
  const dim3 grid((a.n + per_block - 1) / per_block), block(WAVES * 64);
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  if constexpr (STEPS == 1) {
    if ((reinterpret_cast<uintptr_t>(w) & 3) == 0) {
      hipLaunchKernelGGL((gemv_q6k_lds<R, STEPS, WAVES, OutT, true>), grid, block, 0, stream, x, w, out, a.n);
      return hipGetLastError();
    }
  }
  if constexpr (STEPS == 3 && R == 1) {
    if ((reinterpret_cast<uintptr_t>(w) & 3) == 0) {
      constexpr int KS_WAVES = 12, KS_ROWS = KS_WAVES / STEPS;
      hipLaunchKernelGGL((gemv_q6k_lds<1, STEPS, KS_WAVES, OutT, true, true>), dim3((a.n + KS_ROWS - 1) / KS_ROWS),
                         dim3(KS_WAVES * 64), 0, stream, x, w, out, a.n);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((gemv_q6k_lds<R, STEPS, WAVES, OutT>), grid, block, 0, stream, x, w, out, a.n);
  return hipGetLastError();
}

template <typename OutT>
static hipError_t launch_typed(const GemvArgs& a, hipStream_t stream, bool* handled) {
  *handled = true;
  switch (a.k) {
    case 4096: return launch_q6k<1, 1, 8, OutT>(a, stream);
    case 8192: return launch_q6k<1, 2, 8, OutT>(a, stream);
    case 12288: return launch_q6k<1, 3, 8, OutT>(a, stream);
    default: *handled = false; return hipSuccess;
  }
}

hipError_t launch_gemv_q6k_fast(const GemvArgs& a, hipStream_t stream, bool* handled) {
  if (a.m != 1) {
    *handled = false;
    return hipSuccess;
  }
  return a.out_half ? launch_typed<_Float16>(a, stream, handled) : launch_typed<float>(a, stream, handled);
}

}  // namespace tensor_gguf
