// Decode GEMV over raw GGUF rows: out[m, n] = sum_k x[m, k] * W[n, k].
//
// HBM-bound weight streaming (reference kernel: AKAS gemv_packed, called at
// benchmarks/kernels/showcase/kernels.py:114-119; restated by the Triton
// gguf_gemv at triton_kernels.py:214-222).  Design for gfx950:
//
//  * One wave64 owns R consecutive rows.  Its lanes tile one "step" of the
//    row: every lane issues 16-byte loads of packed block bytes, so one wave
//    load instruction streams a contiguous ~1 KiB stretch of the row.
//  * Packed codes are never converted to float element by element: bytes are
//    spread into fp16 pairs "1024 + code" with one v_perm_b32 per two codes,
//    then v_dot2_f32_f16 multiplies them with the fp16 activations and
//    accumulates in fp32.  The 1024 offset (and the code bias of signed
//    formats) is removed once per block run as  scale * (acc - bias * sum(x)),
//    with sum(x) shared by all R rows of the wave.
//  * Block scales and mins are unpacked in registers; the activation slice of
//    a lane is loaded once per step and reused for all R rows.
//  * Each row's partials are reduced across the wave with shuffles.
#include "gguf_common.h"
#include "gguf_decode.h"
#include "gguf_launch.h"

namespace tensor_gguf {

// x is fp16 [M, K] (row stride K), W raw rows of row_bytes, out [M, N].
//
// SWIGLU = true fuses the gate / up pair of an MLP: a wave owns one output row n,
// its two "rows" are row n of the gate matrix w and of the up matrix w2, and it
// stores silu(gate) * up from the fp32 dot products (no rounding in between).

// Row r of a wave: rows row0 .. row0 + R - 1 of w, or row row0 of w (r = 0) and w2 (r = 1).
template <bool PAIR>
__device__ __forceinline__ const uint8_t* pair_row(const uint8_t* w, const uint8_t* w2, int row0, int r,
                                                   size_t row_bytes) {
  return PAIR ? (r == 0 ? w : w2) + (size_t)row0 * row_bytes : w + (size_t)(row0 + r) * row_bytes;
}

// Reduce each row's lane partials over the wave and store them (lane 0), or the pair's epilogue.
template <bool PAIR, int M, int R, typename OutT>
__device__ __forceinline__ void store_rows(float (&acc)[M][R], OutT* out, int n_rows, int row0, int rows, int lane) {
#pragma unroll
  for (int m = 0; m < M; ++m) {
    if constexpr (PAIR) {
      const float g = wave_sum(acc[m][0]), u = wave_sum(acc[m][1]);
      if (lane == 0) store_out<OutT>(out, (size_t)m * n_rows + row0, swiglu(g, u));
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float v = wave_sum(acc[m][r]);
        if (lane == 0 && r < rows) store_out<OutT>(out, (size_t)m * n_rows + row0 + r, v);
      }
    }
  }
}

// ------------------------------------------------------------------ Q4_K ---
// Lane plan: 8 lanes per 144-byte super-block, 8 super-blocks per step.
// Lane (slot, c): super-block slot = lane/8, 16-byte quant chunk c = lane%8,
// i.e. pair j = c/2 (sub-blocks 2j, 2j+1) and half h = c%2 of its 32 bytes.
// Low nibbles are elements 64j+16h+t of the block, high nibbles 64j+32+16h+t.
template <int M, int R, typename OutT, bool SWIGLU = false>
__global__ __launch_bounds__(256) void gemv_q4k(const _Float16* __restrict__ x,
                                                const uint8_t* __restrict__ w,
                                                OutT* __restrict__ out, int n_rows, int k,
                                                const uint8_t* __restrict__ w2 = nullptr) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (SWIGLU ? 1 : R);
  if (row0 >= n_rows) return;
  const int blocks = k >> 8;
  const size_t row_bytes = (size_t)blocks * 144;
  const int slot = lane >> 3, c = lane & 7, j = c >> 1, h = c & 1;
  const int quant_offset = 16 + 32 * j + 16 * h;
  const int x_offset = 64 * j + 16 * h;
  const int rows = SWIGLU ? R : min(R, n_rows - row0);
  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  for (int b = slot; b < blocks; b += 8) {
    uint4 xl[M][2], xh[M][2];
    float sl[M], sh[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint8_t* xp = reinterpret_cast<const uint8_t*>(x + (size_t)m * k + b * 256 + x_offset);
      xl[m][0] = load16(xp);
      xl[m][1] = load16(xp + 16);
      xh[m][0] = load16(xp + 64);
      xh[m][1] = load16(xp + 80);
    }
    uint4 head[R], quant[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r < rows) {
        const uint8_t* block = pair_row<SWIGLU>(w, w2, row0, r, row_bytes) + (size_t)b * 144;
        head[r] = load16(block);
        quant[r] = load16(block + quant_offset);
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      sl[m] = sum16(xl[m][0], xl[m][1]);
      sh[m] = sum16(xh[m][0], xh[m][1]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= rows) break;
      float al[M], ah[M];
#pragma unroll
      for (int m = 0; m < M; ++m) al[m] = ah[m] = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t q = word(quant[r], u);
        const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
        const uint32_t lo01 = magic01(lo), lo23 = magic23(lo);
        const uint32_t hi01 = magic01(hi), hi23 = magic23(hi);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          al[m] = dot2(lo01, word(xl[m][u >> 1], 2 * (u & 1)), al[m]);
          al[m] = dot2(lo23, word(xl[m][u >> 1], 2 * (u & 1) + 1), al[m]);
          ah[m] = dot2(hi01, word(xh[m][u >> 1], 2 * (u & 1)), ah[m]);
          ah[m] = dot2(hi23, word(xh[m][u >> 1], 2 * (u & 1) + 1), ah[m]);
        }
      }
      int sc_lo, mn_lo, sc_hi, mn_hi;
      q4k_scale_pair(head[r].y, head[r].z, head[r].w, j, sc_lo, mn_lo, sc_hi, mn_hi);
      const float d = half_bits_to_float(head[r].x), dmin = half_bits_to_float(head[r].x >> 16);
      const float ds_lo = d * (float)sc_lo, ds_hi = d * (float)sc_hi;
      const float c_lo = 1024.0f * ds_lo + dmin * (float)mn_lo;
      const float c_hi = 1024.0f * ds_hi + dmin * (float)mn_hi;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float v = acc[m][r];
        v = fmaf(ds_lo, al[m], v);
        v = fmaf(-c_lo, sl[m], v);
        v = fmaf(ds_hi, ah[m], v);
        v = fmaf(-c_hi, sh[m], v);
        acc[m][r] = v;
      }
    }
  }
  store_rows<SWIGLU>(acc, out, n_rows, row0, rows, lane);
}

// ------------------------------------------------------------------ Q6_K ---
// Lane plan: 4 lanes per 210-byte super-block, 16 super-blocks per step.
// Lane part p = lane%4: half hh = p/2 (elements 128*hh ..), l0 = 16*(p%2).
// Its 16 bytes of ql at 64hh+l0 (quarters 0 and 2), of ql at 64hh+32+l0
// (quarters 1 and 3) and of qh at 128+32hh+l0 decode the four 16-element
// runs 128hh + 32c + l0 + t (c = 0..3), each one scale group.
template <int M, int R, typename OutT, bool SWIGLU = false>
__global__ __launch_bounds__(256) void gemv_q6k(const _Float16* __restrict__ x,
                                                const uint8_t* __restrict__ w,
                                                OutT* __restrict__ out, int n_rows, int k,
                                                const uint8_t* __restrict__ w2 = nullptr) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (SWIGLU ? 1 : R);
  if (row0 >= n_rows) return;
  const int blocks = k >> 8;
  const size_t row_bytes = (size_t)blocks * 210;
  const int slot = lane >> 2, part = lane & 3, hh = part >> 1, l0 = 16 * (part & 1);
  const int rows = SWIGLU ? R : min(R, n_rows - row0);
  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  for (int b = slot; b < blocks; b += 16) {
    uint4 xs[M][4][2];
    float sx[M][4];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint8_t* xp =
            reinterpret_cast<const uint8_t*>(x + (size_t)m * k + b * 256 + 128 * hh + 32 * c + l0);
        xs[m][c][0] = load16(xp);
        xs[m][c][1] = load16(xp + 16);
      }
    uint4 qa[R], qb[R], qh[R];
    uint2 sc8[R];
    uint32_t dword[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r < rows) {
        const uint8_t* block = pair_row<SWIGLU>(w, w2, row0, r, row_bytes) + (size_t)b * 210;
        qa[r] = load16(block + 64 * hh + l0);
        qb[r] = load16(block + 64 * hh + 32 + l0);
        qh[r] = load16(block + 128 + 32 * hh + l0);
        sc8[r] = load8(block + 192 + 8 * hh);
        dword[r] = load4(block + 206);  // high half is d
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) sx[m][c] = sum16(xs[m][c][0], xs[m][c][1]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= rows) break;
      float a[M][4];
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) a[m][c] = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t A = word(qa[r], u), B = word(qb[r], u), H = word(qh[r], u);
        uint32_t q[4];
        q[0] = (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
        q[1] = (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
        q[2] = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
        q[3] = ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t p01 = magic01(q[c]), p23 = magic23(q[c]);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            a[m][c] = dot2(p01, word(xs[m][c][u >> 1], 2 * (u & 1)), a[m][c]);
            a[m][c] = dot2(p23, word(xs[m][c][u >> 1], 2 * (u & 1) + 1), a[m][c]);
          }
        }
      }
      const float d = half_bits_to_float(dword[r] >> 16);
      // scale of run c sits at byte 2c + (l0/16) of the 8 bytes at 192 + 8hh
      const int p = part & 1;
      float ds[4];
      ds[0] = d * (float)(int8_t)(sc8[r].x >> (8 * p));
      ds[1] = d * (float)(int8_t)(sc8[r].x >> (8 * (2 + p)));
      ds[2] = d * (float)(int8_t)(sc8[r].y >> (8 * p));
      ds[3] = d * (float)(int8_t)(sc8[r].y >> (8 * (2 + p)));
#pragma unroll
      for (int m = 0; m < M; ++m) {
        float v = acc[m][r];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          v = fmaf(ds[c], a[m][c], v);
          v = fmaf(-1056.0f * ds[c], sx[m][c], v);
        }
        acc[m][r] = v;
      }
    }
  }
  store_rows<SWIGLU>(acc, out, n_rows, row0, rows, lane);
}

// ------------------------------------------------------------ Q8_0, Q4_0 ---
// Lane plan: one 32-element block per lane, 64 blocks per step.
//
// XLDS = true stages x (M * K halves, dynamic LDS) once per workgroup behind one barrier and
// reads the per-block activations from LDS: read from global memory, each lane's 64 bytes
// of x per 18 or 34 weight bytes made the L1 path, not HBM, the limit.
template <int TYPE, int M, int R, typename OutT, bool SWIGLU = false, bool XLDS = false>
__global__ __launch_bounds__(256) void gemv_q32(const _Float16* __restrict__ x,
                                                const uint8_t* __restrict__ w,
                                                OutT* __restrict__ out, int n_rows, int k,
                                                const uint8_t* __restrict__ w2 = nullptr) {
  constexpr int kBytes = TYPE == kQ8_0 ? 34 : 18;
  // bias removed per block: 1024 from the fp16 widening, plus 128 for the
  // sign flip of Q8_0 codes or 8 for the Q4_0 code offset
  constexpr float kBias = TYPE == kQ8_0 ? 1152.0f : 1032.0f;
  extern __shared__ __attribute__((aligned(16))) uint8_t xl[];
  if constexpr (XLDS) {
    const int chunks = M * k / 8;
    for (int c = threadIdx.x; c < chunks; c += 256)
      *reinterpret_cast<uint4*>(xl + 16 * c) = load16(reinterpret_cast<const uint8_t*>(x) + 16 * (size_t)c);
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (SWIGLU ? 1 : R);
  if (row0 >= n_rows) return;
  const int blocks = k >> 5;
  const size_t row_bytes = (size_t)blocks * kBytes;
  const int rows = SWIGLU ? R : min(R, n_rows - row0);
  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

#pragma unroll 2
  for (int b = lane; b < blocks; b += 64) {
    uint4 xs[M][4];
    float sx[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      if constexpr (XLDS) {
        const uint4* xp = reinterpret_cast<const uint4*>(xl + 2 * ((size_t)m * k + b * 32));
#pragma unroll
        for (int i = 0; i < 4; ++i) xs[m][i] = xp[i];
      } else {
        const uint8_t* xp = reinterpret_cast<const uint8_t*>(x + (size_t)m * k + b * 32);
#pragma unroll
        for (int i = 0; i < 4; ++i) xs[m][i] = load16(xp + 16 * i);
      }
    }
    uint32_t head[R];
    uint4 q0[R], q1[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r < rows) {
        const uint8_t* block = pair_row<SWIGLU>(w, w2, row0, r, row_bytes) + (size_t)b * kBytes;
        head[r] = load4(block);  // fp16 d in the low half
        q0[r] = load16(block + 2);
        if (TYPE == kQ8_0) q1[r] = load16(block + 18);
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      sx[m] = sum16(xs[m][0], xs[m][1]) + sum16(xs[m][2], xs[m][3]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= rows) break;
      float a[M];
#pragma unroll
      for (int m = 0; m < M; ++m) a[m] = 0.0f;
      if (TYPE == kQ8_0) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          // flip the sign bit: int8 code v becomes the unsigned byte v + 128
          const uint32_t q = word(u < 4 ? q0[r] : q1[r], u & 3) ^ 0x80808080u;
          const uint32_t p01 = magic01(q), p23 = magic23(q);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            a[m] = dot2(p01, word(xs[m][u >> 1], 2 * (u & 1)), a[m]);
            a[m] = dot2(p23, word(xs[m][u >> 1], 2 * (u & 1) + 1), a[m]);
          }
        }
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t q = word(q0[r], u);
          const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
          const uint32_t lo01 = magic01(lo), lo23 = magic23(lo);
          const uint32_t hi01 = magic01(hi), hi23 = magic23(hi);
#pragma unroll
          for (int m = 0; m < M; ++m) {
            // element t = 4u.. low nibbles; 16 + 4u.. high nibbles
            a[m] = dot2(lo01, word(xs[m][u >> 1], 2 * (u & 1)), a[m]);
            a[m] = dot2(lo23, word(xs[m][u >> 1], 2 * (u & 1) + 1), a[m]);
            a[m] = dot2(hi01, word(xs[m][2 + (u >> 1)], 2 * (u & 1)), a[m]);
            a[m] = dot2(hi23, word(xs[m][2 + (u >> 1)], 2 * (u & 1) + 1), a[m]);
          }
        }
      }
      const float d = half_bits_to_float(head[r]);
#pragma unroll
      for (int m = 0; m < M; ++m) acc[m][r] = fmaf(d, a[m] - kBias * sx[m], acc[m][r]);
    }
  }
  store_rows<SWIGLU>(acc, out, n_rows, row0, rows, lane);
}

// M = 1, K a multiple of 2048 (STEPS = K / 2048 blocks per lane, all of them held in registers):
// the form of the Q4_K M = 1 kernel.  Each thread loads its x chunks into registers first, then
// the lane issues every weight load of its row, and only then is x written to LDS and the
// workgroup met at an LDS-only barrier, so the weight latency runs under the x staging instead
// of after it.  x sits in LDS with 16 bytes of padding per 64-byte block (a lane's four b128
// reads of its block then spread over the banks).  The arithmetic and its order per lane are
// gemv_q32's, so the two kernels give identical results.  Timing harness, weights rotated
// through 10 copies: Q8_0 4096x4096 4.65 -> 4.12 us, 12288x4096 14.1 -> 13.0 us, 4096x12288
// 14.9 -> 13.2 us; Q4_0 3.68 -> 3.24, 8.59 -> 7.40, 8.39 -> 8.03 us (WAVES 8 for one or two
// blocks per lane, else 4).
//
// ALIGNED (w 4-byte aligned): the 34- and 18-byte blocks of odd lanes start at 2 mod 4, so half
// of every load instruction's lanes read unaligned, and loads that are not 4-byte aligned cost
// Q8_0 a sixth of its load time (loads alone at 12288 x 4096: 11.95 against 9.81 us with the
// addresses rounded down).  Every load is then 4-aligned: an even lane reads its block from byte
// 0 (2 bytes more, into the odd block that always follows it) and realigns the codes by 2 bytes;
// an odd lane reads its codes from byte 2 as they are, and its d from the dword 2 bytes before
// the block.
template <int TYPE, int WAVES, int STEPS, typename OutT, bool ALIGNED = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_q32_m1(const _Float16* __restrict__ x,
                                                          const uint8_t* __restrict__ w,
                                                          OutT* __restrict__ out, int n_rows) {
  constexpr int kBytes = TYPE == kQ8_0 ? 34 : 18;
  constexpr int NW = TYPE == kQ8_0 ? 8 : 4;  // code dwords per block
  constexpr float kBias = TYPE == kQ8_0 ? 1152.0f : 1032.0f;  // as in gemv_q32
  constexpr int T = WAVES * 64, K = 2048 * STEPS, BLOCKS = K / 32, CHUNKS = K / 8;
  constexpr int XC = (CHUNKS + T - 1) / T;  // 16-byte x chunks per thread
  __shared__ __attribute__((aligned(16))) uint8_t xl[CHUNKS * 20];  // 64 + 16 bytes per block
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * WAVES + (threadIdx.x >> 6);
  // rows past the last reload it (every wave meets the barrier), then return before the sum
  const uint8_t* const wr = w + (size_t)min(row, n_rows - 1) * (size_t)(BLOCKS * kBytes);
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (CHUNKS % T == 0 || c < CHUNKS) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * c);
  }
  uint32_t head[STEPS];
  uint4 q0[STEPS], q1[STEPS];
  const bool odd = lane & 1;  // ALIGNED: block address mod 4 is 2
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const uint8_t* block = wr + (lane + 64 * s) * kBytes;
    if constexpr (ALIGNED) {
      // even: bytes 0 .. 4 NW - 1 and the dword after them (the last 2 code bytes and the next
      // block's d); odd: the codes from byte 2 and the dword at -2 (d in its high half)
      const uint8_t* win = block + (odd ? 2 : 0);
      q0[s] = load16(win);
      if constexpr (TYPE == kQ8_0) q1[s] = load16(win + 16);
      head[s] = load4(odd ? block - 2 : block + 4 * NW);
    } else {
      head[s] = load4(block);  // fp16 d in the low half
      q0[s] = load16(block + 2);
      if constexpr (TYPE == kQ8_0) q1[s] = load16(block + 18);
    }
  }
  asm volatile("" ::: "memory");  // every load above is issued before the x stores below
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (CHUNKS % T == 0 || c < CHUNKS) *reinterpret_cast<uint4*>(xl + 16 * c + 16 * (c >> 2)) = xr[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (row >= n_rows) return;
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const uint4* xp = reinterpret_cast<const uint4*>(xl + 80 * (lane + 64 * s));
    uint4 xs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[i] = xp[i];
    const float sx = sum16(xs[0], xs[1]) + sum16(xs[2], xs[3]);
    float a = 0.0f;
    uint32_t dbits = head[s];
    if constexpr (ALIGNED) {
      // code word u = bytes 2 + 4u .. of the block: window dwords u, u + 1 shifted by 2 (even
      // lanes) or dword u (odd lanes: shift 0)
      const uint32_t sh = odd ? 0u : 2u;
      uint32_t wd[NW + 1];
      wd[0] = q0[s].x; wd[1] = q0[s].y; wd[2] = q0[s].z; wd[3] = q0[s].w;
      if constexpr (TYPE == kQ8_0) {
        wd[4] = q1[s].x; wd[5] = q1[s].y; wd[6] = q1[s].z; wd[7] = q1[s].w;
      }
      wd[NW] = head[s];
      uint32_t cw[NW];
#pragma unroll
      for (int u = 0; u < NW; ++u) cw[u] = __builtin_amdgcn_alignbyte(wd[u + 1], wd[u], sh);
      q0[s] = make_uint4(cw[0], cw[1], cw[2], cw[3]);
      if constexpr (TYPE == kQ8_0) q1[s] = make_uint4(cw[4], cw[5], cw[6], cw[7]);
      dbits = odd ? head[s] >> 16 : wd[0];
    }
    if constexpr (TYPE == kQ8_0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t q = word(u < 4 ? q0[s] : q1[s], u & 3) ^ 0x80808080u;
        a = dot2(magic01(q), word(xs[u >> 1], 2 * (u & 1)), a);
        a = dot2(magic23(q), word(xs[u >> 1], 2 * (u & 1) + 1), a);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t q = word(q0[s], u);
        const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
        a = dot2(magic01(lo), word(xs[u >> 1], 2 * (u & 1)), a);
        a = dot2(magic23(lo), word(xs[u >> 1], 2 * (u & 1) + 1), a);
        a = dot2(magic01(hi), word(xs[2 + (u >> 1)], 2 * (u & 1)), a);
        a = dot2(magic23(hi), word(xs[2 + (u >> 1)], 2 * (u & 1) + 1), a);
      }
    }
    acc = fmaf(half_bits_to_float(dbits), a - kBias * sx, acc);
  }
  const float v = wave_sum(acc);
  if (lane == 0) store_out<OutT>(out, (size_t)row, v);
}

template <int TYPE, int STEPS, typename OutT>
static void launch_q32_m1_steps(const GemvArgs& a, hipStream_t stream) {
  constexpr int WAVES = STEPS <= 2 ? 8 : 4;
  const dim3 grid((a.n + WAVES - 1) / WAVES), block(WAVES * 64);
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  if ((reinterpret_cast<uintptr_t>(w) & 3) == 0) {
    hipLaunchKernelGGL((gemv_q32_m1<TYPE, WAVES, STEPS, OutT, true>), grid, block, 0, stream, x, w, out, a.n);
    return;
  }
  hipLaunchKernelGGL((gemv_q32_m1<TYPE, WAVES, STEPS, OutT>), grid, block, 0, stream, x, w, out, a.n);
}

// Q4_1, Q5_0 and Q5_1 at M = 1, K a multiple of 2048 up to 16384: gemv_q32_m1's plan (one row
// per wave, one 32-element block per lane and STEPS = K / 2048 blocks per lane held in
// registers, x staged in LDS behind an LDS-only barrier).  Element j < 16 of a block is the low
// nibble of code byte j and element j + 16 its high nibble; Q5's fifth bit of element j is bit
// j of qh, spread four at a time into bit 4 of each code byte by one multiply
// (b * 0x00204081 moves bit k of b to bit 8k).  Codes widen to fp16 "1024 + q" (v_perm_b32) for
// v_dot2_f32_f16; per block, with the sum sx of its 32 x values:
//   Q4_1, Q5_1: d * (a - 1024 sx) + m * sx,   Q5_0: d * (a - 1040 sx)   (a: sum of (1024 + q) x).
// Q5_0's 22-byte blocks start at 2 mod 4 in odd lanes, so its loads are made 4-byte aligned as
// Q8_0's are: an even lane reads 24 bytes from the block's start (2 into the odd block after it)
// and realigns qh and the codes by 2 bytes; an odd lane reads them from byte 2 as they are, and
// its d from the dword 2 bytes before the block.
// Block formats (public GGML layouts): Q4_1 fp16 d, fp16 m, 16 code bytes (20 B); Q5_0 fp16 d,
// 4 bytes qh, 16 code bytes (22 B); Q5_1 fp16 d, fp16 m, qh, 16 code bytes (24 B).
__device__ __forceinline__ uint32_t spread4(uint32_t b) { return (b * 0x00204081u) & 0x01010101u; }

template <int TYPE, int WAVES, int STEPS, typename OutT>
__global__ __launch_bounds__(WAVES * 64) void gemv_q5_m1(const _Float16* __restrict__ x, const uint8_t* __restrict__ w,
                                                         OutT* __restrict__ out, int n_rows) {
  constexpr int kBytes = TYPE == kQ4_1 ? 20 : TYPE == kQ5_0 ? 22 : 24;
  constexpr bool HAS_H = TYPE != kQ4_1;
  constexpr int T = WAVES * 64, K = 2048 * STEPS, BLOCKS = K / 32, CHUNKS = K / 8;
  constexpr int XC = (CHUNKS + T - 1) / T;  // 16-byte x chunks per thread
  __shared__ __attribute__((aligned(16))) uint8_t xl[CHUNKS * 20];  // 64 + 16 bytes per block
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * WAVES + (threadIdx.x >> 6);
  const uint8_t* const wr = w + (size_t)min(row, n_rows - 1) * (size_t)(BLOCKS * kBytes);
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (CHUNKS % T == 0 || c < CHUNKS) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * c);
  }
  // Q5_0: six window dwords (16 + 4 bytes, and the sixth: the dword after them for an even
  // lane, the one holding d for an odd lane); Q4_1 / Q5_1: the d, m dword, Q5_1's qh, the codes
  uint4 qv[STEPS];
  uint32_t w4[STEPS], w5[STEPS];
  const bool odd = lane & 1;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const uint8_t* block = wr + (lane + 64 * s) * kBytes;
    if constexpr (TYPE == kQ5_0) {
      const uint8_t* win = block + (odd ? 2 : 0);
      qv[s] = load16(win);
      w4[s] = load4(win + 16);
      w5[s] = load4(odd ? block - 2 : win + 20);
    } else if constexpr (TYPE == kQ4_1) {
      w5[s] = load4(block);  // d, m
      qv[s] = load16(block + 4);
    } else {
      w5[s] = load4(block);      // d, m
      w4[s] = load4(block + 4);  // qh
      qv[s] = load16(block + 8);
    }
  }
  asm volatile("" ::: "memory");  // every load above is issued before the x stores below
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (CHUNKS % T == 0 || c < CHUNKS) *reinterpret_cast<uint4*>(xl + 16 * c + 16 * (c >> 2)) = xr[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (row >= n_rows) return;
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const uint4* xp = reinterpret_cast<const uint4*>(xl + 80 * (lane + 64 * s));
    uint4 xs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[i] = xp[i];
    const float sx = sum16(xs[0], xs[1]) + sum16(xs[2], xs[3]);
    uint32_t q[4], qh = 0;
    float d, m = 0.0f;
    if constexpr (TYPE == kQ5_0) {
      // even lane: window from byte 0, shift 2; odd lane: from byte 2, shift 0
      const uint32_t sh = odd ? 0u : 2u;
      const uint32_t wd[6] = {qv[s].x, qv[s].y, qv[s].z, qv[s].w, w4[s], w5[s]};
      qh = __builtin_amdgcn_alignbyte(wd[1], wd[0], sh);
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = __builtin_amdgcn_alignbyte(wd[u + 2], wd[u + 1], sh);
      d = half_bits_to_float(odd ? w5[s] >> 16 : wd[0]);
    } else {
      q[0] = qv[s].x; q[1] = qv[s].y; q[2] = qv[s].z; q[3] = qv[s].w;
      if constexpr (TYPE == kQ5_1) qh = w4[s];
      d = half_bits_to_float(w5[s]);
      m = half_bits_to_float(w5[s] >> 16);
    }
    float a = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint32_t lo = q[u] & 0x0F0F0F0Fu, hi = (q[u] >> 4) & 0x0F0F0F0Fu;
      if constexpr (HAS_H) {
        lo |= spread4((qh >> (4 * u)) & 15u) << 4;
        hi |= spread4((qh >> (16 + 4 * u)) & 15u) << 4;
      }
      // element 4u.. low nibbles; 16 + 4u.. high nibbles
      a = dot2(magic01(lo), word(xs[u >> 1], 2 * (u & 1)), a);
      a = dot2(magic23(lo), word(xs[u >> 1], 2 * (u & 1) + 1), a);
      a = dot2(magic01(hi), word(xs[2 + (u >> 1)], 2 * (u & 1)), a);
      a = dot2(magic23(hi), word(xs[2 + (u >> 1)], 2 * (u & 1) + 1), a);
    }
    if constexpr (TYPE == kQ5_0) acc = fmaf(d, a - 1040.0f * sx, acc);
    else acc = fmaf(d, a - 1024.0f * sx, fmaf(m, sx, acc));
  }
  const float v = wave_sum(acc);
  if (lane == 0) store_out<OutT>(out, (size_t)row, v);
}

template <int TYPE, int STEPS, typename OutT>
static void launch_q5_m1_steps(const GemvArgs& a, hipStream_t stream) {
  constexpr int WAVES = STEPS <= 2 ? 8 : 4;
  hipLaunchKernelGGL((gemv_q5_m1<TYPE, WAVES, STEPS, OutT>), dim3((a.n + WAVES - 1) / WAVES), dim3(WAVES * 64), 0,
                     stream, static_cast<const _Float16*>(a.x), static_cast<const uint8_t*>(a.w),
                     static_cast<OutT*>(a.out), a.n);
}

// gemv_q5_m1 for Q4_1 / Q5_0 / Q5_1 at M = 1 and K = 2048 .. 16384 in steps of 2048 (Q5_0: w
// 4-byte aligned, as the entry points' 16-byte buffer alignment ensures); false for the other shapes.
template <typename OutT>
static bool launch_q5_m1(const GemvArgs& a, hipStream_t stream) {
  if (a.m != 1 || a.k % 2048 || a.k > 16384 || a.n <= 0) return false;
  if (a.type == kQ5_0 && (reinterpret_cast<uintptr_t>(a.w) & 3)) return false;
  const int steps = a.k / 2048;
#define TENSOR_GGUF_Q5_M1(T)                                          \
  case T:                                                             \
    switch (steps) {                                                  \
      case 1: launch_q5_m1_steps<T, 1, OutT>(a, stream); return true; \
      case 2: launch_q5_m1_steps<T, 2, OutT>(a, stream); return true; \
      case 3: launch_q5_m1_steps<T, 3, OutT>(a, stream); return true; \
      case 4: launch_q5_m1_steps<T, 4, OutT>(a, stream); return true; \
      case 5: launch_q5_m1_steps<T, 5, OutT>(a, stream); return true; \
      case 6: launch_q5_m1_steps<T, 6, OutT>(a, stream); return true; \
      case 7: launch_q5_m1_steps<T, 7, OutT>(a, stream); return true; \
      default: launch_q5_m1_steps<T, 8, OutT>(a, stream); return true; \
    }
  switch (a.type) {
    TENSOR_GGUF_Q5_M1(kQ4_1)
    TENSOR_GGUF_Q5_M1(kQ5_0)
    TENSOR_GGUF_Q5_M1(kQ5_1)
    default: return false;
  }
#undef TENSOR_GGUF_Q5_M1
}

// gemv_q32_m1 for K = 2048 .. 16384 in steps of 2048; false for the other shapes.
template <int TYPE, typename OutT>
static bool launch_q32_m1(const GemvArgs& a, hipStream_t stream) {
  if (a.m != 1 || a.k % 2048) return false;
  switch (a.k / 2048) {
    case 1: launch_q32_m1_steps<TYPE, 1, OutT>(a, stream); return true;
    case 2: launch_q32_m1_steps<TYPE, 2, OutT>(a, stream); return true;
    case 3: launch_q32_m1_steps<TYPE, 3, OutT>(a, stream); return true;
    case 4: launch_q32_m1_steps<TYPE, 4, OutT>(a, stream); return true;
    case 5: launch_q32_m1_steps<TYPE, 5, OutT>(a, stream); return true;
    case 6: launch_q32_m1_steps<TYPE, 6, OutT>(a, stream); return true;
    case 7: launch_q32_m1_steps<TYPE, 7, OutT>(a, stream); return true;
    case 8: launch_q32_m1_steps<TYPE, 8, OutT>(a, stream); return true;
    default: return false;
  }
}

// fp32 activations at M = 1 (the packed call form), Q8_0 and Q4_0, K = 1024 or a multiple of 2048
// (KB = K / 32 blocks; at K = 1024 lanes 32-63 hold no block):
// gemv_q32_m1's lane plan and loads (lane = 32-element block, one row per wave), each code
// converted to fp32 and multiplied by the fp32 activation (the reference's decode numerics, fp32
// operands, benchmark.py:466-472, up to summation order); the code bias (128 for the int8 codes
// read as unsigned bytes, 8 for the nibbles) taken off with the block's fp32 sum of x, d once
// per block.  x sits in LDS as fp32 chunks of 4, 16 bytes of padding per 128-byte block.
template <int TYPE, int WAVES, int KB, typename OutT>
__global__ __launch_bounds__(WAVES * 64) void gemv_q32_m1_f32(const float* __restrict__ x, const uint8_t* __restrict__ w,
                                                              OutT* __restrict__ out, int n_rows) {
  constexpr int kBytes = TYPE == kQ8_0 ? 34 : 18;
  constexpr float kBias = TYPE == kQ8_0 ? 128.0f : 8.0f;
  constexpr int STEPS = (KB + 63) / 64;
  static_assert(KB == 32 || KB % 64 == 0, "K = 1024 or a multiple of 2048");
  constexpr int T = WAVES * 64, K = 32 * KB, BLOCKS = KB, CHUNKS = K / 4;
  constexpr int XC = (CHUNKS + T - 1) / T;
  __shared__ __attribute__((aligned(16))) float xl[CHUNKS * 4 + BLOCKS * 4];
  __shared__ float sxl[BLOCKS];
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * WAVES + (threadIdx.x >> 6);
  const uint8_t* const wr = w + (size_t)min(row, n_rows - 1) * (size_t)(BLOCKS * kBytes);
  uint4 xr[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (CHUNKS % T == 0 || c < CHUNKS) xr[i] = load16(reinterpret_cast<const uint8_t*>(x) + 16 * c);
  }
  uint32_t head[STEPS];
  uint4 q0[STEPS], q1[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    // K = 1024: lanes past the 32 blocks read block 31 again and add nothing
    const uint8_t* block = wr + min(lane + 64 * s, BLOCKS - 1) * kBytes;
    head[s] = load4(block);
    q0[s] = load16(block + 2);
    if constexpr (TYPE == kQ8_0) q1[s] = load16(block + 18);
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int c = threadIdx.x + i * T;
    if (CHUNKS % T == 0 || c < CHUNKS) {
      const uint4 v = xr[i];
      *reinterpret_cast<uint4*>(&xl[4 * c + 4 * (c >> 3)]) = v;
      // a block is 8 consecutive chunks, held by 8 consecutive lanes (CHUNKS is a multiple of 8)
      const float part = (__uint_as_float(v.x) + __uint_as_float(v.y)) + (__uint_as_float(v.z) + __uint_as_float(v.w));
      const float sum = dpp_add<0x141>(quad_sum(part));
      if ((c & 7) == 0) sxl[c >> 3] = sum;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  if (row >= n_rows) return;
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int b = min(lane + 64 * s, BLOCKS - 1);
    const float* xp = &xl[36 * b];  // the block's 8 chunks (32 floats and 4 of padding per block)
    float a = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      uint32_t codes;
      int e;  // first element of the four codes
      if constexpr (TYPE == kQ8_0) {
        codes = word(u < 4 ? q0[s] : q1[s], u & 3) ^ 0x80808080u;  // q + 128 as unsigned bytes
        e = 4 * u;
      } else {
        // byte j's low nibble is element j, its high nibble element j + 16
        codes = (word(q0[s], u & 3) >> (4 * (u >> 2))) & 0x0F0F0F0Fu;
        e = 4 * (u & 3) + 16 * (u >> 2);
      }
      const float4 xv = *reinterpret_cast<const float4*>(xp + e);
      a = fmaf((float)(codes & 0xFF), xv.x, a);
      a = fmaf((float)((codes >> 8) & 0xFF), xv.y, a);
      a = fmaf((float)((codes >> 16) & 0xFF), xv.z, a);
      a = fmaf((float)(codes >> 24), xv.w, a);
    }
    if (BLOCKS % 64 == 0 || lane + 64 * s < BLOCKS) acc = fmaf(half_bits_to_float(head[s]), a - kBias * sxl[b], acc);
  }
  const float v = wave_sum(acc);
  if (lane == 0) store_out<OutT>(out, (size_t)row, v);
}

template <int TYPE, int KB, typename OutT>
static void launch_q32_m1_f32_blocks(const GemvArgs& a, hipStream_t stream) {
  constexpr int WAVES = KB <= 128 ? 8 : 4;
  hipLaunchKernelGGL((gemv_q32_m1_f32<TYPE, WAVES, KB, OutT>), dim3((a.n + WAVES - 1) / WAVES), dim3(WAVES * 64),
                     0, stream, static_cast<const float*>(a.x), static_cast<const uint8_t*>(a.w),
                     static_cast<OutT*>(a.out), a.n);
}

template <int TYPE, typename OutT>
static bool launch_q32_m1_f32(const GemvArgs& a, hipStream_t stream) {
  if (a.m != 1) return false;
  if (a.k == 1024) {
    launch_q32_m1_f32_blocks<TYPE, 32, OutT>(a, stream);
    return true;
  }
  if (a.k % 2048) return false;
  switch (a.k / 2048) {
    case 1: launch_q32_m1_f32_blocks<TYPE, 64, OutT>(a, stream); return true;
    case 2: launch_q32_m1_f32_blocks<TYPE, 128, OutT>(a, stream); return true;
    case 3: launch_q32_m1_f32_blocks<TYPE, 192, OutT>(a, stream); return true;
    case 4: launch_q32_m1_f32_blocks<TYPE, 256, OutT>(a, stream); return true;
    case 5: launch_q32_m1_f32_blocks<TYPE, 320, OutT>(a, stream); return true;
    case 6: launch_q32_m1_f32_blocks<TYPE, 384, OutT>(a, stream); return true;
    case 7: launch_q32_m1_f32_blocks<TYPE, 448, OutT>(a, stream); return true;
    case 8: launch_q32_m1_f32_blocks<TYPE, 512, OutT>(a, stream); return true;
    default: return false;
  }
}

// ------------------------------------------------------ other encodings ---
// Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K: each lane decodes 16-element groups with the
// dequantizer's arithmetic (decode8, twice) and accumulates their products with the
// activations in fp32.  Consecutive lanes take consecutive groups, so one wave
// pass covers 1024 consecutive elements of its rows; the activation group is
// loaded once and reused for all R rows.
//
// XT = float takes fp32 activations (the packed call form at M = 1): each product is then
// the fp32 activation times the fp32 decoded weight, the reference's decode numerics
// (benchmarks/kernels/showcase/benchmark.py:466-472), for every encoding.
template <typename XT>
__device__ __forceinline__ void load_x16(const XT* p, float v[16]) {
  if constexpr (sizeof(XT) == 4) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 raw = load16(reinterpret_cast<const uint8_t*>(p + 4 * q));
#pragma unroll
      for (int i = 0; i < 4; ++i) v[4 * q + i] = __builtin_bit_cast(float, word(raw, i));
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint4 raw = load16(reinterpret_cast<const uint8_t*>(p + 8 * h));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half2_t pair = as_half2(word(raw, i));
        v[8 * h + 2 * i] = (float)pair.x;
        v[8 * h + 2 * i + 1] = (float)pair.y;
      }
    }
  }
}

template <int TYPE, int M, int R, typename OutT, bool SWIGLU = false, typename XT = _Float16>
__global__ __launch_bounds__(256) void gemv_blocks(const XT* __restrict__ x,
                                                   const uint8_t* __restrict__ w,
                                                   OutT* __restrict__ out, int n_rows, int k,
                                                   const uint8_t* __restrict__ w2 = nullptr) {
  constexpr int QK = Block<TYPE>::QK, BYTES = Block<TYPE>::BYTES;
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * (SWIGLU ? 1 : R);
  if (row0 >= n_rows) return;
  const size_t row_bytes = (size_t)(k / QK) * BYTES;
  const int rows = SWIGLU ? R : min(R, n_rows - row0);
  float acc[M][R];
#pragma unroll
  for (int m = 0; m < M; ++m)
#pragma unroll
    for (int r = 0; r < R; ++r) acc[m][r] = 0.0f;

  // 16 elements per lane and pass: one scale group of Q2_K / Q3_K, half a 32-element block
  // (the two decode8 calls share the block's header loads).  Q3_K at M=1 is not unrolled: at
  // 64 VGPRs it keeps 8 waves per SIMD (65 and 7 waves unrolled), 22.1 against 25.1 us at
  // 12288x4096.
  constexpr int UNROLL = (M == 1 && TYPE == kQ3_K) ? 1 : 2;
#pragma unroll UNROLL
  for (int g = lane; g < (k >> 4); g += 64) {
    const int e = 16 * g;
    float xv[M][16];
#pragma unroll
    for (int m = 0; m < M; ++m) load_x16<XT>(x + (size_t)m * k + e, xv[m]);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r >= rows) break;
      const uint8_t* block = pair_row<SWIGLU>(w, w2, row0, r, row_bytes) + (size_t)(e / QK) * BYTES;
      float v[16];
      decode8<TYPE>(block, e % QK, v);
      decode8<TYPE>(block, e % QK + 8, v + 8);
#pragma unroll
      for (int m = 0; m < M; ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[m][r] = fmaf(v[i], xv[m][i], acc[m][r]);
    }
  }
  store_rows<SWIGLU>(acc, out, n_rows, row0, rows, lane);
}

// Every encoding without a dedicated kernel goes to gemv_blocks: one row per wave (the gate /
// up pair for SWIGLU), so that many waves hide the latency of the per-group decoder's loads.
template <int M, typename OutT, bool SWIGLU>
static bool launch_blocks(const GemvArgs& a, const uint8_t* w2, hipStream_t stream) {
  constexpr int R = SWIGLU ? 2 : 1;
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const dim3 grid((a.n + 3) / 4);
  switch (a.type) {
#define TENSOR_GGUF_BLOCKS(T)                                                                                  \
  case T:                                                                                                      \
    hipLaunchKernelGGL((gemv_blocks<T, M, R, OutT, SWIGLU>), grid, dim3(256), 0, stream, x, w, out, a.n, a.k, w2); \
    return true;
    TENSOR_GGUF_BLOCKS(kQ4_1)
    TENSOR_GGUF_BLOCKS(kQ5_0)
    TENSOR_GGUF_BLOCKS(kQ5_1)
    TENSOR_GGUF_BLOCKS(kQ2_K)
    TENSOR_GGUF_BLOCKS(kQ3_K)
    TENSOR_GGUF_BLOCKS(kQ5_K)
#undef TENSOR_GGUF_BLOCKS
    default:
      return false;
  }
}

// fp32 activations at M = 1 (the packed call form), every encoding: gemv_blocks with the
// shared per-element decoder, one row per wave.
template <typename OutT>
static hipError_t launch_f32x(const GemvArgs& a, hipStream_t stream) {
  const float* x = static_cast<const float*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const dim3 grid((a.n + 3) / 4);
  switch (a.type) {
#define TENSOR_GGUF_F32X(T)                                                                                   \
  case T:                                                                                                     \
    hipLaunchKernelGGL((gemv_blocks<T, 1, 1, OutT, false, float>), grid, dim3(256), 0, stream, x, w, out, a.n, \
                       a.k, nullptr);                                                                         \
    break;
    TENSOR_GGUF_F32X(kQ4_0)
    TENSOR_GGUF_F32X(kQ4_1)
    TENSOR_GGUF_F32X(kQ5_0)
    TENSOR_GGUF_F32X(kQ5_1)
    TENSOR_GGUF_F32X(kQ8_0)
    TENSOR_GGUF_F32X(kQ2_K)
    TENSOR_GGUF_F32X(kQ3_K)
    TENSOR_GGUF_F32X(kQ4_K)
    TENSOR_GGUF_F32X(kQ5_K)
    TENSOR_GGUF_F32X(kQ6_K)
#undef TENSOR_GGUF_F32X
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemv_f32x(const GemvArgs& a, hipStream_t stream) {
  if (a.m != 1) return hipErrorInvalidValue;
  bool handled = false;
  hipError_t status = launch_gemv_q4k_f32x(a, stream, &handled);
  if (handled) return status;
  status = launch_gemv_q6k_f32x(a, stream, &handled);
  if (handled) return status;
  if (a.type == kQ8_0 || a.type == kQ4_0) {
    const bool q8 = a.type == kQ8_0;
    if (a.out_half ? (q8 ? launch_q32_m1_f32<kQ8_0, _Float16>(a, stream) : launch_q32_m1_f32<kQ4_0, _Float16>(a, stream))
                   : (q8 ? launch_q32_m1_f32<kQ8_0, float>(a, stream) : launch_q32_m1_f32<kQ4_0, float>(a, stream)))
      return hipGetLastError();
  }
  return a.out_half ? launch_f32x<_Float16>(a, stream) : launch_f32x<float>(a, stream);
}

// --------------------------------------------------------------- launch ---

template <int M, typename OutT>
static hipError_t launch_m(const GemvArgs& a, hipStream_t stream) {
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  constexpr int R = M <= 2 ? 4 : (M <= 4 ? 2 : 1);
  const int waves = (a.n + R - 1) / R;
  const dim3 grid((waves + 3) / 4), block(256);
  // Q8_0 / Q4_0: x in LDS when it takes at most 64 KB, shared by the workgroup's waves, and one
  // row per wave (rows per wave only served the reuse of x loaded from global memory)
  const size_t xbytes = (size_t)M * a.k * 2;
  const bool xlds = xbytes <= 64 * 1024;
  const dim3 grid1((a.n + 3) / 4);
  switch (a.type) {
    case kQ4_K:
      hipLaunchKernelGGL((gemv_q4k<M, R, OutT>), grid, block, 0, stream, x, w, out, a.n, a.k);
      break;
    case kQ6_K:
      hipLaunchKernelGGL((gemv_q6k<M, R, OutT>), grid, block, 0, stream, x, w, out, a.n, a.k);
      break;
    case kQ8_0:
      if (launch_q32_m1<kQ8_0, OutT>(a, stream)) break;
      if (xlds) hipLaunchKernelGGL((gemv_q32<kQ8_0, M, 1, OutT, false, true>), grid1, block, xbytes, stream, x, w, out, a.n, a.k);
      else hipLaunchKernelGGL((gemv_q32<kQ8_0, M, R, OutT>), grid, block, 0, stream, x, w, out, a.n, a.k);
      break;
    case kQ4_0:
      if (launch_q32_m1<kQ4_0, OutT>(a, stream)) break;
      if (xlds) hipLaunchKernelGGL((gemv_q32<kQ4_0, M, 1, OutT, false, true>), grid1, block, xbytes, stream, x, w, out, a.n, a.k);
      else hipLaunchKernelGGL((gemv_q32<kQ4_0, M, R, OutT>), grid, block, 0, stream, x, w, out, a.n, a.k);
      break;
    default:
      if constexpr (M == 1) {
        if (launch_q5_m1<OutT>(a, stream)) break;
      }
      if (!launch_blocks<M, OutT, false>(a, nullptr, stream)) return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename OutT>
static hipError_t launch_out(const GemvArgs& a, hipStream_t stream) {
  switch (a.m) {
    case 1: return launch_m<1, OutT>(a, stream);
    case 2: return launch_m<2, OutT>(a, stream);
    case 3: return launch_m<3, OutT>(a, stream);
    case 4: return launch_m<4, OutT>(a, stream);
    case 5: return launch_m<5, OutT>(a, stream);
    case 6: return launch_m<6, OutT>(a, stream);
    case 7: return launch_m<7, OutT>(a, stream);
    case 8: return launch_m<8, OutT>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

// SwiGLU pairs on the generic kernels: one output row per wave, R = 2 (gate row, up row).
template <int M, typename OutT>
static hipError_t launch_swiglu_m(const GemvArgs& a, const uint8_t* w_up, hipStream_t stream) {
  const _Float16* x = static_cast<const _Float16*>(a.x);
  const uint8_t* w = static_cast<const uint8_t*>(a.w);
  OutT* out = static_cast<OutT*>(a.out);
  const dim3 grid((a.n + 3) / 4), block(256);
  switch (a.type) {
    case kQ4_K:
      hipLaunchKernelGGL((gemv_q4k<M, 2, OutT, true>), grid, block, 0, stream, x, w, out, a.n, a.k, w_up);
      break;
    case kQ6_K:
      hipLaunchKernelGGL((gemv_q6k<M, 2, OutT, true>), grid, block, 0, stream, x, w, out, a.n, a.k, w_up);
      break;
    case kQ8_0:
      hipLaunchKernelGGL((gemv_q32<kQ8_0, M, 2, OutT, true>), grid, block, 0, stream, x, w, out, a.n, a.k, w_up);
      break;
    case kQ4_0:
      hipLaunchKernelGGL((gemv_q32<kQ4_0, M, 2, OutT, true>), grid, block, 0, stream, x, w, out, a.n, a.k, w_up);
      break;
    default:
      if (!launch_blocks<M, OutT, true>(a, w_up, stream)) return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename OutT>
static hipError_t launch_swiglu_out(const GemvArgs& a, const uint8_t* w_up, hipStream_t stream) {
  switch (a.m) {
    case 1: return launch_swiglu_m<1, OutT>(a, w_up, stream);
    case 2: return launch_swiglu_m<2, OutT>(a, w_up, stream);
    case 3: return launch_swiglu_m<3, OutT>(a, w_up, stream);
    case 4: return launch_swiglu_m<4, OutT>(a, w_up, stream);
    case 5: return launch_swiglu_m<5, OutT>(a, w_up, stream);
    case 6: return launch_swiglu_m<6, OutT>(a, w_up, stream);
    case 7: return launch_swiglu_m<7, OutT>(a, w_up, stream);
    case 8: return launch_swiglu_m<8, OutT>(a, w_up, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv_swiglu(const GemvArgs& a, const void* w_up, hipStream_t stream) {
  if (a.type == kQ4_K || a.type == kQ5_K) {
    bool handled = false;
    const hipError_t status = launch_gemv_q4k_swiglu_fast(a, w_up, stream, &handled);
    if (handled) return status;
  }
  const uint8_t* up = static_cast<const uint8_t*>(w_up);
  return a.out_half ? launch_swiglu_out<_Float16>(a, up, stream) : launch_swiglu_out<float>(a, up, stream);
}

hipError_t launch_gemv(const GemvArgs& a, hipStream_t stream) {
  if (a.type == kQ4_K || a.type == kQ5_K || a.type == kQ6_K) {
    bool handled = false;
    const hipError_t status = a.type == kQ4_K   ? launch_gemv_q4k_fast(a, stream, &handled)
                              : a.type == kQ5_K ? launch_gemv_q5k_fast(a, stream, &handled)
                                                : launch_gemv_q6k_fast(a, stream, &handled);
    if (handled) return status;
  }
  if (a.type == kQ2_K || a.type == kQ3_K) {
    bool handled = false;
    const hipError_t status = launch_gemv_q23k_fast(a, stream, &handled);
    if (handled) return status;
  }
  return a.out_half ? launch_out<_Float16>(a, stream) : launch_out<float>(a, stream);
}

}  // namespace tensor_gguf
