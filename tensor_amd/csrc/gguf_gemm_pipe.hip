// Pipelined fused dequant-GEMM for Q4_K, Q5_K, Q6_K, Q8_0 and Q4_0 on gfx950:
// out[m, n] = sum_k fp16(x[m, k]) * fp16(W[n, k]), fp32 accumulation
// (reference kernel: AKAS _packed, benchmarks/kernels/showcase/kernels.py:114-119;
//  Triton restatement triton_kernels.py:185-211).
//
// Same tile algorithm as the generic kernel in gguf_gemm.hip (BM x BN
// workgroup tile, BK = 64 steps, LDS-staged fp16 tiles, 16x16x32 fp16 MFMA
// with fp32 accumulators) with a deeper software pipeline:
//
//   * two register sets of raw bytes: step s+1 is dequantized into LDS while
//     step s+2 is in flight from HBM and step s is multiplied (a four-set ring
//     measured no faster: the steps are not bound by load latency);
//   * the LDS double buffer as two arrays, so the compiler may overlap the
//     staging stores of one buffer with the fragment reads of the other;
//   * each step is one straight-line region in which sched_group_barrier
//     interleaves every MFMA with dequant VALU work, an LDS store or a global
//     load, keeping the matrix pipe fed while the VALU decodes;
//   * XDMA (the 256 x 192 tile): the activation tile goes from global memory
//     straight to LDS (global_load_lds_dwordx4, three swizzled buffers), which
//     frees the staging registers the wider tile needs; half of its waves issue
//     a step's MFMAs before their dequant and half after, so the two waves of a
//     SIMD overlap matrix and vector work (ping-pong);
//   * Q4_K / Q5_K with four (two) threads per weight row: the lanes of a row, a
//     DPP quad (pair), each decode one (two) of the step's four scale factors
//     and share them by broadcasts, instead of each decoding all four.
//
// Weights are dequantized with the reference's fp32 arithmetic (every product
// exact, one rounding) and converted to fp16 with round-to-nearest-even, so
// the staged tiles are bit-exact fp16(dequant(W)).
//   Q4_K (triton_kernels.py:143-162): a step is one 32-byte quant pair j of a
//     super-block, 64 codes: low nibbles = sub-block 2j, high = 2j+1.
//   Q6_K (triton_kernels.py:163-180): a step covers quarters 2(s%2), 2(s%2)+1
//     of half h = (s%4)/2: the 64 low-nibble bytes of ql for that half (nibble
//     s%2), the 32 qh bytes of the half (2 bits per quarter) and 4 scales.
//   Q8_0 / Q4_0 (triton_kernels.py:135-142 for Q4_0): a step is two whole
//     32-element blocks, d * q and (q - 8) * d.
#include <algorithm>

#include "gguf_common.h"
#include "gguf_launch.h"

namespace tensor_gguf {
namespace pipe {

constexpr int BK = 64, ROW = 80;  // halves per LDS row (16-byte aligned, padded)
constexpr float kTwo24 = 16777216.0f, kTwo20 = 1048576.0f;

__device__ __forceinline__ uint32_t pack2(float a, float b) {
  const _Float16 ha = (_Float16)a, hb = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// fp16(scale * q + bias) for four codes q < 1024 given as fp16 subnormal pairs
// p02 = (q0, q2) * 2^-24 and p13 = (q1, q3) * 2^-24 (a code masked into the low
// bits of a half is that subnormal exactly). With scale24 = scale * 2^24 each
// product is exactly scale * q and the fma rounds once to fp32 as fmaf(scale, q,
// bias) does (one fp32-result v_fma_mix per element); each pair is then rounded to
// fp16 by one packed conversion, so the fp16 weight is the cast of the fp32 value.
__device__ __forceinline__ uint2 affine4(uint32_t p02, uint32_t p13, float scale24, float bias) {
  const half2_t a = as_half2(p02), b = as_half2(p13);
  return make_uint2(half2_from_fp32(fmaf((float)a[0], scale24, bias), fmaf((float)b[0], scale24, bias)),
                    half2_from_fp32(fmaf((float)a[1], scale24, bias), fmaf((float)b[1], scale24, bias)));
}

template <int TYPE, int TPR>
struct Geometry;

// Q4_K: TPR threads per weight row share the 32 quant bytes of the step's pair.
template <int TPR>
struct Geometry<kQ4_K, TPR> {
  static constexpr int QB = 32 / TPR;  // quant bytes per thread
  static constexpr int W0 = QB / 4, W1 = 4;  // dwords: quants, header
};

// Q5_K: Q4_K's slices plus the fifth-bit bytes at the same positions of the 32-byte qh run.
template <int TPR>
struct Geometry<kQ5_K, TPR> {
  static constexpr int QB = 32 / TPR;
  static constexpr int W0 = QB / 4, W1 = 4 + QB / 4;  // dwords: quants; header, then fifth bits
};

// Q6_K: TPR threads per weight row, each EPT = 64 / TPR consecutive elements.
template <int TPR>
struct Geometry<kQ6_K, TPR> {
  static constexpr int EPT = 64 / TPR;
  static constexpr int W0 = EPT / 4, W1 = EPT / 4 + 2;  // ql dwords; qh dwords + scales + d
};

// Q8_0 / Q4_0: a step is two 32-element blocks (68 / 36 bytes).  TPR threads per weight row
// share the step's quant bytes (64 / 32): thread p takes QB of them, all in block
// QB p / QPB at byte QB p % QPB (QPB = quant bytes per block), and that block's fp16 d.
template <int TPR>
struct Geometry<kQ8_0, TPR> {
  static constexpr int QPB = 32, QB = 2 * QPB / TPR;
  static constexpr int W0 = QB / 4, W1 = 2;  // dwords: quants; d (low half), unused
};
template <int TPR>
struct Geometry<kQ4_0, TPR> {
  static constexpr int QPB = 16, QB = 2 * QPB / TPR;
  static constexpr int W0 = QB / 4, W1 = 2;
};

// Raw bytes of one step in vector registers (vector values stay in VGPRs; arrays of
// several sets were demoted to the stack). x: XL 16-byte activation chunks; a / b: the
// quant and header dwords of each of the thread's P weight parts.
template <int XL, int W0, int W1, int P>
struct Raw {
  typedef uint32_t XV __attribute__((ext_vector_type(4 * XL)));
  typedef uint32_t AV __attribute__((ext_vector_type(W0)));
  typedef uint32_t BV __attribute__((ext_vector_type(W1)));
  XV x;
  AV a[P];
  BV b[P];
};

}  // namespace pipe

// KS groups of WM x WN waves split K: group g takes steps [g S, g S + S), S = steps / KS,
// with its own LDS staging buffers; the KS partial tiles are summed in LDS at the end
// (KS = 1: the whole K range in one group).
//
// One launch covers the matrices of a GemmJob (they share x and K): blockIdx.x runs over the
// BN-wide column tiles of all of them in order.  With job.splits > 1, blockIdx.z also splits
// K across workgroups: workgroup z takes its split's range of steps and stores its fp32
// partial tile to job.partial, and gemm_reduce adds the splits in order.
//
// XT = float: fp32 activations (the packed call form), rounded to fp16 as they are loaded, so
// the staged tile is fp16(x) as in the reference's prefill numerics (benchmark.py:473-477).
template <int TYPE, int BM, int BN, int WM, int WN, int KS, typename OutT, typename XT = _Float16, bool XDMA = false>
__global__ __launch_bounds__(WM * WN * 64 * KS) void gemm_pipe(const XT* __restrict__ x, const GemmJob job,
                                                               int M, int K) {
  using namespace pipe;
  constexpr int THREADS = WM * WN * 64;  // per K group
  constexpr int MT = BM / WM / 16, NT = BN / WN / 16;
  constexpr int XL = XDMA ? 1 : BM * 8 / THREADS;  // 16-byte activation chunks per thread per step
  static_assert(!XDMA || (KS == 1 && sizeof(XT) == 2), "x by LDS DMA: fp16 x, one K group");
  constexpr int XS = BM * BK;                  // halves per DMA'd x buffer (128-byte rows, swizzled)
  constexpr int XPW = BM * BK * 2 / 1024 / (WM * WN);  // 1 KB DMA blocks per wave per step
  // TPR parts per weight row (a part: the row's step bytes one thread decodes).  Where BN
  // divides the threads, every thread takes one part of one row; otherwise (BN = 96, 192)
  // rows take 4 parts and thread t the parts t, t + THREADS, ... below BN * 4, so a wave
  // either has a part at a given index or has none (the test is wave-uniform).
  constexpr int TPR = THREADS % BN == 0 ? THREADS / BN : 4;
  constexpr int PARTS = (BN * TPR + THREADS - 1) / THREADS;
  static_assert((XDMA || XL * THREADS == BM * 8) && (TPR == 1 || TPR == 2 || TPR == 4) && PARTS <= 2 &&
                    (BN * TPR) % 64 == 0, "tile shape");
  using G = Geometry<TYPE, TPR>;
  using RawT = Raw<XL, G::W0, G::W1, PARTS>;
  constexpr int QK = Block<TYPE>::QK, BYTES = Block<TYPE>::BYTES;
  constexpr bool KQ = TYPE == kQ4_K || TYPE == kQ5_K;  // Q4_K's header and nibble layout
  constexpr bool B32 = TYPE == kQ8_0 || TYPE == kQ4_0;  // 32-element blocks, two per step
  constexpr int STAGE = XDMA ? 3 * XS + 2 * BN * ROW : 2 * (BM + BN) * ROW;  // halves of one group's tiles
  __shared__ __attribute__((aligned(1024))) _Float16 stage[KS * STAGE];
  // wave-uniform (THREADS is a multiple of 64): keeps the step counter and the
  // addressing derived from it in scalar registers
  const int group = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x / THREADS);
  _Float16* const xs0 = stage + group * STAGE;
  _Float16* const xs1 = xs0 + (XDMA ? XS : BM * ROW);
  _Float16* const ws0 = XDMA ? xs0 + 3 * XS : xs1 + BM * ROW;
  _Float16* const ws1 = ws0 + BN * ROW;

  // the wave index in a scalar register: the wave's tile offsets then take no vector registers
  const int tid = threadIdx.x % THREADS, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave / WN) * (16 * MT), wn = (wave % WN) * (16 * NT);
  // the matrix of this column tile (workgroup-uniform)
  const int tile = blockIdx.x;
  const int mi = tile < job.tile_end[0] ? 0 : tile < job.tile_end[1] ? 1 : 2;
  const int N = job.n[mi];
  const int m0 = blockIdx.y * BM, n0 = (tile - (mi ? job.tile_end[mi - 1] : 0)) * BN;
  int wrow[PARTS], wpart[PARTS];
  bool has[PARTS];
  // weight rows as 32-bit byte offsets from the matrix base (matrices stay under 4 GiB)
  const uint8_t* const wmat = job.w[mi];
  uint32_t wbase[PARTS];
#pragma unroll
  for (int p = 0; p < PARTS; ++p) {
    const int part = tid + p * THREADS;
    has[p] = part < BN * TPR;
    wrow[p] = has[p] ? part / TPR : 0;
    wpart[p] = part % TPR;
    wbase[p] = (uint32_t)min(n0 + wrow[p], N - 1) * (uint32_t)((K / QK) * BYTES);
  }
  // this group's steps of this split; the host guarantees that every group takes an even number
  // of steps and (for the 256-element encodings) starts on a super-block
  const int split_steps = K / BK / job.splits;
  const int steps = split_steps / KS, first = blockIdx.z * split_steps + group * steps;

  // XDMA: DMA source rows of this lane.  Block b = XPW wave + i of the x tile (1 KB, 8 rows of
  // 128 B) goes to LDS lane-linear: lane l writes 16 B at 16 l, row 8 b + l / 8, slot l % 8, which
  // holds chunk (l % 8) ^ ((row >> 1) & 7) of the row, so a 16-row fragment read hits 16 bank groups
  // as 32-bit byte offsets from the tile's first row (M * K * 2 stays under 4 GiB)
  const uint8_t* const xtile = reinterpret_cast<const uint8_t*>(x + (size_t)m0 * K);
  uint32_t xsrc[XDMA ? XPW : 1];
  if constexpr (XDMA) {
#pragma unroll
    for (int i = 0; i < XPW; ++i) {
      const int r = 8 * (XPW * wave + i) + (lane >> 3);
      const int cch = (lane & 7) ^ ((r >> 1) & 7);
      xsrc[i] = 2u * ((uint32_t)(min(m0 + r, M - 1) - m0) * (uint32_t)K + 8 * cch);
    }
  }
  auto dma = [&](int step, _Float16* xbuf) {
    if constexpr (XDMA) {
#pragma unroll
      for (int i = 0; i < XPW; ++i)
        __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(xtile + (xsrc[i] + (uint32_t)(2 * step * BK))),
                                         (void __attribute__((address_space(3)))*)(xbuf + (XPW * wave + i) * 512),
                                         16, 0, 0);
    }
  };
  auto load = [&](RawT& r, int step) {
    const int k0 = step * BK;
#pragma unroll
    for (int i = 0; i < (XDMA ? 0 : XL); ++i) {
      const int c = i * THREADS + tid, row = c >> 3, c8 = (c & 7) * 8;
      // rows past M reload row M - 1: their products land in output rows that are never stored
      const XT* src = x + (size_t)min(m0 + row, M - 1) * K + k0 + c8;
      if constexpr (sizeof(XT) == 4) {
        const uint4 lo = load16(reinterpret_cast<const uint8_t*>(src));
        const uint4 hi = load16(reinterpret_cast<const uint8_t*>(src + 4));
        r.x[4 * i] = half2_from_fp32(__builtin_bit_cast(float, lo.x), __builtin_bit_cast(float, lo.y));
        r.x[4 * i + 1] = half2_from_fp32(__builtin_bit_cast(float, lo.z), __builtin_bit_cast(float, lo.w));
        r.x[4 * i + 2] = half2_from_fp32(__builtin_bit_cast(float, hi.x), __builtin_bit_cast(float, hi.y));
        r.x[4 * i + 3] = half2_from_fp32(__builtin_bit_cast(float, hi.z), __builtin_bit_cast(float, hi.w));
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        r.x[4 * i] = v.x; r.x[4 * i + 1] = v.y; r.x[4 * i + 2] = v.z; r.x[4 * i + 3] = v.w;
      }
    }
#pragma unroll
    for (int p = 0; p < PARTS; ++p) {
      if (!has[p]) continue;
      const uint8_t* blk = wmat + (wbase[p] + (uint32_t)((k0 / QK) * BYTES));
      typename RawT::AV& ra = r.a[p];
      typename RawT::BV& rb = r.b[p];
      if constexpr (B32) {
        constexpr int QPB = G::QPB, QB = G::QB;
        const uint8_t* b = blk + (QB * wpart[p] / QPB) * BYTES;  // this part's block: fp16 d, quants
        const uint8_t* q = b + 2 + QB * wpart[p] % QPB;
        if constexpr (G::W0 % 4 == 0) {
#pragma unroll
          for (int i = 0; i < G::W0; i += 4) {
            const uint4 v = load16(q + 4 * i);
            ra[i] = v.x; ra[i + 1] = v.y; ra[i + 2] = v.z; ra[i + 3] = v.w;
          }
        } else {
          const uint2 v = load8(q);
          ra[0] = v.x; ra[1] = v.y;
        }
        rb[0] = load4(b);
        rb[1] = 0;
      } else if constexpr (KQ) {
        const uint4 hd = load16(blk);
        rb[0] = hd.x; rb[1] = hd.y; rb[2] = hd.z; rb[3] = hd.w;
        const uint8_t* q = blk + (TYPE == kQ5_K ? 48 : 16) + 32 * (step & 3) + G::QB * wpart[p];
#pragma unroll
        for (int i = 0; i < G::W0; ++i) ra[i] = load4(q + 4 * i);
        if constexpr (TYPE == kQ5_K) {
#pragma unroll
          for (int i = 0; i < G::W0; ++i) rb[4 + i] = load4(blk + 16 + G::QB * wpart[p] + 4 * i);
        }
      } else {
        const int h = (step & 3) >> 1, e0 = G::EPT * wpart[p];  // element offset inside the step
        const int quarter = 2 * (step & 1) + (e0 >> 5), l0 = e0 & 31;
        const uint8_t* ql = blk + 64 * h + e0;
        const uint8_t* qh = blk + 128 + 32 * h + l0;
#pragma unroll
        for (int i = 0; i < G::W0; ++i) {
          ra[i] = load4(ql + 4 * i);
          rb[i] = load4(qh + 4 * i);
        }
        rb[G::W0] = load4(blk + 192 + 8 * h + 2 * quarter);  // scales 2q .. 2q+3 of this half
        rb[G::W0 + 1] = load4(blk + 206);                    // high half: d
      }
    }
  };

  auto store = [&](const RawT& r, _Float16* xs, _Float16* ws, int step) {
#pragma unroll
    for (int i = 0; i < (XDMA ? 0 : XL); ++i) {
      const int c = i * THREADS + tid, row = c >> 3, c8 = (c & 7) * 8;
      *reinterpret_cast<uint4*>(&xs[row * ROW + c8]) = make_uint4(r.x[4 * i], r.x[4 * i + 1], r.x[4 * i + 2], r.x[4 * i + 3]);
    }
#pragma unroll
    for (int p = 0; p < PARTS; ++p) {
      if (!has[p]) continue;
      const typename RawT::AV& ra = r.a[p];
      const typename RawT::BV& rb = r.b[p];
      if constexpr (B32) {
        constexpr int QPB = G::QPB, QB = G::QB;
        const float d = half_bits_to_float(rb[0]);
        // element e of block b (32 b + e in the step) sits at ws[wrow[p]][32 b + e]
        _Float16* dst = &ws[wrow[p] * ROW + 32 * (QB * wpart[p] / QPB) + QB * wpart[p] % QPB];
        if constexpr (TYPE == kQ8_0) {
          // d * q for the int8 code q, as the fp16 subnormal code q + 128 (byte ^ 0x80) times
          // d 2^24 plus -128 d: the product and the sum (q d) are exact, so is the fp32 value
          const float d24 = d * kTwo24, bias = -128.0f * d;
#pragma unroll
          for (int i = 0; i < G::W0; ++i) {
            const uint32_t u = ra[i] ^ 0x80808080u;
            *reinterpret_cast<uint2*>(dst + 4 * i) = affine4(u & 0x00FF00FFu, (u >> 8) & 0x00FF00FFu, d24, bias);
          }
        } else {
          // (q - 8) * d: byte j's low nibble is element j, its high nibble element j + 16 (left in
          // bits 4-7 of its half, 16 q * 2^-24, against d 2^20)
          const float d24 = d * kTwo24, d20 = d * kTwo20, bias = -8.0f * d;
#pragma unroll
          for (int i = 0; i < G::W0; ++i) {
            const uint32_t q = ra[i], q8 = q >> 8;
            *reinterpret_cast<uint2*>(dst + 4 * i) = affine4(q & 0x000F000Fu, q8 & 0x000F000Fu, d24, bias);
            *reinterpret_cast<uint2*>(dst + 16 + 4 * i) = affine4(q & 0x00F000F0u, q8 & 0x00F000F0u, d20, bias);
          }
        }
      } else if constexpr (KQ) {
        // d*sc*q - dmin*m: the product is exact, the subtraction rounds once; high nibbles stay in
        // bits 4-7 of their halves (16 q * 2^-24), so their scale takes 2^20
        float ds_lo, dm_lo, ds_hi, dm_hi;
        if constexpr (TPR == 4) {
          // the four lanes of a row (a DPP quad) each decode one of the step's four factors,
          // lane f: f & 2 picks sub-block 2j + 1, f & 1 the min, and share them by broadcasts
          const int f = lane & 3, jj = step & 3, t8 = 16 * (jj & 1) + 8 * (f >> 1);
          // the scale bytes (rb[1]) or the min bytes (rb[2]) by one byte permute
          const uint32_t word = __builtin_amdgcn_perm(rb[2], rb[1], f & 1 ? 0x07060504u : 0x03020100u);
          const uint32_t low6 = __builtin_amdgcn_ubfe(word, t8, 6);  // sub-blocks 0-3
          const uint32_t split = __builtin_amdgcn_ubfe(rb[3], t8 + 4 * (f & 1), 4) |
                                 (__builtin_amdgcn_ubfe(word, t8 + 6, 2) << 4);
          const uint32_t code = jj < 2 ? low6 : split;
          const float lane_scale = f & 1 ? -1.0f : (f & 2 ? kTwo20 : kTwo24);
          const float v = half_bits_to_float(rb[0] >> (16 * (f & 1))) * lane_scale * (float)code;
          const int vi = __builtin_bit_cast(int, v);
          ds_lo = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(vi, 0x00, 0xF, 0xF, false));
          dm_lo = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(vi, 0x55, 0xF, 0xF, false));
          ds_hi = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(vi, 0xAA, 0xF, 0xF, false));
          dm_hi = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(vi, 0xFF, 0xF, 0xF, false));
        } else if constexpr (TPR == 2) {
          // the two lanes of a row each decode the scale and min of one sub-block (lane f: 2j + f)
          // and take the other lane's by pair broadcasts within the DPP quad
          const int f = lane & 1, jj = step & 3, t8 = 16 * (jj & 1) + 8 * f;
          const uint32_t sc = jj < 2 ? __builtin_amdgcn_ubfe(rb[1], t8, 6)
                                     : __builtin_amdgcn_ubfe(rb[3], t8, 4) | (__builtin_amdgcn_ubfe(rb[1], t8 + 6, 2) << 4);
          const uint32_t mn = jj < 2 ? __builtin_amdgcn_ubfe(rb[2], t8, 6)
                                     : __builtin_amdgcn_ubfe(rb[3], t8 + 4, 4) | (__builtin_amdgcn_ubfe(rb[2], t8 + 6, 2) << 4);
          const float d = half_bits_to_float(rb[0]), dmin = half_bits_to_float(rb[0] >> 16);
          const int ds = __builtin_bit_cast(int, d * (f ? kTwo20 : kTwo24) * (float)sc);
          const int dm = __builtin_bit_cast(int, -(dmin * (float)mn));
          ds_lo = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(ds, 0xA0, 0xF, 0xF, false));  // lanes 0, 2
          dm_lo = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(dm, 0xA0, 0xF, 0xF, false));
          ds_hi = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(ds, 0xF5, 0xF, 0xF, false));  // lanes 1, 3
          dm_hi = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(dm, 0xF5, 0xF, 0xF, false));
        } else {
          int sc_lo, mn_lo, sc_hi, mn_hi;
          q4k_scale_pair(rb[1], rb[2], rb[3], step & 3, sc_lo, mn_lo, sc_hi, mn_hi);
          const float d = half_bits_to_float(rb[0]), dmin = half_bits_to_float(rb[0] >> 16);
          ds_lo = d * (float)sc_lo * kTwo24;
          dm_lo = -(dmin * (float)mn_lo);
          ds_hi = d * (float)sc_hi * kTwo20;
          dm_hi = -(dmin * (float)mn_hi);
        }
        _Float16* dst = &ws[wrow[p] * ROW + G::QB * wpart[p]];
#pragma unroll
        for (int i = 0; i < G::W0; ++i) {
          const uint32_t q = ra[i];  // low nibbles: sub-block 2j, high nibbles: 2j+1
          const uint32_t q8 = q >> 8;
          uint32_t lo02 = q & 0x000F000Fu, lo13 = q8 & 0x000F000Fu;
          uint32_t hi02 = q & 0x00F000F0u, hi13 = q8 & 0x00F000F0u;
          if constexpr (TYPE == kQ5_K) {
            // fifth bits: bit 2j (sub-block 2j) and 2j+1 of the qh byte at the quant byte's position
            const uint32_t h = rb[4 + i] >> (2 * (step & 3));
            lo02 |= (h & 0x00010001u) << 4;
            lo13 |= ((h >> 8) & 0x00010001u) << 4;
            hi02 |= ((h >> 1) & 0x00010001u) << 8;
            hi13 |= ((h >> 9) & 0x00010001u) << 8;
          }
          *reinterpret_cast<uint2*>(dst + 4 * i) = affine4(lo02, lo13, ds_lo, dm_lo);
          *reinterpret_cast<uint2*>(dst + 32 + 4 * i) = affine4(hi02, hi13, ds_hi, dm_hi);
        }
      } else {
        const int e0 = G::EPT * wpart[p];
        const int quarter = 2 * (step & 1) + (e0 >> 5), l0 = e0 & 31;
        const float d = half_bits_to_float(rb[G::W0 + 1] >> 16);
        _Float16* dst = &ws[wrow[p] * ROW + e0];
#pragma unroll
        for (int i = 0; i < G::W0; ++i) {
          // 6-bit codes of elements l0 + 4i .. + 3 of this quarter
          const uint32_t lo = (ra[i] >> (4 * (step & 1))) & 0x0F0F0F0Fu;
          const uint32_t hi = ((rb[i] >> (2 * quarter)) & 0x03030303u) << 4;
          const uint32_t q = lo | hi;
          // scale index 8h + 2 quarter + l / 16: byte l / 16 of the dword loaded at 2 quarter
          const float sc = (float)(int8_t)(rb[G::W0] >> (8 * ((l0 + 4 * i) >> 4)));
          // (q - 32) * sc * d == q * (sc d) - 32 (sc d): exact, one fused rounding
          const float scd = sc * d;
          *reinterpret_cast<uint2*>(dst + 4 * i) =
              affine4(q & 0x003F003Fu, (q >> 8) & 0x003F003Fu, scd * kTwo24, -32.0f * scd);
        }
      }
    }
  };

  float4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  // one K step: fragment reads of (xs, ws), then MFMAs interleaved with the
  // staging of `staged` into (xn, wnext) and the prefetch of `fetch_step`
  auto step_body = [&](const _Float16* xs, const _Float16* ws, _Float16* xn, _Float16* wnext, const RawT& staged,
                       int staged_step, RawT& fetched, int fetch_step, _Float16* xdma = nullptr) {
    half8_t a[2][MT], b[2][NT];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int koff = 32 * kk + 8 * (lane >> 4);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int row = wm + 16 * i + (lane & 15);
        if constexpr (XDMA)
          a[kk][i] = *reinterpret_cast<const half8_t*>(&xs[row * BK + 8 * ((4 * kk + (lane >> 4)) ^ ((row >> 1) & 7))]);
        else
          a[kk][i] = *reinterpret_cast<const half8_t*>(&xs[row * ROW + koff]);
      }
#pragma unroll
      for (int j = 0; j < NT; ++j)
        b[kk][j] = *reinterpret_cast<const half8_t*>(&ws[(wn + 16 * j + (lane & 15)) * ROW + koff]);
    }
    if constexpr (XDMA) {
      // the x DMA of the fetched step is issued ahead of its weight loads and the order is pinned:
      // loads complete in order, so once a wave's dequant has waited on those weights (the next
      // step's store), its DMA'd x has landed too, before the barrier that follows.
      // Ping-pong: the upper half of the waves (one weight part each) issue their MFMAs before
      // they dequantize, the lower half (two parts) after, so the two waves that share a SIMD
      // keep its matrix pipe and its VALU busy at the same time.
      auto mfma_all = [&]() {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[kk][i], b[kk][j], acc[i][j], 0, 0, 0);
      };
      const bool mfma_first = wave >= WM * WN / 2;
      if (mfma_first) {
        mfma_all();
        __builtin_amdgcn_sched_barrier(0);
      }
      store(staged, xn, wnext, staged_step);
      dma(fetch_step, xdma);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      load(fetched, fetch_step);
      if (!mfma_first) {
        __builtin_amdgcn_sched_barrier(0);
        mfma_all();
      }
      return;
    }
    store(staged, xn, wnext, staged_step);
    load(fetched, fetch_step);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[kk][i], b[kk][j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 2 * MT * NT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two VALU
      if (i % 4 == 0) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // an LDS store
      if (i % 4 == 2) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // a global load
    }
  };

  // two register sets of raw bytes: step s+1 is staged into LDS while step s+2 is fetched
  RawT ra, rb;
  const int last = first + steps - 1;
  if constexpr (XDMA) {
    // three x buffers: step s reads buffer s % 3 while the DMA of step s + 2 fills (s + 2) % 3;
    // the barrier between steps orders LDS only (this wave's DMA'd x of the next step has landed
    // by then), so the weight loads in flight stay in flight
    dma(first, xs0);
    asm volatile("" ::: "memory");
    dma(first + 1, xs1);
    asm volatile("" ::: "memory");
    load(ra, first);
    load(rb, first + 1);
    store(ra, xs0, ws0, first);
    __builtin_amdgcn_s_waitcnt(0);  // the first two x tiles have landed (every counter)
    __syncthreads();
    int cur = 0;
    for (int step = first; step < first + steps; step += 2) {
      const int c1 = cur == 2 ? 0 : cur + 1, c2 = c1 == 2 ? 0 : c1 + 1;
      step_body(xs0 + cur * XS, ws0, nullptr, ws1, rb, step + 1, ra, min(step + 2, last), xs0 + c2 * XS);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      const int c3 = c2 == 2 ? 0 : c2 + 1;
      step_body(xs0 + c1 * XS, ws1, nullptr, ws0, ra, min(step + 2, last), rb, min(step + 3, last), xs0 + c3 * XS);
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      cur = c2;
    }
  } else {
    load(ra, first);
    load(rb, first + 1);
    store(ra, xs0, ws0, first);
    __syncthreads();
    for (int step = first; step < first + steps; step += 2) {
      // the last step stages and fetches clamped copies that are never read
      step_body(xs0, ws0, xs1, ws1, rb, step + 1, ra, min(step + 2, last));
      __syncthreads();
      step_body(xs1, ws1, xs0, ws0, ra, min(step + 2, last), rb, min(step + 3, last));
      __syncthreads();
    }
  }
  if constexpr (KS > 1) {
    // partial tiles of groups 1 .. KS-1 -> LDS (over the staging buffers), summed by group 0
    float* red = reinterpret_cast<float*>(stage);
    static_assert((KS - 1) * MT * NT * 4 * THREADS * 4 <= KS * STAGE * 2, "reduction buffer");
    if (group > 0) {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) red[(((group - 1) * MT + i) * NT + j) * 4 * THREADS + e * THREADS + tid] = acc[i][j][e];
    }
    __syncthreads();
    if (group > 0) return;
#pragma unroll
    for (int g = 1; g < KS; ++g)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[i][j][e] += red[(((g - 1) * MT + i) * NT + j) * 4 * THREADS + e * THREADS + tid];
  }
  const bool split = job.splits > 1;
  OutT* const out = static_cast<OutT*>(job.out[mi]);
  float* const part = split ? job.partial + (size_t)blockIdx.z * M * job.n_total + job.col0[mi] : nullptr;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int col = n0 + wn + 16 * j + (lane & 15);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = m0 + wm + 16 * i + 4 * (lane >> 4) + e;
        if (row < M && col < N) {
          if (split) part[(size_t)row * job.n_total + col] = acc[i][j][e];
          else store_out<OutT>(out, (size_t)row * N + col, acc[i][j][e]);
        }
      }
    }
}

// out_i[row, c] = the sum of the splits' partial sums, added in split order (so the result does
// not depend on which workgroup finished first), converted once to the output type.
// A thread takes four consecutive columns of one row (blockIdx.y strides over the rows): one
// 16-byte load per split when the row width is a multiple of 4 (every row then starts
// 16-byte aligned in each split's plane), and one 4-wide store when the four columns fall in
// one matrix at a 4-aligned offset.
template <typename OutT>
__global__ __launch_bounds__(256) void gemm_reduce(const GemmJob job, int M) {
  const int n = job.n_total;
  const size_t plane = (size_t)M * n;
  const int c = 4 * (blockIdx.x * 256 + threadIdx.x);
  if (c >= n) return;
  const bool wide = (n & 3) == 0;
  for (int row = blockIdx.y; row < M; row += gridDim.y) {
    const float* p = job.partial + (size_t)row * n + c;
    float s[4];
    if (wide) {
      float4 v = *reinterpret_cast<const float4*>(p);
      for (int z = 1; z < job.splits; ++z) {
        const float4 u = *reinterpret_cast<const float4*>(p + z * plane);
        v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
      }
      s[0] = v.x; s[1] = v.y; s[2] = v.z; s[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[i] = 0.f;
        if (c + i < n) {
          s[i] = p[i];
          for (int z = 1; z < job.splits; ++z) s[i] += p[z * plane + i];
        }
      }
    }
    const int mi = job.count > 1 && c >= job.col0[1] ? (job.count > 2 && c >= job.col0[2] ? 2 : 1) : 0;
    const int local = c - job.col0[mi];
    OutT* out = static_cast<OutT*>(job.out[mi]) + (size_t)row * job.n[mi];
    if (wide && local + 4 <= job.n[mi] && ((job.n[mi] | local) & 3) == 0) {
      if constexpr (sizeof(OutT) == 2) {
        *reinterpret_cast<uint2*>(out + local) = make_uint2(half2_from_fp32(s[0], s[1]), half2_from_fp32(s[2], s[3]));
      } else {
        *reinterpret_cast<float4*>(out + local) = make_float4(s[0], s[1], s[2], s[3]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = c + i;
        if (col >= n) break;
        const int m = job.count > 1 && col >= job.col0[1] ? (job.count > 2 && col >= job.col0[2] ? 2 : 1) : 0;
        store_out<OutT>(static_cast<OutT*>(job.out[m]), (size_t)row * job.n[m] + (col - job.col0[m]), s[i]);
      }
    }
  }
}

namespace {

// Workgroup tiles of the pipelined GEMM, by index: 0..3 without a K split inside the workgroup,
// 4..7 with two or four wave groups per workgroup (LDS holds one double-buffered stage per
// group, so 128 x 128 and 128 x 64 take KS <= 2 and 64 x 64 KS <= 4), 8 the 256 x 96 tile (8
// waves of 64 x 48), 9 the 256 x 192 tile (8 waves of 64 x 96, x by LDS DMA).
struct Tile {
  int bm, bn, ks;
};
constexpr int kTileCount = 10;
constexpr Tile kTiles[kTileCount] = {{256, 128, 1}, {128, 128, 1}, {128, 64, 1}, {64, 64, 1}, {128, 128, 2},
                                     {128, 64, 2},  {64, 64, 2},   {64, 64, 4},  {256, 96, 1}, {256, 192, 1}};
constexpr int kDmaTile = 9;  // x tile by LDS DMA: fp16 x only

// The 256 x 192 tile's 8 waves of 64 x 96 fit the register file only without the activation
// staging registers (x by LDS DMA); with Q5_K's fifth bits or Q6_K's layout they still spill.
template <int TYPE, typename XT>
constexpr bool dma_tile_type() {
  return sizeof(XT) == 2 && (TYPE == kQ4_K || TYPE == kQ8_0 || TYPE == kQ4_0);
}

long tile_count(const GemmGroupArgs& a, const Tile& t) {
  long columns = 0;
  for (int i = 0; i < a.count; ++i) columns += (a.n[i] + t.bn - 1) / t.bn;
  return (long)((a.m + t.bm - 1) / t.bm) * columns;
}

int total_columns(const GemmGroupArgs& a) {
  int n = 0;
  for (int i = 0; i < a.count; ++i) n += a.n[i];
  return n;
}

// The job of one launch: per-matrix column tiles and partial-sum columns.
GemmJob make_job(const GemmGroupArgs& a, const Tile& t, int splits, void* workspace) {
  GemmJob job{};
  int tiles = 0, col = 0;
  for (int i = 0; i < kGemmGroupMax; ++i) {
    if (i < a.count) {
      job.w[i] = static_cast<const uint8_t*>(a.w[i]);
      job.out[i] = a.out[i];
      job.n[i] = a.n[i];
      tiles += (a.n[i] + t.bn - 1) / t.bn;
      job.col0[i] = col;
      col += a.n[i];
    } else {
      job.col0[i] = col;  // past the last matrix: never selected
    }
    job.tile_end[i] = tiles;
  }
  job.count = a.count;
  job.n_total = col;
  job.splits = splits;
  job.partial = static_cast<float*>(workspace);
  return job;
}

template <int TYPE, int BM, int BN, int WM, int WN, int KS, typename OutT, typename XT, bool XDMA = false>
hipError_t launch_pipe(const GemmGroupArgs& a, int splits, void* workspace, hipStream_t stream) {
  const GemmJob job = make_job(a, Tile{BM, BN, KS}, splits, workspace);
  const dim3 grid(job.tile_end[kGemmGroupMax - 1], (a.m + BM - 1) / BM, splits), block(WM * WN * 64 * KS);
  hipLaunchKernelGGL((gemm_pipe<TYPE, BM, BN, WM, WN, KS, OutT, XT, XDMA>), grid, block, 0, stream,
                     static_cast<const XT*>(a.x), job, a.m, a.k);
  if (splits > 1) {
    // four columns per thread across x; rows over y (strided past 65535 rows)
    const unsigned cols = (unsigned)((job.n_total + 1023) / 1024), rows = (unsigned)std::min(a.m, 65535);
    hipLaunchKernelGGL((gemm_reduce<OutT>), dim3(cols, rows), dim3(256), 0, stream, job, a.m);
  }
  return hipGetLastError();
}

template <int TYPE, typename OutT, typename XT>
hipError_t launch_tile(const GemmGroupArgs& a, int tile, int splits, void* workspace, hipStream_t stream) {
  switch (tile) {
    case 0: return launch_pipe<TYPE, 256, 128, 4, 2, 1, OutT, XT>(a, splits, workspace, stream);
    case 1: return launch_pipe<TYPE, 128, 128, 2, 2, 1, OutT, XT>(a, splits, workspace, stream);
    case 2: return launch_pipe<TYPE, 128, 64, 2, 2, 1, OutT, XT>(a, splits, workspace, stream);
    case 3: return launch_pipe<TYPE, 64, 64, 1, 2, 1, OutT, XT>(a, splits, workspace, stream);
    case 4: return launch_pipe<TYPE, 128, 128, 2, 2, 2, OutT, XT>(a, splits, workspace, stream);
    case 5: return launch_pipe<TYPE, 128, 64, 2, 2, 2, OutT, XT>(a, splits, workspace, stream);
    case 6: return launch_pipe<TYPE, 64, 64, 1, 2, 2, OutT, XT>(a, splits, workspace, stream);
    case 7: return launch_pipe<TYPE, 64, 64, 1, 2, 4, OutT, XT>(a, splits, workspace, stream);
    case 8: return launch_pipe<TYPE, 256, 96, 4, 2, 1, OutT, XT>(a, splits, workspace, stream);
    case kDmaTile:
      if constexpr (dma_tile_type<TYPE, XT>())
        return launch_pipe<TYPE, 256, 192, 4, 2, 1, OutT, XT, true>(a, splits, workspace, stream);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

template <int TYPE>
hipError_t launch_typed(const GemmGroupArgs& a, int tile, int splits, void* workspace, hipStream_t stream) {
  if (a.x_f32)
    return a.out_half ? launch_tile<TYPE, _Float16, float>(a, tile, splits, workspace, stream)
                      : launch_tile<TYPE, float, float>(a, tile, splits, workspace, stream);
  return a.out_half ? launch_tile<TYPE, _Float16, _Float16>(a, tile, splits, workspace, stream)
                    : launch_tile<TYPE, float, _Float16>(a, tile, splits, workspace, stream);
}

bool pipe_type(int type) {
  return type == kQ4_K || type == kQ5_K || type == kQ6_K || type == kQ8_0 || type == kQ4_0;
}

// The kernel addresses weights and the x tile by 32-bit offsets: every matrix stays under 4 GiB
// and a 256-row x tile under 2 GiB (K <= 2^22); larger shapes take the generic kernel.
bool offsets_fit(const GemmGroupArgs& a) {
  if (a.k > (1 << 22)) return false;
  const uint64_t row = a.type == kQ4_K ? (uint64_t)a.k / 256 * Block<kQ4_K>::BYTES
                       : a.type == kQ5_K ? (uint64_t)a.k / 256 * Block<kQ5_K>::BYTES
                       : a.type == kQ6_K ? (uint64_t)a.k / 256 * Block<kQ6_K>::BYTES
                       : a.type == kQ8_0 ? (uint64_t)a.k / 32 * Block<kQ8_0>::BYTES
                                         : (uint64_t)a.k / 32 * Block<kQ4_0>::BYTES;
  for (int i = 0; i < a.count; ++i)
    if ((uint64_t)a.n[i] * row >= (1ull << 32)) return false;
  return true;
}

// A tile and split count that fit the shape: K is whole 64-element steps, and the steps of a
// split divide evenly into the workgroup's wave groups, each taking an even number of them (the
// main loop runs two steps per pass) that starts on a super-block (4 steps) for the 256-element
// encodings.
// The LDS-DMA tile takes fp16 x and the encodings whose kernel fits the register file.
bool valid_plan(const GemmGroupArgs& a, int tile, int splits) {
  if (!offsets_fit(a)) return false;
  const int steps = a.k / pipe::BK, unit = a.type == kQ8_0 || a.type == kQ4_0 ? 2 : 4;
  if (tile == kDmaTile && (a.x_f32 || !(a.type == kQ4_K || a.type == kQ8_0 || a.type == kQ4_0))) return false;
  return tile >= 0 && tile < kTileCount && splits >= 1 && a.k % pipe::BK == 0 &&
         steps % (unit * kTiles[tile].ks * splits) == 0;
}

// Largest tile that still gives the 256 CUs work: the workgroup count of a tile must reach
// kMinBlocks, else a smaller tile is taken, and below 256 x 128 the K range is split over two
// or four wave groups of one workgroup so that every SIMD holds at least one wave (measured at
// M = 256: 1.4x to 4x faster than the unsplit tiles for the q/k/v/o, gate/up and down shapes).
constexpr long kMinBlocks = 160;

// A tile is taken only where M fills more than half its rows: 256-row tiles from M = 129,
// 128-row tiles from M = 65 (timing harness, Q4_K gate + up 2 x 12288 x 4096: M = 32 69.8 ->
// 39.8 us on 64 x 64 KS2, M = 128 72.3 -> 51.4 on 128 x 128 KS2; one 12288-row gate at M = 96 /
// 128 on 128 x 64 KS2 33.1 / 33.9 us; the Q6_K LM head at M = 32 414 -> 320 us).  At M <= 64
// the 64 x 64 tile splits K over 4 wave groups while its tiles stay within 256, else over 2.
//
// 256 x 96 against 256 x 128: per workgroup a 96-column step takes 0.84 of a 128-column one
// (timing harness, Q4_K M = 2048: 1.008 against 1.196 us per step), so the narrower tile wins
// where its extra workgroups still fit the rounds of the wider one: C4 at M = 512 and C5's gate
// + up at M = 256 (192 -> 256 workgroups, one round): 70.9 -> 64.9 us and 71.1 -> 64.6 us; Q6_K
// and Q8_0 at C4 M = 512 88.4 -> 79.9 and 79.2 -> 67.0 us; at M = 2048 (three rounds against
// four) the 128-column tile stays (229.7 against 257.4 us).
//
// 256 x 192 (x by LDS DMA, ping-pong waves) steps take 1.3 of a 256 x 128 step and 1.5 of a
// 256 x 96 one (Q4_K, timing harness: 1.50-1.54 against 1.12 and 0.97-0.99 us per step at
// M = 1024 / 2048) for 1.5 and 2 times their columns; it wins where it needs fewer rounds: C4 at
// M = 2048 214.7 (256 x 128) -> 192.6 us, M = 1024 124.6 (256 x 96) -> 98.3 us, and at M = 1536
// (two rounds, the second half full, against three of 256 x 96) 200.2 -> 185.6 us; at M = 512
// (half a round) it takes 84 us against 63 on 256 x 96.
int wide_tile(const GemmGroupArgs& a) {
  const auto rounds = [&](int tile) { return (tile_count(a, kTiles[tile]) + 255) / 256; };
  const long cost0 = rounds(0) * 119, cost8 = rounds(8) * 99;  // rounds x step time (10 ns)
  const long cost9 = valid_plan(a, kDmaTile, 1) ? rounds(kDmaTile) * 145 : cost0 + 1;
  if (cost9 < cost0 && cost9 < cost8) return kDmaTile;
  return rounds(8) * 84 < rounds(0) * 100 ? 8 : 0;
}

int base_tile(const GemmGroupArgs& a) {
  const int steps = a.k / pipe::BK;  // even (whole 32-element block pairs or super-blocks)
  const bool ks2 = steps % 8 == 0, ks4 = steps % 16 == 0;
  if (a.m > 128 && tile_count(a, kTiles[0]) >= kMinBlocks) return wide_tile(a);
  if (a.m > 64) {
    const long wide = tile_count(a, kTiles[1]);
    if (wide >= 512) return 1;
    if (wide >= kMinBlocks) return ks2 ? 4 : 1;
    if (a.m <= 128 && tile_count(a, kTiles[2]) >= kMinBlocks) return ks2 ? 5 : 2;
  }
  if (ks4 && (a.m > 64 || tile_count(a, kTiles[3]) < 256)) return 7;
  if (ks2) return 6;
  if (tile_count(a, kTiles[2]) >= kMinBlocks) return 2;
  return 3;
}

}  // namespace

GemmPlan plan_gemm_group(const GemmGroupArgs& a, size_t workspace_bytes) {
  GemmPlan plan{base_tile(a), 1};
  if (!pipe_type(a.type)) return plan;
  // M <= 64 with every N <= 4096 (where one matrix alone takes the small-M kernel): 64 x 64
  // tiles with K over four wave groups, split across workgroups while the grid stays within
  // 256 workgroups and each split keeps >= 16 steps; taken when that grid reaches 128
  // workgroups, else each matrix keeps its small-M launch.  Timing harness at M = 32: q + k + v
  // (4096, 1024, 1024) x 4096 Q4_K 41.2 -> 16.5 us with 2 splits, down 4096 x 12288 Q4_K 40.7 ->
  // 22.5 us with 4, Q6_K 44.3 -> 34.5, Q8_0 37.7 -> 30.9, o 4096 x 4096 15.0 -> 13.6.
  bool narrow = a.m <= kSkinnyMaxM;
  for (int i = 0; i < a.count; ++i) narrow = narrow && a.n[i] <= 4096;
  if (narrow) {
    const long tiles = tile_count(a, kTiles[7]);
    int splits = 1;
    while (tiles * splits * 2 <= 256 && valid_plan(a, 7, splits * 2) && a.k / pipe::BK / (splits * 2) >= 16 &&
           (size_t)splits * 2 * a.m * total_columns(a) * sizeof(float) <= workspace_bytes)
      splits *= 2;
    if (valid_plan(a, 7, splits) && tiles * splits >= 128) return GemmPlan{7, splits, true};
    return plan;
  }
  // Split K across workgroups with the 256 x 128 tile when that tile alone leaves most CUs
  // idle and the small tiles are no better: when even 64 x 64 tiles need more than one round
  // of 256 workgroups, or K is long (>= 8192).  Measured at M = 256 (q + k + v grouped 68 ->
  // 34 us with 4 splits, the Q6_K down 4096 x 12288 90 -> 54 us with 8); the 4096 x 4096 o
  // projection stays on 64 x 64 tiles (25 us against 30 split).  From M = 65 (timing harness,
  // M = 96 / 128 / 160): the down 4096 x 12288 Q6_K 96 / 95 / 93 -> 46 / 48 / 50 us with 8
  // splits, Q8_0 85 / 89 / 85 -> 46 / 48 / 49, Q4_K 55 / 55 / 56 -> 40 / 41 / 43; q + k + v at
  // M = 160 40 -> 31 with 4.  Splits double while the grid stays within 256 workgroups and each
  // split keeps >= 8 steps (512 of K).
  const long tiles = tile_count(a, kTiles[0]);
  const bool big_tile = plan.tile != 3 && plan.tile != 6 && plan.tile != 7;  // already fills the CUs
  const bool crowded = tile_count(a, kTiles[3]) > 256 || a.k >= 8192;
  if (a.m <= kSkinnyMaxM || big_tile || !crowded) return plan;
  int splits = 1;
  while (tiles * splits * 2 <= 256 && valid_plan(a, 0, splits * 2) && a.k / pipe::BK / (splits * 2) >= 8 &&
         (size_t)splits * 2 * a.m * total_columns(a) * sizeof(float) <= workspace_bytes)
    splits *= 2;
  if (splits > 1) plan = GemmPlan{0, splits};
  return plan;
}

size_t gemm_group_workspace(const GemmGroupArgs& a, const GemmPlan& plan) {
  return plan.splits > 1 ? (size_t)plan.splits * a.m * total_columns(a) * sizeof(float) : 0;
}

hipError_t launch_gemm_group_plan(const GemmGroupArgs& a, const GemmPlan& plan, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  if (!gemm_group_pipelined(a, plan) || a.count < 1 || a.count > kGemmGroupMax ||
      gemm_group_workspace(a, plan) > workspace_bytes || (plan.splits > 1 && !workspace))
    return hipErrorInvalidValue;
  switch (a.type) {
    case kQ4_K: return launch_typed<kQ4_K>(a, plan.tile, plan.splits, workspace, stream);
    case kQ5_K: return launch_typed<kQ5_K>(a, plan.tile, plan.splits, workspace, stream);
    case kQ6_K: return launch_typed<kQ6_K>(a, plan.tile, plan.splits, workspace, stream);
    case kQ8_0: return launch_typed<kQ8_0>(a, plan.tile, plan.splits, workspace, stream);
    default: return launch_typed<kQ4_0>(a, plan.tile, plan.splits, workspace, stream);
  }
}

bool gemm_tile_geometry(int tile, int* bm, int* bn, int* ks) {
  if (tile < 0 || tile >= kTileCount) return false;
  *bm = kTiles[tile].bm;
  *bn = kTiles[tile].bn;
  *ks = kTiles[tile].ks;
  return true;
}

bool gemm_group_pipelined(const GemmGroupArgs& a, const GemmPlan& plan) {
  return pipe_type(a.type) && valid_plan(a, plan.tile, plan.splits);
}

static GemmGroupArgs single(const GemvArgs& a) {
  GemmGroupArgs g{};
  g.x = a.x;
  g.w[0] = a.w;
  g.out[0] = a.out;
  g.n[0] = a.n;
  g.count = 1;
  g.type = a.type;
  g.m = a.m;
  g.k = a.k;
  g.out_half = a.out_half;
  g.x_f32 = a.x_f32;
  return g;
}

hipError_t launch_gemm_pipe_config(const GemvArgs& a, hipStream_t stream, int config) {
  if (a.x_f32 || !pipe_type(a.type)) return hipErrorInvalidValue;
  return launch_gemm_group_plan(single(a), GemmPlan{config, 1}, nullptr, 0, stream);
}

bool gemm_pipe_supported(const GemvArgs& a) {
  const GemmGroupArgs g = single(a);
  return gemm_group_pipelined(g, plan_gemm_group(g, 0));
}

hipError_t launch_gemm_pipe(const GemvArgs& a, hipStream_t stream, bool* handled) {
  const GemmGroupArgs g = single(a);
  const GemmPlan plan = plan_gemm_group(g, 0);
  *handled = gemm_group_pipelined(g, plan);
  if (!*handled) return hipSuccess;
  return launch_gemm_group_plan(g, plan, nullptr, 0, stream);
}

}  // namespace tensor_gguf
