// gemv.hip — decode-shaped fused dequant + matmul (small M).
//
// C[m, n] = sum_k A[m, k] * deq(W)[n, k], fp32 accumulation.  f32 path:
// exact f32 weights d*q; f16 path: each weight rounded to fp16 first,
// RNE(d*q), f16 activations, C rounded to fp16 (metal_provider.mm:1396-1468).
// Reassociation is allowed (block scales are factored out of each block's
// partial sum); dequantized values are never approximated.
//
// The kernel is HBM-bound: every weight byte is read exactly once.
//
// Pair kernel (K % 64 == 0):
//   * A "pair" is two consecutive blocks = 64 elements: 36 B of Q4_0
//     (9 dwords) or 68 B of Q8_0 (17 dwords).  Row strides are multiples of
//     the pair size, so every pair starts on a 4-byte boundary and one lane
//     fetches it with dword-aligned dwordx4 loads (2 x16 + 1 x4 for Q4_0,
//     4 x16 + 1 x4 for Q8_0).  Consecutive lanes read consecutive pairs, so
//     a wave's loads cover one contiguous span of the row.
//   * The first block of a pair starts 2 bytes into the pair: its code
//     dwords are realigned with v_alignbyte; the second block's codes are
//     already dword aligned.
//   * The activations (M rows of K) are staged once per workgroup in LDS,
//     64-element pair by pair, each pair followed by one 16-byte chunk of
//     padding (xslot), so the 16 lanes of a ds_read_b128 phase hit 16
//     different bank groups.
//   * A row is covered by a group of L lanes (L = 16, 32 or 64, chosen on the
//     host so the pairs of a row spread evenly); a wave holds 64/L groups and
//     each group works on R2 rows at once, reading each activation chunk
//     from LDS once for all R2 rows.  The weights of the next pair (two
//     pairs ahead when a lane has three or more) are loaded before the
//     current pair is computed.
//   * Partial sums are reduced across the L lanes of a group with DPP adds;
//     the group's last lane writes the R2 x M outputs.
//   * The grid is capped at two workgroups per CU; larger row counts loop,
//     reusing the staged activations.
//
// Unpacking (per 32-bit word of codes = 8 Q4_0 codes / 4 Q8_0 codes):
//   f32, Q4_0: the nibbles are masked in place into fp16 subnormals (n *
//       2^-24 or n * 2^-20) that v_fma_mix_f32 multiplies by the f32
//       activations exactly (pair_f32_q4).  The "-8" offset is applied once
//       per block: sum (n-8) x = sum n x - 8 sum x, with sum x per block
//       precomputed during staging.
//   f32, Q8_0: v_cvt_f32_i32 with SDWA byte select and sign extension.
//   f16: bytes are placed under 0x64 (fp16 1024 + n), shifted to the signed
//       code with one packed f16 add (exact), and multiplied by the fp16 scale
//       with one packed f16 multiply — RNE(d*q), the same bits as
//       dequant_*_f16 — then v_dot2c_f32_f16 accumulates in fp32.
//
// Block kernel (fallback for K % 64 == 32): one wave per output row, lanes
// stride over the row's 32-element blocks.
#include <cstdlib>

#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef float float2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2v as_h2(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t as_u32(half2v h) { return __builtin_bit_cast(uint32_t, h); }

template <class QF> struct PairFmt;
template <> struct PairFmt<Q4_0> {
  static constexpr int kBytes = 36, kDwords = 9, kQd = 4;  // kQd: code dwords per block
};
template <> struct PairFmt<Q8_0> {
  static constexpr int kBytes = 68, kDwords = 17, kQd = 8;
};

template <class QF>
__device__ __forceinline__ void load_pair(const uint8_t* p, uint32_t (&w)[PairFmt<QF>::kDwords]) {
  const u32x4a4* v = reinterpret_cast<const u32x4a4*>(p);
#pragma unroll
  for (int i = 0; i < PairFmt<QF>::kDwords / 4; ++i) {
    const u32x4 t = v[i];
    w[4 * i + 0] = t.x;
    w[4 * i + 1] = t.y;
    w[4 * i + 2] = t.z;
    w[4 * i + 3] = t.w;
  }
  w[PairFmt<QF>::kDwords - 1] = reinterpret_cast<const uint32_t*>(p)[PairFmt<QF>::kDwords - 1];
}

// Code dword t of block `blk` (0 or 1) of a loaded pair, and its fp16 scale bits.
template <class QF>
__device__ __forceinline__ uint32_t code_dword(const uint32_t* w, int blk, int t) {
  constexpr int qd = PairFmt<QF>::kQd;
  // block 0: codes start at byte 2 of the pair (realigned from two dwords);
  // block 1: scale in the upper half of dword qd, codes in dwords qd+1...
  if (blk == 0) return __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2);
  return w[qd + 1 + t];
}

template <class QF>
__device__ __forceinline__ uint32_t scale_bits(const uint32_t* w, int blk) {
  constexpr int qd = PairFmt<QF>::kQd;
  return blk == 0 ? (w[0] & 0xFFFFu) : (w[qd] >> 16);
}

// ---- LDS activation layout ------------------------------------------------
// f32: 16 chunks of 4 floats per pair; f16: 8 chunks of 8 halves per pair.
template <typename XT> struct XChunk;
template <> struct XChunk<float> {
  typedef float4v T;
  static constexpr int kPerPair = 16, kElems = 4;
};
template <> struct XChunk<half_t> {
  typedef half8 T;
  static constexpr int kPerPair = 8, kElems = 8;
};

// Chunk c of activation pair gp = m * P + pair (the pair's index over all
// M rows) lives at slot gp * (cp + 1) + c: each pair's chunks are followed
// by one chunk of padding.  The 16 lanes of one ds_read_b128 phase read
// chunk c of 16 consecutive pairs; with pairs 272 B (f32) or 144 B (f16)
// apart they fall in 16 different 16-byte bank groups of the 256-byte bank
// row (17 and 9 are odd), so the reads are conflict-free and every chunk of
// a pair is the pair's base address plus a constant offset.  (An XOR
// swizzle of the chunk index is conflict-free too but costs address
// arithmetic per read; f16 pairs swizzled with gp & 7 collided for pairs p
// and p + 8: 1.8 M bank-conflict cycles per 132 MB launch.)
template <typename XT>
__device__ __forceinline__ int xslot(int m, int P, int pair, int c) {
  constexpr int cp = XChunk<XT>::kPerPair;
  return (m * P + pair) * (cp + 1) + c;
}

// ---- per-pair compute -----------------------------------------------------

// f32 activations, Q4_0.  Masking a code dword leaves each nibble as an
// fp16 subnormal: (q & 0x000F000F) holds n * 2^-24 for elements (4t, 4t+2),
// (q & 0x00F000F0) 16n * 2^-24 = n * 2^-20 for (16+4t, 18+4t), and the same
// masks of q >> 8 the odd elements.  v_fma_mix_f32 widens an fp16 half to
// f32 inside the FMA (exactly, subnormals included: checked on MI355X for
// every nibble in both positions), so each product code * x is exact and
// rounded once into its fp32 chain: 5 instructions place 8 codes (against
// 7 for masking into bytes and four fp8 conversions).  Elements 16..31 of
// every block are staged divided by 16 (exact), so the 2^-20 codes times
// them count in the same units, 2^-24, as the rest; the block value is
// d * 2^24 * (sum - 8 * 2^-24 * sum x), the last term staged per block.
constexpr float kCodeUnit = 0x1p-24f;

template <int R2, int MM>
__device__ __forceinline__ void pair_f32_q4(const uint32_t (&w)[R2][9], const float4v* __restrict__ xs,
                                            const float* __restrict__ sxs, int P, int pair,
                                            float (&acc)[R2][MM]) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    // four independent FMA chains per block (one per code dword), added at
    // the end, so consecutive FMAs do not wait on each other
    float s[4][R2][MM];
    // all of the block's activation chunks are requested from LDS before
    // any arithmetic, so their latencies overlap
    float4v xa[4][MM], xb[4][MM];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        xa[t][m] = xs[xslot<float>(m, P, pair, blk * 8 + t)];
        xb[t][m] = xs[xslot<float>(m, P, pair, blk * 8 + 4 + t)];
      }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float4v* xl = xa[t];  // x[4t .. 4t+3]
      const float4v* xh = xb[t];  // x[16+4t .. 16+4t+3] / 16
#pragma unroll
      for (int j = 0; j < R2; ++j) {
        const uint32_t q = code_dword<Q4_0>(w[j], blk, t);
        const uint32_t q8 = q >> 8;
        const half2v ev_lo = as_h2(q & 0x000F000Fu);   // elements 4t, 4t+2
        const half2v ev_hi = as_h2(q & 0x00F000F0u);   // 16+4t, 18+4t
        const half2v od_lo = as_h2(q8 & 0x000F000Fu);  // 4t+1, 4t+3
        const half2v od_hi = as_h2(q8 & 0x00F000F0u);  // 17+4t, 19+4t
#pragma unroll
        for (int m = 0; m < MM; ++m) {
          // the chain starts with an FMA into zero: one v_fma_mix_f32, where
          // a product would be a conversion and a multiply
          float v = __builtin_fmaf((float)ev_lo[0], xl[m].x, 0.0f);
          v = __builtin_fmaf((float)od_lo[0], xl[m].y, v);
          v = __builtin_fmaf((float)ev_lo[1], xl[m].z, v);
          v = __builtin_fmaf((float)od_lo[1], xl[m].w, v);
          v = __builtin_fmaf((float)ev_hi[0], xh[m].x, v);
          v = __builtin_fmaf((float)od_hi[0], xh[m].y, v);
          v = __builtin_fmaf((float)ev_hi[1], xh[m].z, v);
          v = __builtin_fmaf((float)od_hi[1], xh[m].w, v);
          s[t][j][m] = v;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < R2; ++j) {
      const float d = h2f_bits((uint16_t)scale_bits<Q4_0>(w[j], blk)) * (1.0f / kCodeUnit);
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        const float sum = (s[0][j][m] + s[1][j][m]) + (s[2][j][m] + s[3][j][m]);
        acc[j][m] = __builtin_fmaf(d, sum - sxs[(m * P + pair) * 2 + blk], acc[j][m]);
      }
    }
  }
}

// f32 activations, Q8_0.
template <int R2, int MM>
__device__ __forceinline__ void pair_f32_q8(const uint32_t (&w)[R2][17], const float4v* __restrict__ xs,
                                            int P, int pair, float (&acc)[R2][MM]) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    // four independent FMA chains per block (code dwords t and t+4 share one)
    float s[4][R2][MM];
    float4v xall[8][MM];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int m = 0; m < MM; ++m) xall[t][m] = xs[xslot<float>(m, P, pair, blk * 8 + t)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float4v* xv = xall[t];
#pragma unroll
      for (int j = 0; j < R2; ++j) {
        const uint32_t q = code_dword<Q8_0>(w[j], blk, t);
        const float f0 = (float)(int8_t)(q);
        const float f1 = (float)(int8_t)(q >> 8);
        const float f2 = (float)(int8_t)(q >> 16);
        const float f3 = (float)((int32_t)q >> 24);
#pragma unroll
        for (int m = 0; m < MM; ++m) {
          float v = t < 4 ? f0 * xv[m].x : __builtin_fmaf(f0, xv[m].x, s[t & 3][j][m]);
          v = __builtin_fmaf(f1, xv[m].y, v);
          v = __builtin_fmaf(f2, xv[m].z, v);
          v = __builtin_fmaf(f3, xv[m].w, v);
          s[t & 3][j][m] = v;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < R2; ++j) {
      const float d = h2f_bits((uint16_t)scale_bits<Q8_0>(w[j], blk));
#pragma unroll
      for (int m = 0; m < MM; ++m)
        acc[j][m] = __builtin_fmaf(d, (s[0][j][m] + s[1][j][m]) + (s[2][j][m] + s[3][j][m]), acc[j][m]);
    }
  }
}


// (q & mask) | bits in one v_and_or_b32.  Its VOP3 encoding cannot carry
// 32-bit literals and reads at most one scalar register, so the mask comes
// from a scalar register and the bits from a (loop-invariant) vector one;
// the compiler otherwise emits a separate AND and OR.
__device__ __forceinline__ uint32_t and_or(uint32_t q, uint32_t mask, uint32_t bits) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(q), "s"(mask), "v"(bits));
  return r;
}

// f16 activations (weights rounded to fp16 exactly as dequant_*_f16).
//
// Q4_0: the four half2 of code dword t come straight from its nibble
// positions with one AND-OR each, no byte shuffle: a nibble in bits 0-3 of
// a 16-bit half under exponent bits 0x64 reads as 1024 + n, a nibble in
// bits 4-7 under 0x54 as 64 + n (fp16 with unit spacing there), so
//   (q & 0x000F000F) | 0x64006400       -> elements (4t,    4t+2)
//   (q & 0x00F000F0) | 0x54005400       -> elements (16+4t, 18+4t)
//   ((q>>8) & 0x000F000F) | 0x64006400  -> elements (4t+1,  4t+3)
//   ((q>>8) & 0x00F000F0) | 0x54005400  -> elements (17+4t, 19+4t)
// then one packed add (-1032 / -72: exact, the signed code) and one packed
// multiply by d (RNE(d*q), the dequant_q4_0_f16 bits).  The staged
// activations hold each block's chunk t in that element order (stage_f16_q4).
// Q8_0: each code byte under 0x64 via a byte permute (1024 + 128 + q).
template <class QF, int R2, int MM>
__device__ __forceinline__ void pair_f16(const uint32_t (&w)[R2][PairFmt<QF>::kDwords],
                                         const half8* __restrict__ xs, int P, int pair,
                                         float (&acc)[R2][MM]) {
  constexpr bool kQ4 = PairFmt<QF>::kQd == 4;
  constexpr int qd = PairFmt<QF>::kQd;
  // four independent accumulation chains (code dword t feeds chain t & 3),
  // folded into acc at the end of the pair
  float part[4][R2][MM];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int j = 0; j < R2; ++j)
#pragma unroll
      for (int m = 0; m < MM; ++m) part[c][j][m] = 0.f;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    half8 xv[MM][4];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
      for (int c = 0; c < 4; ++c) xv[m][c] = xs[xslot<half_t>(m, P, pair, blk * 4 + c)];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < R2; ++j) {
      const uint32_t db = scale_bits<QF>(w[j], blk);
      const half2v d2 = as_h2(db | (db << 16));
#pragma unroll
      for (int t = 0; t < qd; ++t) {
        const uint32_t q = code_dword<QF>(w[j], blk, t);
        if constexpr (kQ4) {
          const uint32_t s8 = q >> 8;
          const half2v lo_off = {(half_t)-1032.f, (half_t)-1032.f};
          const half2v hi_off = {(half_t)-72.f, (half_t)-72.f};
          const half2v w0 = (as_h2(and_or(q, 0x000F000Fu, 0x64006400u)) + lo_off) * d2;
          const half2v w1 = (as_h2(and_or(q, 0x00F000F0u, 0x54005400u)) + hi_off) * d2;
          const half2v w2 = (as_h2(and_or(s8, 0x000F000Fu, 0x64006400u)) + lo_off) * d2;
          const half2v w3 = (as_h2(and_or(s8, 0x00F000F0u, 0x54005400u)) + hi_off) * d2;
#pragma unroll
          for (int m = 0; m < MM; ++m) {
            const half8 xc = xv[m][t];
            float v = part[t & 3][j][m];
            v = __builtin_amdgcn_fdot2(w0, half2v{xc[0], xc[1]}, v, false);
            v = __builtin_amdgcn_fdot2(w1, half2v{xc[2], xc[3]}, v, false);
            v = __builtin_amdgcn_fdot2(w2, half2v{xc[4], xc[5]}, v, false);
            v = __builtin_amdgcn_fdot2(w3, half2v{xc[6], xc[7]}, v, false);
            part[t & 3][j][m] = v;
          }
        } else {
          // Q8_0: 4 signed codes -> elements 4t..4t+3 (chunk t/2, halves 4*(t&1)..)
          const uint32_t u = q ^ 0x80808080u;  // code + 128, unsigned
          const half2v off = {(half_t)-1152.f, (half_t)-1152.f};
          const half2v w0 = (as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + off) * d2;
          const half2v w1 = (as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + off) * d2;
#pragma unroll
          for (int m = 0; m < MM; ++m) {
            const half8 xc = xv[m][t >> 1];
            const int o = (t & 1) * 4;
            float v = part[t & 3][j][m];
            v = __builtin_amdgcn_fdot2(w0, half2v{xc[o + 0], xc[o + 1]}, v, false);
            v = __builtin_amdgcn_fdot2(w1, half2v{xc[o + 2], xc[o + 3]}, v, false);
            part[t & 3][j][m] = v;
          }
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < R2; ++j)
#pragma unroll
    for (int m = 0; m < MM; ++m)
      acc[j][m] += (part[0][j][m] + part[1][j][m]) + (part[2][j][m] + part[3][j][m]);
}

// The Q4_0 f16 order of one 32-element block of activations: chunk t (t = 0..3)
// = (x[4t], x[4t+2]), (x[16+4t], x[18+4t]), (x[4t+1], x[4t+3]), (x[17+4t], x[19+4t]),
// from the block's four consecutive 8-element chunks v[0..3].
__device__ __forceinline__ half8 q4_f16_chunk(const half8 (&v)[4], int t) {
  const u32x4 a = __builtin_bit_cast(u32x4, v[t >> 1]);
  const u32x4 b = __builtin_bit_cast(u32x4, v[2 + (t >> 1)]);
  const uint32_t a0 = (t & 1) ? a.z : a.x, a1 = (t & 1) ? a.w : a.y;  // x[4t..4t+1], x[4t+2..4t+3]
  const uint32_t b0 = (t & 1) ? b.z : b.x, b1 = (t & 1) ? b.w : b.y;
  u32x4 o;
  o.x = __builtin_amdgcn_perm(a1, a0, 0x05040100u);  // low halves: x[4t], x[4t+2]
  o.y = __builtin_amdgcn_perm(b1, b0, 0x05040100u);
  o.z = __builtin_amdgcn_perm(a1, a0, 0x07060302u);  // high halves: x[4t+1], x[4t+3]
  o.w = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
  return __builtin_bit_cast(half8, o);
}

// ---- cross-lane sums --------------------------------------------------------

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xF, false));
}

// Sum over aligned groups of 2^log2L lanes (16, 32 or 64).  Within a row of
// 16: quad_perm xor 1, xor 2, row_half_mirror, row_mirror leave the row sum
// in every lane; row_bcast15 / row_bcast31 then fold rows 0+1 (2+3) and
// 01+23.  The group sum is in the group's last lane.
__device__ __forceinline__ float group_sum(float v, int log2L) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  if (log2L >= 5) v += dpp_f<0x142, 0xA>(v);  // row_bcast15 -> rows 1, 3
  if (log2L >= 6) v += dpp_f<0x143, 0xC>(v);  // row_bcast31 -> rows 2, 3
  return v;
}

// ---- the pair kernel ------------------------------------------------------

// Up to kGroupMax GEMVs over the same activations in one launch: job j owns
// workgroups begin[j] .. begin[j+1]-1, a share of the capped grid in
// proportion to its rows, which loop over the job's rows exactly as the
// grid of a single launch loops over one matrix's (a single launch is a
// group of one).  The job is uniform per workgroup, so weight and output
// bases stay scalar.
constexpr int kGroupMax = nfhip::kGemvGroupMax;
static_assert(kGroupMax == 4, "gemv_pair_kernel passes begin[1..3] as scalar arguments");
struct GemvGroup {
  const uint8_t* W[kGroupMax];
  void* C[kGroupMax];
  int N[kGroupMax];
  int begin[kGroupMax + 1];
};

// NS register sets of weights in rotation: the loads run NS - 1 steps ahead.
//
// Arguments: job 0's weights, output and rows and the job boundaries
// begin[1..3] come first as plain scalars (W0 = grp.W[0], ...), so they are
// among the arguments preloaded into SGPRs at wave launch: a workgroup of
// job 0 (every workgroup of a single launch) issues its first loads without
// waiting on a scalar load from the argument block.  Other jobs read their
// entries of `grp` (one round trip).
template <class QF, typename XT, int R2, int MM, int NS>
__global__ __launch_bounds__(256) void gemv_pair_kernel(const XT* __restrict__ A, const uint8_t* __restrict__ W0,
                                                        void* C0, int N0, int b1, int b2, int b3, int M, int K,
                                                        int log2L, const GemvGroup grp) {
  // This workgroup's job (uniform): begin[] is non-decreasing, and unused
  // entries equal the grid size.
  const int bx = (int)blockIdx.x;
  const int job = (bx >= b1) + (bx >= b2) + (bx >= b3);
  const uint8_t* __restrict__ W = W0;
  void* Cv = C0;
  int N = N0, wg0 = 0, wg1 = b1;
  if (job > 0) {
    W = grp.W[job];
    Cv = grp.C[job];
    N = grp.N[job];
    wg0 = grp.begin[job];
    wg1 = grp.begin[job + 1];
  }
  XT* __restrict__ C = static_cast<XT*>(Cv);
  const int bid = (int)blockIdx.x - wg0, nwg = wg1 - wg0;
  constexpr bool kF32 = sizeof(XT) == 4;
  constexpr bool kQ4 = PairFmt<QF>::kQd == 4;
  constexpr bool kSx = kF32 && kQ4;  // block sums of x needed for the nibble offset
  constexpr int CP = XChunk<XT>::kPerPair;
  constexpr int EPC = XChunk<XT>::kElems;
  constexpr int DW = PairFmt<QF>::kDwords;
  typedef typename XChunk<XT>::T ChunkT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  const int P = K >> 6;
  ChunkT* xs = reinterpret_cast<ChunkT*>(smem);
  float* sxs = reinterpret_cast<float*>(smem + (size_t)MM * P * (CP + 1) * 16);
  const int tid = threadIdx.x;


  const int lane = tid & 63, wave = tid >> 6;
  const int L = 1 << log2L;
  const int R = 64 >> log2L;
  const int g = lane >> log2L, li = lane & (L - 1);
  const int rows_per_pass = 4 * R * R2;
  const int pass_stride = nwg * rows_per_pass;
  const size_t row_bytes = (size_t)P * PairFmt<QF>::kBytes;

  // Iteration space of a lane group: npass passes over the grid's rows, IP
  // pair steps per pass (pair = li + L * step).  Both are uniform across the
  // workgroup, so every lane runs the same straight-line loop; loads past
  // the end are clamped to the last row / pair and never stored.
  const int base0 = bid * rows_per_pass;
  const int grp_row = base0 + (wave * R + g) * R2;
  const int IP = (P + L - 1) >> log2L;
  const int npass = base0 < N ? (N - 1 - base0) / pass_stride + 1 : 0;
  const int T = npass * IP;

  int lpass = 0, lk = 0;  // position of the next weight load
  auto next_load = [&](uint32_t (&w)[R2][DW]) {
    const int r0 = grp_row + lpass * pass_stride;
    int pair = li + (lk << log2L);
    pair = pair < P ? pair : P - 1;
#pragma unroll
    for (int j = 0; j < R2; ++j) {
      const int r = r0 + j < N ? r0 + j : N - 1;
      load_pair<QF>(W + (size_t)r * row_bytes + (size_t)pair * PairFmt<QF>::kBytes, w[j]);
    }
    if (++lk == IP) {
      lk = 0;
      ++lpass;
    }
  };

  uint32_t wr[NS][R2][DW];

  // ---- stage A into LDS (and the per-block sums of x) ----
  // The first two rounds of activations (all of them up to M * K = 16384
  // f32 / 32768 f16 elements) are requested before the first weights, so
  // the two memory round trips overlap; the activations go first because
  // loads complete in issue order: the (L2-resident) activations are then
  // staged while the weights stream from HBM (measured on MI355X: 3.3
  // against 3.8 us at 2048 x 2048 with the weights first).  Later rounds,
  // if any, follow the weights.  Loads past the end are clamped to the last
  // item and dropped, so no load is predicated and all of a round are in
  // flight together (skipping whole rounds past the end behind a uniform
  // branch instead measured 542 against 437 us for the TinyLlama decode
  // step).
  if constexpr (!kF32 && kQ4) {
    // f16 Q4_0: thread tid takes 32-element blocks tid, tid + 256, ... (four
    // 16-byte loads each) and writes them in the order pair_f16 reads.
    const int totb = M * P * 2;
    typedef half8 Blk[2][4];
    auto load = [&](int b0, Blk& v) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int b = b0 + u * 256 + tid;
        const half8* src = reinterpret_cast<const half8*>(A + (size_t)(b < totb ? b : totb - 1) * 32);
#pragma unroll
        for (int c = 0; c < 4; ++c) v[u][c] = src[c];
      }
    };
    auto put = [&](int b0, const Blk& v) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int b = b0 + u * 256 + tid;
        if (b < totb) {
          const int gp = b >> 1, blk = b & 1;
#pragma unroll
          for (int t = 0; t < 4; ++t) xs[gp * (CP + 1) + blk * 4 + t] = q4_f16_chunk(v[u], t);
        }
      }
    };
    Blk v0, v1;
    load(0, v0);
    const bool two = totb > 512;
    if (two) load(512, v1);
    if (T > 0) next_load(wr[0]);
    put(0, v0);
    if (two) put(512, v1);
    for (int b0 = 1024; b0 < totb; b0 += 512) {
      load(b0, v0);
      put(b0, v0);
    }
  } else {
    // Thread tid takes 16-byte chunks tid, tid + 256, ... of the M x K
    // activations, so every load instruction reads contiguous memory.  A
    // 32-element block is 8 (f32) chunks held by 8 consecutive lanes; its
    // sum is formed with DPP adds across them (total is a multiple of 8, so
    // the 8 lanes of a block are in or out of range together).
    const int total = M * P * CP;
    // chunk c is 4 elements of a 32-element block; its position in the block
    // is c & 7, which (every round starting at a multiple of 16 chunks) is
    // tid & 7: elements 16..31 for tid & 4
    const float xscale = (tid & 4) ? 0.0625f : 1.0f;
    auto load = [&](int c0, ChunkT (&v)[8]) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = c0 + u * 256 + tid;
        v[u] = *reinterpret_cast<const ChunkT*>(A + (size_t)(c < total ? c : total - 1) * EPC);
      }
    };
    auto put = [&](int c0, const ChunkT (&v)[8]) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = c0 + u * 256 + tid;
        if (c < total) {
          const int gp = c / CP, j = c & (CP - 1);
          if constexpr (kSx) {
            // f32 Q4_0 stages elements 16..31 of each block divided by 16
            // (pair_f32_q4); the block sums below use the values as given
            xs[gp * (CP + 1) + j] = v[u] * xscale;
          } else {
            xs[gp * (CP + 1) + j] = v[u];
          }
          if constexpr (kSx) {
            float sum = (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
            sum += dpp_f<0xB1>(sum);   // quad_perm [1,0,3,2]
            sum += dpp_f<0x4E>(sum);   // quad_perm [2,3,0,1]
            sum += dpp_f<0x141>(sum);  // row_half_mirror: every lane of the 8 holds the block sum
            if ((j & 7) == 0) sxs[gp * 2 + (j >> 3)] = sum * (8.0f * kCodeUnit);
          }
        }
      }
    };
    ChunkT v0[8], v1[8];
    load(0, v0);
    const bool two = total > 256 * 8;
    if (two) load(256 * 8, v1);
    if (T > 0) next_load(wr[0]);
    put(0, v0);
    if (two) put(256 * 8, v1);
    for (int c0 = 2 * 256 * 8; c0 < total; c0 += 256 * 8) {
      load(c0, v0);
      put(c0, v0);
    }
  }
  __syncthreads();

  float acc[R2][MM];
#pragma unroll
  for (int j = 0; j < R2; ++j)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[j][m] = 0.f;

  int cpass = 0, ck = 0;  // position of the next compute step
  auto step = [&](const uint32_t (&w)[R2][DW]) {
    const int pair = li + (ck << log2L);
    if (pair < P) {
      if constexpr (kF32) {
        if constexpr (kQ4) {
          pair_f32_q4<R2, MM>(w, reinterpret_cast<const float4v*>(xs), sxs, P, pair, acc);
        } else {
          pair_f32_q8<R2, MM>(w, reinterpret_cast<const float4v*>(xs), P, pair, acc);
        }
      } else {
        pair_f16<QF, R2, MM>(w, reinterpret_cast<const half8*>(xs), P, pair, acc);
      }
    }
    if (++ck == IP) {
      // end of a pass: reduce across the L lanes of the group (DPP; the sum
      // lands in lane L-1), store, restart the sums
      const int r0 = grp_row + cpass * pass_stride;
#pragma unroll
      for (int j = 0; j < R2; ++j)
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[j][m] = group_sum(acc[j][m], log2L);
      if (li == L - 1) {
#pragma unroll
        for (int j = 0; j < R2; ++j) {
          if (r0 + j >= N) continue;
#pragma unroll
          for (int m = 0; m < MM; ++m)
            if (m < M) C[(size_t)m * N + r0 + j] = (XT)acc[j][m];
        }
      }
#pragma unroll
      for (int j = 0; j < R2; ++j)
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[j][m] = 0.f;
      ck = 0;
      ++cpass;
    }
  };

  // Register sets in rotation: the loads of step t + NS - 1 are issued
  // before step t is computed (NS from gemv_sets).  Set 0 was requested
  // during staging; loads past the last step are clamped and never used.
#pragma unroll
  for (int i = 1; i < NS - 1; ++i) next_load(wr[i]);
  for (int t = 0; t < T; t += NS) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      next_load(wr[(i + NS - 1) % NS]);
      __builtin_amdgcn_sched_barrier(0);
      if (t + i < T) step(wr[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// ---- block kernel (odd number of blocks per row) ----------------------------

template <typename AT>
__device__ __forceinline__ float dot32(const AT* __restrict__ x, const float w[32]);

template <>
__device__ __forceinline__ float dot32<float>(const float* __restrict__ x, const float w[32]) {
  const float4v* xv = reinterpret_cast<const float4v*>(x);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float4v t = xv[j];
    s = __builtin_fmaf(w[4 * j + 0], t[0], s);
    s = __builtin_fmaf(w[4 * j + 1], t[1], s);
    s = __builtin_fmaf(w[4 * j + 2], t[2], s);
    s = __builtin_fmaf(w[4 * j + 3], t[3], s);
  }
  return s;
}

template <>
__device__ __forceinline__ float dot32<half_t>(const half_t* __restrict__ x, const float w[32]) {
  const half8* xv = reinterpret_cast<const half8*>(x);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const half8 t = xv[j];
#pragma unroll
    for (int i = 0; i < 8; ++i) s = __builtin_fmaf(w[8 * j + i], (float)t[i], s);
  }
  return s;
}

template <class QF, typename AT, int MT>
__global__ __launch_bounds__(256) void gemv_block_kernel(const AT* __restrict__ A,
                                                         const uint8_t* __restrict__ W,
                                                         AT* __restrict__ C, int M, int N, int K) {
  constexpr bool kHalfW = sizeof(AT) == 2;
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;  // whole wave leaves; no CTA barriers below
  const int m0 = blockIdx.y * MT;
  const int nb = K >> 5;
  const uint8_t* wrow = W + (size_t)n * nb * QF::kBytes;
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.f;

  for (int b = lane; b < nb; b += 64) {
    float w[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) quarter_f32<QF>(wrow + (size_t)b * QF::kBytes, q, &w[8 * q]);
    if constexpr (kHalfW) {
#pragma unroll
      for (int i = 0; i < 32; ++i) w[i] = (float)(half_t)w[i];
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (m0 + m < M) acc[m] += dot32<AT>(A + (size_t)(m0 + m) * K + (size_t)b * 32, w);
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const float v = wave_sum(acc[m]);
    if (lane == 0 && m0 + m < M) C[(size_t)(m0 + m) * N + n] = (AT)v;
  }
}

template <class QF, typename AT>
hipError_t gemv_block_dispatch(const void* A, const void* W, void* C, uint32_t M, uint32_t N,
                               uint32_t K, hipStream_t s) {
  const dim3 block(256);
  const int mt = M == 1 ? 1 : (M == 2 ? 2 : (M <= 4 ? 4 : 8));
  const dim3 grid((N + 3) / 4, (M + mt - 1) / mt);
  if (grid.y > 65535) return hipErrorInvalidConfiguration;
  const AT* a = static_cast<const AT*>(A);
  const uint8_t* w = static_cast<const uint8_t*>(W);
  AT* c = static_cast<AT*>(C);
  switch (mt) {
    case 1: gemv_block_kernel<QF, AT, 1><<<grid, block, 0, s>>>(a, w, c, M, N, K); break;
    case 2: gemv_block_kernel<QF, AT, 2><<<grid, block, 0, s>>>(a, w, c, M, N, K); break;
    case 4: gemv_block_kernel<QF, AT, 4><<<grid, block, 0, s>>>(a, w, c, M, N, K); break;
    default: gemv_block_kernel<QF, AT, 8><<<grid, block, 0, s>>>(a, w, c, M, N, K); break;
  }
  return hipGetLastError();
}

// Host-side geometry of the pair kernel.
struct PairGeom {
  int log2L = 5, R2 = 1, MM = 1, sets = 2;
  unsigned grid = 1;
  size_t lds = 0;
};

// Lanes per row: the largest of 64/32/16 whose round-robin split of the P
// pairs keeps >= 95% of the lanes busy, else the best split.
inline int pick_log2L(int P) {
  static const int forced = [] {
    const char* e = std::getenv("NF_HIP_GEMV_LOG2L");  // tuning override: 4, 5 or 6
    const int v = e ? std::atoi(e) : 0;
    return v >= 4 && v <= 6 ? v : 0;
  }();
  if (forced) return forced;
  static const double min_u = [] {
    const char* e = std::getenv("NF_HIP_GEMV_MIN_UTIL");  // tuning override
    const double v = e ? std::atof(e) : 0.0;
    return v > 0.0 && v <= 1.0 ? v : 0.95;
  }();
  int best = 6;
  double best_u = 0.0;
  for (int lg = 6; lg >= 4; --lg) {
    const int L = 1 << lg;
    const int it = (P + L - 1) / L;
    const double u = (double)P / (double)(L * it);
    if (u >= min_u) return lg;
    if (u > best_u + 1e-9) {
      best_u = u;
      best = lg;
    }
  }
  return best;
}

// Activations staged per workgroup: up to 136 KB of LDS (above 64 KB the
// kernel has to opt in, once per instantiation): the planner's 120 KB of
// activations (plan.cpp) plus the padding chunks and the f32 block sums.
constexpr size_t kPairMaxLds = 136 * 1024;

template <class QF, typename XT, int R2, int MM, int NS>
hipError_t gemv_pair_launch(const PairGeom& g, const void* A, const GemvGroup& grp, uint32_t M, uint32_t K,
                            hipStream_t s) {
  if (g.lds > 64 * 1024) {
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_pair_kernel<QF, XT, R2, MM, NS>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPairMaxLds);
    if (attr != hipSuccess) return attr;
  }
  gemv_pair_kernel<QF, XT, R2, MM, NS><<<dim3(g.grid), dim3(256), g.lds, s>>>(
      static_cast<const XT*>(A), grp.W[0], grp.C[0], grp.N[0], grp.begin[1], grp.begin[2], grp.begin[3], (int)M,
      (int)K, g.log2L, grp);
  return hipGetLastError();
}

// Weight register sets for a lane running `steps` steps: one step ahead for
// one or two steps (a second set's loads would be wasted), two ahead from
// three steps (11008 x 4096: 8.1 against 8.8 us) with one or two activation
// rows; four activation rows keep two sets (a third costs occupancy).
// Three and four steps ahead measured slower on MI355X (Llama-2-7B decode
// step 1264 / 1234 against 1162 us, 4096 x 11008 11.1 / 10.8 against
// 10.3 us), so the kernel is instantiated for two and three sets.
inline int gemv_sets(int MM, long steps) { return (MM <= 2 && steps >= 3) ? 3 : 2; }

// Geometry of a pair-kernel launch over `rows` rows (one matrix or a whole
// group) with M activation rows of K; false when its activation stage would
// not fit in LDS.
template <class QF, typename XT>
bool pair_geom(uint32_t M, uint32_t K, long rows, PairGeom& g) {
  constexpr bool kF32 = sizeof(XT) == 4;
  const int P = (int)(K / 64);
  g.MM = M == 1 ? 1 : (M == 2 ? 2 : 4);
  // staged pairs with one padding chunk each (xslot)
  const size_t xbytes = (size_t)g.MM * P * ((kF32 ? 16 : 8) + 1) * 16;
  const size_t sxbytes = (kF32 && PairFmt<QF>::kQd == 4) ? (size_t)g.MM * P * 2 * 4 : 0;
  g.lds = xbytes + sxbytes;
  if (g.lds > kPairMaxLds) return false;
  g.log2L = pick_log2L(P);
  const int R = 64 >> g.log2L;
  // The grid is capped at two workgroups per CU, which loop over the rows
  // reusing their staged activations (measured on MI355X: at 4096x4096 the
  // capped grid takes 5.8 us against 6.6 us for one workgroup per 4 rows).
  // One row per lane group: with the loads two steps ahead (three register
  // sets) that keeps enough bytes in flight, and it measured faster than two
  // rows per lane group with one step ahead (11008 x 4096: 8.1 against
  // 9.5 us; 32000 x 2048: 10.2 against 11.0 us).
  static const long cap = [] {
    const char* e = std::getenv("NF_HIP_GEMV_WG_CAP");  // tuning override
    const long v = e ? std::atol(e) : 0;
    return v > 0 ? v : 256L * 2;
  }();
  const long wgs = (rows + 4L * R - 1) / (4L * R);
  g.R2 = 1;
  g.grid = (unsigned)(wgs < cap ? wgs : cap);
  // steps of a lane: passes over the rows times pair steps per row
  const long passes = (rows + (long)g.grid * 4L * R - 1) / ((long)g.grid * 4L * R);
  g.sets = gemv_sets(g.MM, passes * ((P + (1 << g.log2L) - 1) >> g.log2L));
  return true;
}

template <class QF, typename XT>
hipError_t gemv_pair_group(const PairGeom& g, const void* A, const GemvGroup& grp, uint32_t M, uint32_t K,
                           hipStream_t s) {
  switch (g.MM * 8 + g.sets) {
    case 8 + 2: return gemv_pair_launch<QF, XT, 1, 1, 2>(g, A, grp, M, K, s);
    case 8 + 3: return gemv_pair_launch<QF, XT, 1, 1, 3>(g, A, grp, M, K, s);
    case 16 + 2: return gemv_pair_launch<QF, XT, 1, 2, 2>(g, A, grp, M, K, s);
    case 16 + 3: return gemv_pair_launch<QF, XT, 1, 2, 3>(g, A, grp, M, K, s);
    default: return gemv_pair_launch<QF, XT, 1, 4, 2>(g, A, grp, M, K, s);
  }
}

template <class QF, typename XT>
hipError_t gemv_dispatch(const void* A, const void* W, void* C, uint32_t M, uint32_t N, uint32_t K,
                         hipStream_t s) {
  const bool aligned = ((uintptr_t)A % 16 == 0) && ((uintptr_t)W % 4 == 0);
  PairGeom g;
  if (K % 64 != 0 || M > 4 || !aligned || !pair_geom<QF, XT>(M, K, (long)N, g))
    return gemv_block_dispatch<QF, XT>(A, W, C, M, N, K, s);
  GemvGroup grp{};
  grp.W[0] = static_cast<const uint8_t*>(W);
  grp.C[0] = C;
  grp.N[0] = (int)N;
  grp.begin[0] = 0;
  for (int q = 1; q <= kGroupMax; ++q) grp.begin[q] = (int)g.grid;
  return gemv_pair_group<QF, XT>(g, A, grp, M, K, s);
}

// A group: the geometry of a single matrix with all the jobs' rows, its
// capped grid split among the jobs in proportion to their rows (at least
// one workgroup each, never more than a job's rows need).
template <class QF, typename XT>
hipError_t gemv_group_dispatch(const void* A, const nfhip::GemvJob* jobs, uint32_t n, uint32_t M, uint32_t K,
                               hipStream_t s) {
  if (n < 1 || n > (uint32_t)kGroupMax || K % 64 != 0 || M < 1 || M > 4 || (uintptr_t)A % 16 != 0)
    return hipErrorNotSupported;
  long total = 0;
  for (uint32_t j = 0; j < n; ++j) {
    if ((uintptr_t)jobs[j].W % 4 != 0 || jobs[j].N == 0) return hipErrorNotSupported;
    total += jobs[j].N;
  }
  PairGeom g;
  if (!pair_geom<QF, XT>(M, K, total, g)) return hipErrorNotSupported;
  const long rows_per_wg = 4L * (64 >> g.log2L);
  GemvGroup grp{};
  long wg = 0, rows_before = 0;
  for (uint32_t j = 0; j < n; ++j) {
    grp.W[j] = static_cast<const uint8_t*>(jobs[j].W);
    grp.C[j] = jobs[j].C;
    grp.N[j] = (int)jobs[j].N;
    grp.begin[j] = (int)wg;
    // workgroups [begin_j, begin_j+1): job j's share of the grid, rounded at
    // the running row total so the shares add up to the grid
    rows_before += jobs[j].N;
    long end = (long)((double)g.grid * (double)rows_before / (double)total + 0.5);
    const long need = ((long)jobs[j].N + rows_per_wg - 1) / rows_per_wg;
    if (end < wg + 1) end = wg + 1;
    if (end > wg + need) end = wg + need;
    wg = end;
  }
  for (int q = (int)n; q <= kGroupMax; ++q) grp.begin[q] = (int)wg;
  g.grid = (unsigned)wg;
  return gemv_pair_group<QF, XT>(g, A, grp, M, K, s);
}

// ---- launch-floor calibration ------------------------------------------------
// Reads `n16` 16-byte chunks (PER per thread, all issued before any is used)
// and reduces them to nothing that is stored: the cost of streaming the same
// bytes as a GEMV with none of its work, for the benchmark's per-launch floor.
template <int PER>
__global__ __launch_bounds__(256) void diag_read_kernel(const u32x4a4* __restrict__ src, uint64_t n16,
                                                        uint32_t* __restrict__ sink) {
  const uint64_t t = (uint64_t)blockIdx.x * 256 + threadIdx.x, nt = (uint64_t)gridDim.x * 256;
  u32x4 v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const uint64_t j = t + (uint64_t)i * nt;
    v[i] = src[j < n16 ? j : n16 - 1];
  }
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < PER; ++i) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
  if (x == 0x9E3779B9u && sink) sink[0] = x;  // keeps the loads; never true for the benchmark's data
}

__global__ void diag_empty_kernel() {}

}  // namespace nfk

namespace nfhip {

hipError_t launch_diag_read(const void* src, uint64_t bytes, hipStream_t s) {
  if (bytes < 16 || !src) {
    nfk::diag_empty_kernel<<<1, 64, 0, s>>>();
    return hipGetLastError();
  }
  const uint64_t n16 = bytes / 16;
  const nfk::u32x4a4* p = static_cast<const nfk::u32x4a4*>(src);
  // Two workgroups per CU while that covers the bytes with <= 8 chunks per
  // thread, else 16 chunks per thread and as many workgroups as needed.
  const uint64_t threads = 512ull * 256;
  const uint64_t per = (n16 + threads - 1) / threads;
  if (per <= 1) nfk::diag_read_kernel<1><<<512, 256, 0, s>>>(p, n16, nullptr);
  else if (per <= 2) nfk::diag_read_kernel<2><<<512, 256, 0, s>>>(p, n16, nullptr);
  else if (per <= 4) nfk::diag_read_kernel<4><<<512, 256, 0, s>>>(p, n16, nullptr);
  else if (per <= 8) nfk::diag_read_kernel<8><<<512, 256, 0, s>>>(p, n16, nullptr);
  else nfk::diag_read_kernel<16><<<(unsigned)((n16 + 16 * 256 - 1) / (16 * 256)), 256, 0, s>>>(p, n16, nullptr);
  return hipGetLastError();
}

hipError_t launch_gemv_group(QFmt q, EType t, const void* A, const GemvJob* jobs, uint32_t n, uint32_t M,
                             uint32_t K, hipStream_t s) {
  if (q == QFmt::Q4_0)
    return t == EType::F32 ? nfk::gemv_group_dispatch<nfk::Q4_0, float>(A, jobs, n, M, K, s)
                           : nfk::gemv_group_dispatch<nfk::Q4_0, nfk::half_t>(A, jobs, n, M, K, s);
  return t == EType::F32 ? nfk::gemv_group_dispatch<nfk::Q8_0, float>(A, jobs, n, M, K, s)
                         : nfk::gemv_group_dispatch<nfk::Q8_0, nfk::half_t>(A, jobs, n, M, K, s);
}

hipError_t launch_gemv(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                       uint32_t N, uint32_t K, hipStream_t s) {
  if (q == QFmt::Q4_0)
    return t == EType::F32 ? nfk::gemv_dispatch<nfk::Q4_0, float>(A, W, C, M, N, K, s)
                           : nfk::gemv_dispatch<nfk::Q4_0, nfk::half_t>(A, W, C, M, N, K, s);
  return t == EType::F32 ? nfk::gemv_dispatch<nfk::Q8_0, float>(A, W, C, M, N, K, s)
                         : nfk::gemv_dispatch<nfk::Q8_0, nfk::half_t>(A, W, C, M, N, K, s);
}

}  // namespace nfhip
