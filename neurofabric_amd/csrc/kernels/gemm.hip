// gemm.hip — prefill-shaped fused dequant + matmul on CDNA4 MFMA.
//
// f16 path (metal_provider.mm:1433-1468 semantics): A f16 [M,K]; W quantized
// [N,K]; each weight is dequantized to fp16 as RNE(d*q) — the same bits
// dequant_*_f16 produces — and multiplied with fp32 accumulation; C is
// rounded to fp16.
//
// Three kernels:
//   * register-dequantizing tiled kernel (gemm_wq_kernel, K % 64 == 0): the
//     default prefill path.  Workgroup tile 128(M) x 256(N), 4 waves side by
//     side along N, each owning 128x64 = 4x2 v_mfma_f32_32x32x16_f16 tiles.
//     A goes through a two-stage LDS buffer; each wave loads its own weight
//     blocks straight into registers four K steps ahead and dequantizes them
//     there (weights never touch LDS, and no weight is dequantized twice).
//     The issue order of each K step is fixed slot by slot so that loads,
//     LDS writes and dequantization VALU sit in the shadow of the MFMAs.
//   * LDS-staged tiled kernel (gemm_tile_kernel, K % 64 == 0): A streams into
//     LDS with direct-to-LDS loads, the workgroup dequantizes each weight
//     tile once into LDS as fp16, and the waves read both operands from LDS;
//     tile shapes 256x256 .. 128x128 (selectable; also the dense fp16 path).
//   * small-tile kernel (any K % 32 == 0): fallback for shapes the two above
//     do not take.
//
// MFMA 32x32x16 f16 operand layout (lane l of a wave64):
//   A: row l%32, k = 8*(l/32) .. +7     (8 halves, one ds_read_b128)
//   B: col l%32, k = 8*(l/32) .. +7
//   D: col l%32, row (r/4)*8 + (l/32)*4 + r%4 for accumulator r = 0..15
//
// Small-tile kernel (any K % 32 == 0): CTA tile 64x64, 4 waves of 32x32
// built from v_mfma_f32_16x16x32_f16, one block per K step.
#include <cstdlib>
#include <string>
#include <type_traits>

#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

typedef uint32_t u32x4a4_g __attribute__((ext_vector_type(4), aligned(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// dequantization of one pair (64 weights of one row) into 8 chunks of 8 fp16

__device__ __forceinline__ half2v h2_of(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t u32_of(half2v h) { return __builtin_bit_cast(uint32_t, h); }

// Q4_0 code dword q (bytes = qs[4t..4t+3]) -> fp16 weights of elements
// 4t..4t+3 (lo[0..1]) and 16+4t..16+4t+3 (hi[0..1]), each RNE(d*(n-8)).
__device__ __forceinline__ void q4_word_f16(uint32_t q, half2v d2, uint32_t lo[2], uint32_t hi[2]) {
  const uint32_t l = q & 0x0F0F0F0Fu;
  const uint32_t h = (q >> 4) & 0x0F0F0F0Fu;
  const half2v off = {(half_t)-1032.f, (half_t)-1032.f};
  lo[0] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, l, 0x04010400u)) + off) * d2);
  lo[1] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, l, 0x04030402u)) + off) * d2);
  hi[0] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, h, 0x04010400u)) + off) * d2);
  hi[1] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, h, 0x04030402u)) + off) * d2);
}

// Q8_0 code dword (4 signed codes) -> 2 fp16x2 = RNE(d*q).
__device__ __forceinline__ void q8_word_f16(uint32_t q, half2v d2, uint32_t out[2]) {
  const uint32_t u = q ^ 0x80808080u;  // code + 128
  const half2v off = {(half_t)-1152.f, (half_t)-1152.f};
  out[0] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + off) * d2);
  out[1] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + off) * d2);
}

template <class QF> struct GPair;
template <> struct GPair<Q4_0> {
  static constexpr int kBytes = 36, kDwords = 9;
};
template <> struct GPair<Q8_0> {
  static constexpr int kBytes = 68, kDwords = 17;
};

template <class QF>
__device__ __forceinline__ void gload_pair(const uint8_t* p, uint32_t (&w)[GPair<QF>::kDwords]) {
  const u32x4a4_g* v = reinterpret_cast<const u32x4a4_g*>(p);
#pragma unroll
  for (int i = 0; i < GPair<QF>::kDwords / 4; ++i) {
    const u32x4 t = v[i];
    w[4 * i + 0] = t.x;
    w[4 * i + 1] = t.y;
    w[4 * i + 2] = t.z;
    w[4 * i + 3] = t.w;
  }
  w[GPair<QF>::kDwords - 1] = reinterpret_cast<const uint32_t*>(p)[GPair<QF>::kDwords - 1];
}

// 64 fp16 weights (natural element order) of a loaded pair, as 32 dwords.
template <class QF>
__device__ __forceinline__ void dequant_pair_f16(const uint32_t (&w)[GPair<QF>::kDwords], uint32_t (&o)[32]);

template <>
__device__ __forceinline__ void dequant_pair_f16<Q4_0>(const uint32_t (&w)[9], uint32_t (&o)[32]) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const uint32_t db = blk == 0 ? (w[0] & 0xFFFFu) : (w[4] >> 16);
    const half2v d2 = h2_of(db | (db << 16));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t q = blk == 0 ? __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2) : w[5 + t];
      uint32_t lo[2], hi[2];
      q4_word_f16(q, d2, lo, hi);
      // elements 4t..4t+3 -> dwords 2t, 2t+1; 16+4t.. -> dwords 8+2t, 8+2t+1
      o[blk * 16 + 2 * t + 0] = lo[0];
      o[blk * 16 + 2 * t + 1] = lo[1];
      o[blk * 16 + 8 + 2 * t + 0] = hi[0];
      o[blk * 16 + 8 + 2 * t + 1] = hi[1];
    }
  }
}

template <>
__device__ __forceinline__ void dequant_pair_f16<Q8_0>(const uint32_t (&w)[17], uint32_t (&o)[32]) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const uint32_t db = blk == 0 ? (w[0] & 0xFFFFu) : (w[8] >> 16);
    const half2v d2 = h2_of(db | (db << 16));
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint32_t q = blk == 0 ? __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2) : w[9 + t];
      uint32_t v[2];
      q8_word_f16(q, d2, v);
      o[blk * 16 + 2 * t + 0] = v[0];
      o[blk * 16 + 2 * t + 1] = v[1];
    }
  }
}

// 32 fp16 weights (natural element order) of block `h` (0 or 1) of a loaded pair.
template <class QF>
__device__ __forceinline__ void dequant_block_f16(const uint32_t (&w)[GPair<QF>::kDwords], int h,
                                                  uint32_t (&o)[16]);

template <>
__device__ __forceinline__ void dequant_block_f16<Q4_0>(const uint32_t (&w)[9], int h, uint32_t (&o)[16]) {
  const uint32_t db = h == 0 ? (w[0] & 0xFFFFu) : (w[4] >> 16);
  const half2v d2 = h2_of(db | (db << 16));
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t q = h == 0 ? __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2) : w[5 + t];
    uint32_t lo[2], hi[2];
    q4_word_f16(q, d2, lo, hi);
    o[2 * t + 0] = lo[0];
    o[2 * t + 1] = lo[1];
    o[8 + 2 * t + 0] = hi[0];
    o[8 + 2 * t + 1] = hi[1];
  }
}

template <>
__device__ __forceinline__ void dequant_block_f16<Q8_0>(const uint32_t (&w)[17], int h, uint32_t (&o)[16]) {
  const uint32_t db = h == 0 ? (w[0] & 0xFFFFu) : (w[8] >> 16);
  const half2v d2 = h2_of(db | (db << 16));
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t q = h == 0 ? __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2) : w[9 + t];
    uint32_t v[2];
    q8_word_f16(q, d2, v);
    o[2 * t + 0] = v[0];
    o[2 * t + 1] = v[1];
  }
}

// Half of block `h`'s code words (part 0: the first half, part 1: the
// second) -> their fp16 weights in o[] (same positions as dequant_block_f16).
template <class QF>
__device__ __forceinline__ void dequant_block_part_f16(const uint32_t (&w)[GPair<QF>::kDwords], int h,
                                                       int part, uint32_t (&o)[16]);

template <>
__device__ __forceinline__ void dequant_block_part_f16<Q4_0>(const uint32_t (&w)[9], int h, int part,
                                                             uint32_t (&o)[16]) {
  const uint32_t db = h == 0 ? (w[0] & 0xFFFFu) : (w[4] >> 16);
  const half2v d2 = h2_of(db | (db << 16));
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int t = part * 2 + tt;
    const uint32_t q = h == 0 ? __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2) : w[5 + t];
    uint32_t lo[2], hi[2];
    q4_word_f16(q, d2, lo, hi);
    o[2 * t + 0] = lo[0];
    o[2 * t + 1] = lo[1];
    o[8 + 2 * t + 0] = hi[0];
    o[8 + 2 * t + 1] = hi[1];
  }
}

template <>
__device__ __forceinline__ void dequant_block_part_f16<Q8_0>(const uint32_t (&w)[17], int h, int part,
                                                             uint32_t (&o)[16]) {
  const uint32_t db = h == 0 ? (w[0] & 0xFFFFu) : (w[8] >> 16);
  const half2v d2 = h2_of(db | (db << 16));
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int t = part * 4 + tt;
    const uint32_t q = h == 0 ? __builtin_amdgcn_alignbyte(w[t + 1], w[t], 2) : w[9 + t];
    uint32_t v[2];
    q8_word_f16(q, d2, v);
    o[2 * t + 0] = v[0];
    o[2 * t + 1] = v[1];
  }
}

// ---------------------------------------------------------------------------
// tiled MFMA kernel

constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;  // halves per LDS row (144 B)

// W staging per thread: one 32-element block of a row's pair.  Block h of
// a Q4_0 pair lives in dwords 4h..4h+4 (5 dwords), of a Q8_0 pair in dwords
// 8h..8h+8 (9 dwords); both windows start on a 4-byte boundary.
template <class QF> struct WBlk;
template <> struct WBlk<Q4_0> {
  static constexpr int kDwords = 5, kStride = 4, kLoads = 2;  // kLoads: load instructions
};
template <> struct WBlk<Q8_0> {
  static constexpr int kDwords = 9, kStride = 8, kLoads = 3;
};
// Dense fp16 B ([N,K] halves): streamed into LDS like A, no register staging.
struct F16B {};
template <> struct GPair<F16B> {
  static constexpr int kBytes = 128, kDwords = 32;
};
template <> struct WBlk<F16B> {
  static constexpr int kDwords = 1, kStride = 0, kLoads = 0;
};

template <class QF>
__device__ __forceinline__ void load_wblk(const uint8_t* p, uint32_t (&w)[WBlk<QF>::kDwords]) {
  const u32x4a4_g* v = reinterpret_cast<const u32x4a4_g*>(p);
#pragma unroll
  for (int i = 0; i < WBlk<QF>::kDwords / 4; ++i) {
    const u32x4 t = v[i];
    w[4 * i + 0] = t.x;
    w[4 * i + 1] = t.y;
    w[4 * i + 2] = t.z;
    w[4 * i + 3] = t.w;
  }
  w[WBlk<QF>::kDwords - 1] = reinterpret_cast<const uint32_t*>(p)[WBlk<QF>::kDwords - 1];
}

// fp16 weights of the loaded block in natural element order, 16 dwords.
// The thread's window starts 0 (h = 0) or 2 (h = 1) bytes before the block's
// scale, so code dword t is bytes 2+2h+4t.. of the window: one v_perm with a
// per-thread selector `sel` (0x05040302 or 0x07060504) extracts it, and
// `sh` (0 or 16) shifts the scale down.  `valid` = false zeroes the scale,
// and with it the block (rows past N).
template <class QF>
__device__ __forceinline__ void dequant_wblk(const uint32_t (&w)[WBlk<QF>::kDwords], uint32_t sel, uint32_t sh,
                                             bool valid, uint32_t (&o)[16]);

template <>
__device__ __forceinline__ void dequant_wblk<Q4_0>(const uint32_t (&w)[5], uint32_t sel, uint32_t sh, bool valid,
                                                   uint32_t (&o)[16]) {
  uint32_t db = (w[0] >> sh) & 0xFFFFu;
  db = valid ? db : 0u;
  const half2v d2 = h2_of(db | (db << 16));
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t q = __builtin_amdgcn_perm(w[t + 1], w[t], sel);
    uint32_t lo[2], hi[2];
    q4_word_f16(q, d2, lo, hi);
    o[2 * t + 0] = lo[0];
    o[2 * t + 1] = lo[1];
    o[8 + 2 * t + 0] = hi[0];
    o[8 + 2 * t + 1] = hi[1];
  }
}

template <>
__device__ __forceinline__ void dequant_wblk<Q8_0>(const uint32_t (&w)[9], uint32_t sel, uint32_t sh, bool valid,
                                                   uint32_t (&o)[16]) {
  uint32_t db = (w[0] >> sh) & 0xFFFFu;
  db = valid ? db : 0u;
  const half2v d2 = h2_of(db | (db << 16));
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const uint32_t q = __builtin_amdgcn_perm(w[t + 1], w[t], sel);
    uint32_t v[2];
    q8_word_f16(q, d2, v);
    o[2 * t + 0] = v[0];
    o[2 * t + 1] = v[1];
  }
}

// 16 bytes per lane, global -> LDS without registers (global_load_lds_dwordx4):
// lane i of the wave writes lds_base + 16*i.  The builtin only exists in the
// device pass; the host pass must not see it or the kernel stub is dropped.
__device__ __forceinline__ void lds_dma16(const void* g, void* lds_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(g, lds_base, 16, 0, 0);
#endif
}

// LDS tile layout: rows of 64 halves (128 B, no padding); the 16-B chunk c of
// row r sits at chunk slot c ^ ((r >> 1) & 7).  The 16 lanes of one
// ds_read_b128 phase (16 consecutive rows, same chunk) then cover all 16
// 16-B positions of the 256-B bank window, and a wave's direct-to-LDS load
// (64 lanes x 16 B, contiguous) fills 8 whole rows.
__device__ __forceinline__ int tile_off(int r, int c) { return r * 64 + ((c ^ ((r >> 1) & 7)) << 3); }

// Workgroup -> output tile, XCD-aware.  The dispatcher hands consecutive
// workgroup ids to the 8 XCDs in turn, and each XCD has its own L2.  The
// tiles are enumerated in groups of GM M-tiles (N-tile outer, M-tile inner,
// GM = max(1, M-tiles / 8)), and that sequence is cut into 8 contiguous
// pieces, one per XCD: an XCD then works on about 1/8 of the activation rows
// against a sweep of weight tiles, so its activation rows stay in its L2 and
// each weight tile is fetched about once per XCD.
__device__ __forceinline__ void xcd_tile(int bid, int mt, int nt, int& tm, int& tn) {
  constexpr int kXcd = 8;
  const int total = mt * nt;
  const int per = (total + kXcd - 1) / kXcd;  // tiles of the larger pieces
  const int tall = total - (per - 1) * kXcd;   // number of larger pieces
  const int x = bid % kXcd, j = bid / kXcd;
  const int pid = x < tall ? x * per + j : tall * per + (x - tall) * (per - 1) + j;
  const int gm = mt / kXcd > 1 ? mt / kXcd : 1;
  const int group = pid / (gm * nt), within = pid - group * gm * nt;
  const int rows = mt - group * gm < gm ? mt - group * gm : gm;
  tm = group * gm + within % rows;
  tn = within / rows;
}

// Split-K fix-up of the last workgroup to arrive at a tile: every workgroup
// of the tile (this one included) has parked its fp32 partial tile in
// `tile_ws` (partial g at float4 offset g * stride; values 4q..4q+3 of tile
// (i, j) of thread tid at ((i*TN + j)*4 + q)*NT + tid).  Their sum, in order
// g = 0..KG-1 whichever workgroup arrives last, replaces acc.  All of one
// partial's loads for CH tiles of TM are issued before any is added, so a
// thread keeps 4*TN*CH loads in flight: the gather costs about KG*TM/CH
// memory round trips, not one per 16-byte group.
template <int TM, int TN, int NT, int CH>
__device__ __forceinline__ void splitk_gather(float16v (&acc)[TM][TN], const CoherentTile& tile_ws,
                                              uint32_t stride, int KG, int tid) {
  static_assert(TM % CH == 0, "chunks of whole tile rows");
#pragma unroll
  for (int i0 = 0; i0 < TM; i0 += CH) {
    for (int g = 0; g < KG; ++g) {
      float4v p[CH][TN][4];
#pragma unroll
      for (int ii = 0; ii < CH; ++ii)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            p[ii][j][q] = tile_ws.load((uint32_t)g * stride + (((i0 + ii) * TN + j) * 4 + q) * NT + tid);
#pragma unroll
      for (int ii = 0; ii < CH; ++ii)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              acc[i0 + ii][j][4 * q + e] = g == 0 ? p[ii][j][q][e] : acc[i0 + ii][j][4 * q + e] + p[ii][j][q][e];
    }
  }
}

// CTA tile BM x BN, WGM x WGN waves, each owning (BM/WGM) x (BN/WGN) =
// TM x TN tiles of 32x32; K step 64, two LDS stages.
//
// Per K step s (LDS stage s&1):
//   * A rows for step s+1 stream straight into the other stage with
//     global_load_lds_dwordx4 (no registers, no VALU);
//   * W blocks for step s+2 are fetched into one of two register sets;
//   * the MFMAs of step s run from LDS;
//   * W of step s+1 (fetched one step earlier) is dequantized to fp16 and
//     written into the other stage;
//   * one barrier.
template <class QF, int BM, int BN, int WGM, int WGN, int NS, bool SPLIT, typename CT = half_t>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_tile_kernel(const half_t* __restrict__ A,
                                                                    const uint8_t* __restrict__ W,
                                                                    CT* __restrict__ C, int M,
                                                                    int N, int K,
                                                                    float* __restrict__ ws_part,
                                                                    uint32_t* __restrict__ ws_cnt) {
  constexpr int NWAVE = WGM * WGN;
  constexpr int NT = 64 * NWAVE;
  constexpr int TM = BM / WGM / 32, TN = BN / WGN / 32;
  constexpr int A_DMA = BM / 8 / NWAVE;  // direct-to-LDS loads (8 rows each) per wave per step
  constexpr int STAGE = (BM + BN) * 64;  // halves
  static_assert(NS == 2 || NS == 3, "two or three LDS stages");
  constexpr int WD = WBlk<QF>::kDwords;
  static_assert(BM % (8 * NWAVE) == 0, "A rows per wave");
  static_assert(BN * 2 <= NT || WBlk<QF>::kLoads == 0, "W staging: one block per thread");
  extern __shared__ __attribute__((aligned(16))) half_t lds[];  // [2][A rows | B rows][64]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = (wave / WGN) * (BM / WGM), wn = (wave % WGN) * (BN / WGN);
  int tm, tn;
  xcd_tile(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // Split K: the KG = gridDim.y workgroups of a tile take contiguous ranges
  // of K steps.
  const int KG = SPLIT ? (int)gridDim.y : 1, kg = SPLIT ? (int)blockIdx.y : 0;
  const int nk_all = K / kBK;
  const int k_first = (int)((long)nk_all * kg / KG);
  const int nk = (int)((long)nk_all * (kg + 1) / KG) - k_first;

  // A: lane -> (row within its 8-row group, chunk slot); the global chunk is
  // the one the swizzle places in that slot.  Rows past M read row M-1
  // (their outputs are never stored).
  const half_t* asrc[A_DMA];
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    const int r = (wave * A_DMA + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int gr = m0 + r < M ? m0 + r : M - 1;
    asrc[i] = A + (size_t)gr * K + (size_t)k_first * kBK + c * 8;
  }
  // Dense fp16 B: rows stream into LDS with the same mapping as A; rows past
  // N read row N-1 (their outputs are never stored).
  constexpr bool kDenseB = WBlk<QF>::kLoads == 0;
  constexpr int B_DMA = kDenseB ? BN / 8 / NWAVE : 0;
  const half_t* bsrc[B_DMA > 0 ? B_DMA : 1];
  if constexpr (kDenseB) {
    static_assert(BN % (8 * NWAVE) == 0, "B rows per wave");
    const half_t* Bh = reinterpret_cast<const half_t*>(W);
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
      const int r = (wave * B_DMA + i) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int gr = n0 + r < N ? n0 + r : N - 1;
      bsrc[i] = Bh + (size_t)gr * K + (size_t)k_first * kBK + c * 8;
    }
  }
  // W: thread -> (row, block); extra threads duplicate a row (identical
  // writes).  Block h's window starts at dword h * kStride of the pair: the
  // scale is then in its low (h = 0) or high (h = 1) half of window dword 0.
  const int w_row = (tid >> 1) % BN, w_half = tid & 1;
  const bool w_valid = n0 + w_row < N;
  const uint32_t w_sel = w_half ? 0x07060504u : 0x05040302u, w_sh = w_half ? 16u : 0u;
  const uint8_t* wsrc = nullptr;
  if constexpr (!kDenseB) {
    const size_t row_bytes = (size_t)(K / 64) * GPair<QF>::kBytes;
    wsrc = W + (size_t)(w_valid ? n0 + w_row : 0) * row_bytes + (size_t)k_first * GPair<QF>::kBytes +
           w_half * 4 * WBlk<QF>::kStride;
  }

  auto dma_a = [&](int ks, int buf) {
    half_t* dst = lds + (size_t)buf * STAGE;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i)
      lds_dma16(asrc[i] + (size_t)ks * kBK, dst + (wave * A_DMA + i) * 8 * 64);
    if constexpr (kDenseB) {
#pragma unroll
      for (int i = 0; i < B_DMA; ++i)
        lds_dma16(bsrc[i] + (size_t)ks * kBK, dst + (BM + (wave * B_DMA + i) * 8) * 64);
    }
  };
  auto load_w = [&](int ks, uint32_t (&w)[WD]) {
    if constexpr (!kDenseB) load_wblk<QF>(wsrc + (size_t)ks * GPair<QF>::kBytes, w);
  };
  auto stage_w = [&](int buf, const uint32_t (&w)[WD]) {
    if constexpr (!kDenseB) {
      uint32_t o[16];
      dequant_wblk<QF>(w, w_sel, w_sh, w_valid, o);
      half_t* Bs = lds + (size_t)buf * STAGE + BM * 64;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 v = {o[4 * c + 0], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]};
        *reinterpret_cast<u32x4*>(Bs + tile_off(w_row, w_half * 4 + c)) = v;
      }
    }
  };

  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};

  const int r32 = lane & 31, kc = lane >> 5;  // operand row, k-chunk within a 16-k slice
  auto compute = [&](int buf) {
    const half_t* As = lds + (size_t)buf * STAGE;
    const half_t* Bs = As + BM * 64;
    half8 a[2][TM], b[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[0][i] = *reinterpret_cast<const half8*>(As + tile_off(wm + 32 * i + r32, kc));
#pragma unroll
    for (int j = 0; j < TN; ++j) b[0][j] = *reinterpret_cast<const half8*>(Bs + tile_off(wn + 32 * j + r32, kc));
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int cur = kk & 1;
      if (kk + 1 < kBK / 16) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          a[cur ^ 1][i] = *reinterpret_cast<const half8*>(As + tile_off(wm + 32 * i + r32, 2 * (kk + 1) + kc));
#pragma unroll
        for (int j = 0; j < TN; ++j)
          b[cur ^ 1][j] = *reinterpret_cast<const half8*>(Bs + tile_off(wn + 32 * j + r32, 2 * (kk + 1) + kc));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[cur][i], b[cur][j], acc[i][j], 0, 0, 0);
    }
  };
  // Order for the scheduler: the first slice's operand reads, then per slice
  // the next slice's reads ahead of this slice's MFMAs, so the MFMA pipe
  // always has a slice queued while operands load; VALU work of the step
  // (the weight dequantization) is spread over the MFMA issue shadow, and the
  // dequantized weights' LDS writes go last.
  constexpr int kMfma = TM * TN * (kBK / 16);
  constexpr int kValuPerMfma = (72 + kMfma - 1) / kMfma;
  auto schedule = [&]() {
    __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      if (kk + 1 < kBK / 16) __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0);
#pragma unroll
      for (int m = 0; m < TM * TN; ++m) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (!kDenseB) __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);
      }
    }
    if constexpr (!kDenseB) __builtin_amdgcn_sched_group_barrier(0x200, 4, 0);
  };

  // Loads are unconditional (step indices clamped to the last step): a
  // conditional load into a register set would force a copy, and the copy a
  // wait for every outstanding load.  Past the end, the extra loads and
  // stores only touch idle stages.  A runs NS-1 steps ahead in the LDS ring;
  // W runs two steps ahead in registers and is staged one step ahead.
  uint32_t wr[2][WD] = {};
#pragma unroll
  for (int i = 0; i < NS - 1; ++i) dma_a(i < nk ? i : nk - 1, i);
  load_w(0, wr[0]);
  load_w(nk > 1 ? 1 : 0, wr[1]);
  stage_w(0, wr[0]);
  __syncthreads();

  // End-of-step barrier: this wave's LDS writes and its A loads for the next
  // step must be complete; loads issued during this step for later steps
  // (the W loads, and with three stages the A loads for step s+2) may stay
  // in flight.  __syncthreads() would wait for every outstanding load.
  constexpr int kInFlight = WBlk<QF>::kLoads + (NS == 3 ? A_DMA + B_DMA : 0);
  auto step_barrier = [&]() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kInFlight) : "memory");
  };
  auto half_step = [&](int s, uint32_t (&wload)[WD], const uint32_t (&wstage)[WD]) {
    const int ahead = s + NS - 1;
    dma_a(ahead < nk ? ahead : nk - 1, ahead % NS);
    __builtin_amdgcn_sched_barrier(0);
    load_w(s + 2 < nk ? s + 2 : nk - 1, wload);  // wload held W(s), staged last step
    __builtin_amdgcn_sched_barrier(0);
    compute(s % NS);
    stage_w((s + 1) % NS, wstage);  // W(s+1), dequantized in the MFMA shadow
    schedule();
    __builtin_amdgcn_sched_barrier(0);
    step_barrier();
  };
  int ks = 0;
  for (; ks + 1 < nk; ks += 2) {
    half_step(ks, wr[0], wr[1]);
    half_step(ks + 1, wr[1], wr[0]);
  }
  if (ks < nk) half_step(ks, wr[0], wr[1]);

  // epilogue: round to fp16 and store
  const int col = lane & 31, rq = (lane >> 5) * 4;
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int gn = n0 + wn + 32 * j + col;
        if (gn >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gm = m0 + wm + 32 * i + (r >> 2) * 8 + rq + (r & 3);
          if (gm < M) C[(size_t)gm * N + gn] = (CT)acc[i][j][r];
        }
      }
  };
  if constexpr (!SPLIT) {
    store();
    return;
  }
  // Split K across workgroups: each parks its fp32 accumulators in the
  // workspace as 16-byte groups (values 4q..4q+3 of tile (i, j) of thread
  // tid at float4 index ((i*TN + j)*4 + q)*NT + tid, coalesced per wave);
  // the last workgroup of the tile to arrive (per-tile counter; the partials
  // move through sc1 accesses, CoherentTile) adds the KG partial tiles in
  // order kg = 0..KG-1 (splitk_gather), stores C and resets the counter.
  const int tile = blockIdx.x;
  const CoherentTile tile_ws(reinterpret_cast<float4v*>(ws_part) + (size_t)tile * KG * (BM * BN / 4),
                             (uint32_t)(KG * BM * BN * 4));
  {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          tile_ws.store((uint32_t)kg * (BM * BN / 4) + ((i * TN + j) * 4 + q) * NT + tid,
                        float4v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ uint32_t is_last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ws_cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == (uint32_t)(KG - 1);
  }
  __syncthreads();
  if (!is_last) return;
  splitk_gather<TM, TN, NT, (TM % 2 == 0 && TM * TN >= 8) ? TM / 2 : TM>(acc, tile_ws, BM * BN / 4, KG, tid);
  store();
  if (tid == 0) __hip_atomic_store(&ws_cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// quantized-W tiled kernel: weights dequantized in registers, A through LDS
//
// Each wave owns a 32*TM (M) x 32*TN (N) output tile; the NW waves of a
// workgroup sit side by side along N and share one BM = 32*TM row block of
// A in LDS.  The weights never touch LDS: lane (n = l%32, kb = l/32) loads,
// for each of its TN weight rows, block kb of the step's Q4_0/Q8_0 pair
// (5 / 9 dwords, dword-aligned window) PF steps ahead and dequantizes it to
// 32 fp16 values one step ahead.
//
// K order inside a step: the MFMA sums over its 16 k slots, so any
// permutation of the step's 64 k values that A and W share gives the same
// sum.  Slice kk (0..3) pairs slot group kb with elements 8kk..8kk+7 of
// block kb, i.e. step offset 32*kb + 8*kk: the weight operand is then dwords
// 4kk..4kk+3 of the lane's own dequantized block, and the A operand is the
// 16-B chunk 4*kb + kk of the row.
//
// The weight block is MFMA operand "A" and the activation operand "B", so
// accumulator r of lane l is C[m = l%32][n = (r/4)*8 + (l/32)*4 + r%4]: four
// consecutive columns of one row per r/4, stored as one 8-byte write.
//
// A is prefetched PF steps ahead into registers (16 B per lane per 8 rows)
// and written to a two-stage LDS buffer one step ahead.  Every load has a
// register destination, so the compiler's wait insertion tracks each one
// exactly and waits only for the oldest (direct-to-LDS loads would make it
// drain the whole queue before each use of a weight register).
//
// Per step s (LDS stage s & 1):
//   * slices 0-2: operand reads of the next slice, then this slice's MFMAs;
//     in their shadow: W(s+1) dequantized, A(s+1) written to stage
//     (s+1) & 1, and W(s+PF), A(s+PF) loaded;
//   * one barrier (every wave's A(s+1) writes are done and every wave has
//     read its last operands from stage s & 1);
//   * slice 0 of step s+1 is read, and the slice-3 MFMAs of step s
//     (operands already in registers) run.
template <class QF, int TM, int TN, int NW, int PF, bool SPLIT>
__global__ __launch_bounds__(64 * NW, 1) void gemm_wq_kernel(const half_t* __restrict__ A,
                                                             const uint8_t* __restrict__ W,
                                                             half_t* __restrict__ C, int M, int N, int K,
                                                             float* __restrict__ ws_part,
                                                             uint32_t* __restrict__ ws_cnt) {
  constexpr int BM = 32 * TM, BN = 32 * TN * NW, NT = 64 * NW;
  constexpr int STAGE = BM * 64;      // halves per LDS stage
  constexpr int A_LD = BM / 8 / NW;   // 16-B A loads per lane per step
  constexpr int WD = WBlk<QF>::kDwords;
  static_assert(PF == 2 || PF == 4, "even prefetch depth (register sets alternate by step parity)");
  static_assert(BM % (8 * NW) == 0, "A rows per wave");
  extern __shared__ __attribute__((aligned(16))) half_t lds[];  // [2][BM][64]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, kb = lane >> 5;
  int tm, tn;
  xcd_tile(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN, wn = wave * 32 * TN;
  const int KG = SPLIT ? (int)gridDim.y : 1, kg = SPLIT ? (int)blockIdx.y : 0;
  const int nk_all = K / kBK;
  const int k_first = (int)((long)nk_all * kg / KG);
  const int nk = (int)((long)nk_all * (kg + 1) / KG) - k_first;

  // A: load i of a lane covers row (wave*A_LD + i)*8 + l/8, chunk l%8 (eight
  // lanes read one row's 128 B).  Rows past M read row M-1 (their outputs
  // are never stored).
  const half_t* asrc[A_LD];
  int adst[A_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int r = (wave * A_LD + i) * 8 + (lane >> 3);
    const int gr = m0 + r < M ? m0 + r : M - 1;
    asrc[i] = A + (size_t)gr * K + (size_t)k_first * kBK + (lane & 7) * 8;
    adst[i] = tile_off(r, lane & 7);
  }
  // W: frag j of this lane is row n0 + wn + 32j + r32, block kb of each pair.
  // Rows past N read row 0 with the scale forced to zero.
  const size_t row_bytes = (size_t)(K / 64) * GPair<QF>::kBytes;
  const uint32_t w_sel = kb ? 0x07060504u : 0x05040302u, w_sh = kb ? 16u : 0u;
  const uint8_t* wsrc[TN];
  bool w_valid[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn + 32 * j + r32;
    w_valid[j] = n < N;
    wsrc[j] = W + (size_t)(w_valid[j] ? n : 0) * row_bytes + (size_t)k_first * GPair<QF>::kBytes +
              kb * 4 * WBlk<QF>::kStride;
  }

  u32x4 ra[PF][A_LD];
  auto load_a = [&](int ks, int set) {
#pragma unroll
    for (int i = 0; i < A_LD; ++i) ra[set][i] = *reinterpret_cast<const u32x4*>(asrc[i] + (size_t)ks * kBK);
  };
  auto write_a = [&](int set, int stage) {
    half_t* dst = lds + stage * STAGE;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) *reinterpret_cast<u32x4*>(dst + adst[i]) = ra[set][i];
  };
  uint32_t wr[PF][TN][WD];
  auto load_w = [&](int ks, int set) {
#pragma unroll
    for (int j = 0; j < TN; ++j) load_wblk<QF>(wsrc[j] + (size_t)ks * GPair<QF>::kBytes, wr[set][j]);
  };
  uint32_t bq[2][TN][16];
  auto dequant = [&](int set, int buf) {
#pragma unroll
    for (int j = 0; j < TN; ++j) dequant_wblk<QF>(wr[set][j], w_sel, w_sh, w_valid[j], bq[buf][j]);
  };
  half8 af[2][TM];
  auto read_a = [&](int stage, int kk, int buf) {
    const half_t* As = lds + stage * STAGE;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      af[buf][i] = *reinterpret_cast<const half8*>(As + tile_off(32 * i + r32, 4 * kb + kk));
  };
  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};
  auto mfma = [&](int kk, int abuf, int wbuf) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const u32x4 wv = {bq[wbuf][j][4 * kk + 0], bq[wbuf][j][4 * kk + 1], bq[wbuf][j][4 * kk + 2],
                          bq[wbuf][j][4 * kk + 3]};
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, wv), af[abuf][i], acc[i][j],
                                                           0, 0, 0);
      }
  };
  // LDS operations of this wave done, then barrier.  The s_waitcnt builtin
  // (lgkmcnt(0), vmcnt and expcnt untouched) is visible to the compiler's
  // wait insertion; the empty asm statements keep memory accesses in place.
  auto lds_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: loads of steps 0..PF-1 (clamped: loads past the last step
  // re-read it and are never used).
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    load_w(i < nk ? i : nk - 1, i);
    load_a(i < nk ? i : nk - 1, i);
  }
  write_a(0, 0);
  dequant(0, 0);
  lds_barrier();
  read_a(0, 0, 0);

  // Issue order of a step, fixed slot by slot (sched_barrier between
  // slots).  A wave stalls at issue when the vector-memory queue is full,
  // and with one wave per SIMD nothing else feeds the MFMA pipe meanwhile;
  // left alone the compiler bunches the loads and the dequantization VALU.
  // So each MFMA is followed by at most one small piece of other work, about
  // as much VALU as fits in the issue shadow of one 32-cycle MFMA (six):
  //   slices 0-2 (MFMA idx 0..23): idx % 3 == 1: one global load of step
  //     s+PF; idx 14, 17, 20, 23: one LDS write of A(s+1); otherwise one
  //     dequantization piece of W(s+1);
  //   slice 3 (after the barrier, MFMA m 0..7): m < 4: dequantization
  //     pieces; m = 4, 5: the remaining loads (Q8_0 has ten).
  // A piece is half of one Q4_0 code dword (four weights) or one Q8_0 code
  // dword (four weights): 16 per step.
  static_assert(TM == 4 && TN == 2, "slot plan below is laid out for 4x2 tiles per wave");
  static_assert(A_LD == 4 && TN * WBlk<QF>::kLoads + A_LD <= 10, "slot plan: at most 10 loads, 4 LDS writes");
  constexpr bool kQ4 = std::is_same<QF, Q4_0>::value;
  half2v dscale[TN];
  uint32_t qword[TN];
  auto dequant_piece = [&](int set, int buf, int piece) {
    const int j = piece / 8;
    const int t = kQ4 ? (piece / 2) % 4 : piece % 8;  // code dword within the block
    if (piece % 8 == 0) {
      uint32_t db = (wr[set][j][0] >> w_sh) & 0xFFFFu;
      db = w_valid[j] ? db : 0u;
      dscale[j] = h2_of(db | (db << 16));
    }
    if constexpr (kQ4) {
      const half2v off = {(half_t)-1032.f, (half_t)-1032.f};
      if (piece % 2 == 0) {
        qword[j] = __builtin_amdgcn_perm(wr[set][j][t + 1], wr[set][j][t], w_sel);
        const uint32_t l = qword[j] & 0x0F0F0F0Fu;
        bq[buf][j][2 * t + 0] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, l, 0x04010400u)) + off) * dscale[j]);
        bq[buf][j][2 * t + 1] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, l, 0x04030402u)) + off) * dscale[j]);
      } else {
        const uint32_t h = (qword[j] >> 4) & 0x0F0F0F0Fu;
        bq[buf][j][8 + 2 * t + 0] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, h, 0x04010400u)) + off) * dscale[j]);
        bq[buf][j][8 + 2 * t + 1] = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, h, 0x04030402u)) + off) * dscale[j]);
      }
    } else {
      const uint32_t q = __builtin_amdgcn_perm(wr[set][j][t + 1], wr[set][j][t], w_sel);
      uint32_t v[2];
      q8_word_f16(q, dscale[j], v);
      bq[buf][j][2 * t + 0] = v[0];
      bq[buf][j][2 * t + 1] = v[1];
    }
  };
  auto load_piece = [&](int ks, int set, int piece) {
    constexpr int kWl = TN * WBlk<QF>::kLoads;
    if (piece < kWl) {
      const int j = piece / WBlk<QF>::kLoads, part = piece % WBlk<QF>::kLoads;
      const uint8_t* p = wsrc[j] + (size_t)ks * GPair<QF>::kBytes;
      if (part < WBlk<QF>::kDwords / 4) {
        const u32x4 t = reinterpret_cast<const u32x4a4_g*>(p)[part];
        wr[set][j][4 * part + 0] = t.x;
        wr[set][j][4 * part + 1] = t.y;
        wr[set][j][4 * part + 2] = t.z;
        wr[set][j][4 * part + 3] = t.w;
      } else {
        wr[set][j][WD - 1] = reinterpret_cast<const uint32_t*>(p)[WD - 1];
      }
    } else if (piece < kWl + A_LD) {
      const int i = piece - kWl;
      ra[set][i] = *reinterpret_cast<const u32x4*>(asrc[i] + (size_t)ks * kBK);
    }
  };
  auto mfma_one = [&](int kk, int i, int j, int abuf, int wbuf) {
    const u32x4 wv = {bq[wbuf][j][4 * kk + 0], bq[wbuf][j][4 * kk + 1], bq[wbuf][j][4 * kk + 2],
                      bq[wbuf][j][4 * kk + 3]};
    acc[i][j] =
        __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, wv), af[abuf][i], acc[i][j], 0, 0, 0);
  };

  // One K step; u = s % PF (compile time: the loop advances PF steps).
  auto step = [&](auto uc, int s) {
    constexpr int u = decltype(uc)::value;
    constexpr int wb = u & 1;
    const int ks = s + PF < nk ? s + PF : nk - 1;
    int dq = 0;
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
      read_a(wb, kk + 1, (kk + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < TM * TN; ++m) {
        const int idx = kk * TM * TN + m;
        mfma_one(kk, m / TN, m % TN, kk & 1, wb);
        if (idx % 3 == 1) {
          load_piece(ks, u, idx / 3);
        } else if (idx >= 14 && idx % 3 == 2) {
          half_t* dst = lds + (wb ^ 1) * STAGE;
          *reinterpret_cast<u32x4*>(dst + adst[(idx - 14) / 3]) = ra[(u + 1) % PF][(idx - 14) / 3];
        } else {
          dequant_piece((u + 1) % PF, wb ^ 1, dq++);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    lds_barrier();
    read_a(wb ^ 1, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < TM * TN; ++m) {
      mfma_one(3, m / TN, m % TN, 1, wb);
      if (m < 4) dequant_piece((u + 1) % PF, wb ^ 1, dq++);
      if (m == 4 || m == 5) load_piece(ks, u, 8 + (m - 4));
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  int s = 0;
  for (; s + PF <= nk; s += PF) {
    step(std::integral_constant<int, 0>{}, s);
    step(std::integral_constant<int, 1>{}, s + 1);
    if constexpr (PF == 4) {
      step(std::integral_constant<int, 2>{}, s + 2);
      step(std::integral_constant<int, 3>{}, s + 3);
    }
  }
  if (s < nk) step(std::integral_constant<int, 0>{}, s);
  if (s + 1 < nk) step(std::integral_constant<int, 1>{}, s + 1);
  if constexpr (PF == 4) {
    if (s + 2 < nk) step(std::integral_constant<int, 2>{}, s + 2);
  }

  auto store = [&]() {
    const bool vec = (N & 3) == 0 && ((uintptr_t)C & 7) == 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int gm = m0 + 32 * i + r32;
      if (gm >= M) continue;
      half_t* crow = C + (size_t)gm * N;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int gn = n0 + wn + 32 * j + 8 * q + 4 * kb;
          const half_t h0 = (half_t)acc[i][j][4 * q + 0], h1 = (half_t)acc[i][j][4 * q + 1];
          const half_t h2 = (half_t)acc[i][j][4 * q + 2], h3 = (half_t)acc[i][j][4 * q + 3];
          if (vec && gn + 3 < N) {
            typedef _Float16 half4v __attribute__((ext_vector_type(4)));
            *reinterpret_cast<half4v*>(crow + gn) = half4v{h0, h1, h2, h3};
          } else {
            if (gn + 0 < N) crow[gn + 0] = h0;
            if (gn + 1 < N) crow[gn + 1] = h1;
            if (gn + 2 < N) crow[gn + 2] = h2;
            if (gn + 3 < N) crow[gn + 3] = h3;
          }
        }
    }
  };
  if constexpr (!SPLIT) {
    store();
    return;
  }
  // Split K across workgroups: each parks its fp32 accumulators in the
  // workspace as 16-byte groups (values 4q..4q+3 of tile (i, j) of thread tid
  // at float4 index ((i*TN + j)*4 + q)*NT + tid, coalesced per wave); the
  // last workgroup of the tile to arrive (per-tile counter; the partials
  // move through sc1 accesses, CoherentTile) adds the KG partial tiles in
  // order kg = 0..KG-1 (splitk_gather), stores C and resets the counter.
  const int tile = blockIdx.x;
  const CoherentTile tile_ws(reinterpret_cast<float4v*>(ws_part) + (size_t)tile * KG * (BM * BN / 4),
                             (uint32_t)(KG * BM * BN * 4));
  {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          tile_ws.store((uint32_t)kg * (BM * BN / 4) + ((i * TN + j) * 4 + q) * NT + tid,
                        float4v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ uint32_t is_last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ws_cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == (uint32_t)(KG - 1);
  }
  __syncthreads();
  if (!is_last) return;
  splitk_gather<TM, TN, NT, TM>(acc, tile_ws, BM * BN / 4, KG, tid);
  store();
  if (tid == 0) __hip_atomic_store(&ws_cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// two waves per SIMD: gemm_wq2_kernel
//
// The register-dequantizing design of gemm_wq_kernel (weights straight from
// global memory into registers, dequantized there; A through LDS; TM x 2
// v_mfma_f32_32x32x16_f16 tiles per wave, the same K permutation and output
// layout) with two waves on every SIMD (TM = 4, NW = 4: 8 waves, at most 256
// registers each, 128 of them the accumulators), so that one wave's
// load-issue stalls, LDS waits and dequantization VALU run in the shadow of
// the other wave's MFMAs.  The workgroup's 2*NW waves form two K-groups of
// NW: group g takes the second half (g = 1) or the first half of the
// workgroup's K steps for the same 32*TM x 64*NW output tile, with its own
// two-stage A buffer in LDS.  To fit the register budget:
//   * A streams global -> LDS with direct-to-LDS loads (no registers), one
//     step ahead;
//   * the weights are loaded two steps ahead into two register sets and
//     dequantized one MFMA slice (8 halves per fragment) ahead, not a whole
//     step ahead.
// The end-of-step barrier waits for the A loads only (vmcnt = the weight
// loads issued after them), through the s_waitcnt intrinsic so the
// compiler's own wait insertion sees it and does not add a vmcnt(0).
// After the K loop group 1's accumulators are added to group 0's through
// LDS, element by element in that order (deterministic), and group 0 stores
// the tile or, with K split across workgroups as well, parks it for the
// fix-up of gemm_wq_kernel.  (TM = 8 with one wave per SIMD, 256-row waves
// that halve the dequantization per MFMA, measured slower: 693 against 816
// TFLOP/s at 4096 x 4096, M = 2048.)

// Q4_0: the lane's loaded window realigned in place, once per block, so
// w[t] = code dword t (bytes 2+2h+4t.. of the window, h = the block's 2-byte
// misalignment, selected by `sel`); the four slices then read it directly
// (a realignment per slice would redo dwords 0..3 twice).
__device__ __forceinline__ void realign_q4(uint32_t (&w)[WBlk<Q4_0>::kDwords], uint32_t sel) {
#pragma unroll
  for (int t = 0; t < 4; ++t) w[t] = __builtin_amdgcn_perm(w[t + 1], w[t], sel);
}

// Elements 8kk..8kk+7 of the lane's block as 4 dwords of fp16 (the
// dequant_*_f16 bits): Q4_0 low nibbles of code dwords 2(kk&1), 2(kk&1)+1
// for kk < 2, high nibbles for kk >= 2 (w realigned by realign_q4); Q8_0
// code dwords 2kk, 2kk+1 (w as loaded).  A low nibble n goes under exponent
// byte 0x64 (fp16 1024 + n), a high one, masked in place (16n), under 0x54
// (fp16 64 + 16n/16 = 64 + n: unit spacing there), so no shift is needed;
// the packed add of -1032 or -72 leaves n - 8 exactly, and the packed
// multiply rounds d(n - 8) once.
template <class QF>
__device__ __forceinline__ u32x4 dequant_slice(const uint32_t (&w)[WBlk<QF>::kDwords], uint32_t sel, half2v d2,
                                               int kk) {
  u32x4 o;
  if constexpr (std::is_same<QF, Q4_0>::value) {
    const bool hi = (kk >> 1) != 0;
    const half2v off = hi ? half2v{(half_t)-72.f, (half_t)-72.f} : half2v{(half_t)-1032.f, (half_t)-1032.f};
    const uint32_t mask = hi ? 0xF0F0F0F0u : 0x0F0F0F0Fu, expo = hi ? 0x54545454u : 0x64646464u;
    const int t0 = 2 * (kk & 1);
    const uint32_t xa = w[t0] & mask, xb = w[t0 + 1] & mask;
    o.x = u32_of((h2_of(__builtin_amdgcn_perm(expo, xa, 0x04010400u)) + off) * d2);
    o.y = u32_of((h2_of(__builtin_amdgcn_perm(expo, xa, 0x04030402u)) + off) * d2);
    o.z = u32_of((h2_of(__builtin_amdgcn_perm(expo, xb, 0x04010400u)) + off) * d2);
    o.w = u32_of((h2_of(__builtin_amdgcn_perm(expo, xb, 0x04030402u)) + off) * d2);
  } else {
    const half2v off = {(half_t)-1152.f, (half_t)-1152.f};
    const uint32_t ua = __builtin_amdgcn_perm(w[2 * kk + 1], w[2 * kk], sel) ^ 0x80808080u;
    const uint32_t ub = __builtin_amdgcn_perm(w[2 * kk + 2], w[2 * kk + 1], sel) ^ 0x80808080u;
    o.x = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, ua, 0x04010400u)) + off) * d2);
    o.y = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, ua, 0x04030402u)) + off) * d2);
    o.z = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, ub, 0x04010400u)) + off) * d2);
    o.w = u32_of((h2_of(__builtin_amdgcn_perm(0x64646464u, ub, 0x04030402u)) + off) * d2);
  }
  return o;
}

// Dynamic LDS of gemm_wq2_kernel: the four A stages (two per K-group), or,
// if larger, one row of 32x32 tiles of group 1's accumulators for the final
// reduction (2 x 16 floats x 64*NW threads).
constexpr int wq2_lds_bytes(int TM, int NW) {
  return (4 * 32 * TM * 64 * 2) > (2 * 16 * 64 * NW * 4) ? (4 * 32 * TM * 64 * 2) : (2 * 16 * 64 * NW * 4);
}

template <class QF, int TM, int NW, bool SPLIT>
__global__ __launch_bounds__(128 * NW, 1) void gemm_wq2_kernel(const half_t* __restrict__ A,
                                                              const uint8_t* __restrict__ W, half_t* __restrict__ C,
                                                              int M, int N, int K, float* __restrict__ ws_part,
                                                              uint32_t* __restrict__ ws_cnt) {
  constexpr int TN = 2, BM = 32 * TM, BN = 32 * TN * NW, NT0 = 64 * NW;
  constexpr int STAGE = BM * 64;     // halves per LDS stage
  constexpr int A_DMA = BM / 8 / NW;  // direct-to-LDS loads (8 rows each) per wave per step
  static_assert(BM % (8 * NW) == 0 && A_DMA >= 1, "A rows per wave");
  constexpr int WD = WBlk<QF>::kDwords;
  extern __shared__ __attribute__((aligned(16))) half_t lds[];  // [group][2][BM][64]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int grp = wave / NW, wv = wave % NW;
  const int r32 = lane & 31, kb = lane >> 5;
  int tm, tn;
  xcd_tile(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN, wn = wv * 32 * TN;
  // K steps: the KG workgroups of a tile take ranges of whole step pairs;
  // the two groups of a workgroup split its range in halves.
  const int KG = SPLIT ? (int)gridDim.y : 1, kg = SPLIT ? (int)blockIdx.y : 0;
  const int np_all = K / (2 * kBK);
  const int p_first = (int)((long)np_all * kg / KG);
  const int nk = (int)((long)np_all * (kg + 1) / KG) - p_first;  // steps per group
  const int k0 = 2 * p_first + grp * nk;                            // this group's first step

  // A: load i of a lane fills row (wv*A_DMA + i)*8 + l/8 of the stage, slot
  // l%8, with the global chunk the swizzle places in that slot.  Rows past M
  // read row M-1 (their outputs are never stored).
  const half_t* asrc[A_DMA];
#pragma unroll
  for (int i = 0; i < A_DMA; ++i) {
    const int r = (wv * A_DMA + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int gr = m0 + r < M ? m0 + r : M - 1;
    asrc[i] = A + (size_t)gr * K + (size_t)k0 * kBK + c * 8;
  }
  const size_t row_bytes = (size_t)(K / 64) * GPair<QF>::kBytes;
  const uint32_t w_sel = kb ? 0x07060504u : 0x05040302u, w_sh = kb ? 16u : 0u;
  const uint8_t* wsrc[TN];
  bool w_valid[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn + 32 * j + r32;
    w_valid[j] = n < N;
    wsrc[j] = W + (size_t)(w_valid[j] ? n : 0) * row_bytes + (size_t)k0 * GPair<QF>::kBytes + kb * 4 * WBlk<QF>::kStride;
  }
  half_t* my_lds = lds + (size_t)grp * 2 * STAGE;

  uint32_t wr[2][TN][WD];
  auto load_w = [&](int ks, int set) {
#pragma unroll
    for (int j = 0; j < TN; ++j) load_wblk<QF>(wsrc[j] + (size_t)ks * GPair<QF>::kBytes, wr[set][j]);
  };
  auto dma_a = [&](int ks, int stage) {
    half_t* dst = my_lds + stage * STAGE;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) lds_dma16(asrc[i] + (size_t)ks * kBK, dst + (wv * A_DMA + i) * 8 * 64);
  };
  half2v dsc[2][TN];  // fp16 scales of the two register sets' blocks
  // Once a register set has landed: its blocks' scales, and (Q4_0) its code
  // dwords realigned in place.
  auto scales = [&](int set) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      uint32_t db = (wr[set][j][0] >> w_sh) & 0xFFFFu;
      db = w_valid[j] ? db : 0u;
      dsc[set][j] = h2_of(db | (db << 16));
      if constexpr (std::is_same<QF, Q4_0>::value) realign_q4(wr[set][j], w_sel);
    }
  };
  u32x4 bw[2][TN];
  auto dequant = [&](int set, int kk, int buf) {
#pragma unroll
    for (int j = 0; j < TN; ++j) bw[buf][j] = dequant_slice<QF>(wr[set][j], w_sel, dsc[set][j], kk);
  };
  half8 af[2][TM];
  auto read_a = [&](int stage, int kk, int buf) {
    const half_t* As = my_lds + stage * STAGE;
#pragma unroll
    for (int i = 0; i < TM; ++i)
      af[buf][i] = *reinterpret_cast<const half8*>(As + tile_off(32 * i + r32, 4 * kb + kk));
  };
  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};
  auto mfma = [&](int buf) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, bw[buf][j]), af[buf][i],
                                                           acc[i][j], 0, 0, 0);
  };
  // End-of-step barrier: this wave's LDS reads and its A loads for the next
  // step must be complete; the weight loads issued during the step for the
  // step after next (kInFlight instructions, issued after the A loads) may
  // stay in flight.
  constexpr int kInFlight = TN * WBlk<QF>::kLoads;
  // (The wait is the intrinsic, not inline asm, so the compiler's own wait
  // insertion knows the older loads have landed and adds no vmcnt(0).)
  static_assert(kInFlight < 16, "vmcnt field");
  auto step_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0070 | kInFlight);  // vmcnt(kInFlight) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: A of step 0 into stage 0; weights of steps 0 and 1 (past the
  // last step: its loads again, never used) into register sets 0 and 1.
  // The barrier's wait leaves at most kInFlight (one weight set's) loads
  // outstanding, so A, issued first, has landed for every wave.  The
  // compiler may move set 1's loads below the barrier (the loads through the
  // restrict-qualified W are free to cross its empty asm statements); then
  // set 0 is the set left in flight, and the compiler waits for its
  // registers where they are first read.  Either way set 1 is first read
  // after step 0's barrier, whose own wait covers it.  Measured on MI355X
  // against waiting for all three: 4096x4096 M = 2048 875 -> 885 TFLOP/s,
  // 11008x4096 857 -> 874, 4096x4096 M = 512 461 -> 469.
  dma_a(0, 0);
  load_w(0, 0);
  load_w(nk > 1 ? 1 : 0, 1);
  step_barrier();
  scales(0);
  read_a(0, 0, 0);
  dequant(0, 0, 0);

  // Step s (weight register set and LDS stage u = s & 1):
  //   A of step s+1 streams into stage u^1 (read last in step s-1, released
  //   by that step's barrier);
  //   slice kk: read A of slice kk+1 and dequantize its weights, then the
  //   MFMAs of slice kk;
  //   the weights of step s+2 are loaded into set u once its last slice is
  //   dequantized (before the last slice's MFMAs);
  //   barrier; then slice 0 of step s+1 read and dequantized.
  auto step = [&](auto uc, int s) {
    constexpr int u = decltype(uc)::value;
    dma_a(s + 1 < nk ? s + 1 : nk - 1, u ^ 1);  // past the last step: an unused reload
    // The weight loads below must issue after these (the barrier's vmcnt
    // counts them as the only loads younger than the A loads).
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk < 3) {
        read_a(u, kk + 1, (kk + 1) & 1);
        dequant(u, kk + 1, (kk + 1) & 1);
      } else {
        load_w(s + 2 < nk ? s + 2 : nk - 1, u);
      }
      mfma(kk & 1);
    }
    step_barrier();
    if (s + 1 < nk) {
      scales(u ^ 1);
      read_a(u ^ 1, 0, 0);
      dequant(u ^ 1, 0, 0);
    }
  };
  int s = 0;
  for (; s + 2 <= nk; s += 2) {
    step(std::integral_constant<int, 0>{}, s);
    step(std::integral_constant<int, 1>{}, s + 1);
  }
  if (s < nk) step(std::integral_constant<int, 0>{}, s);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Group 1 hands its sums to group 0 through LDS (the stages are free now),
  // RT tiles of TM at a time: value (i, j, r) of thread t at float index
  // ((i' * TN + j) * 16 + r) * NT0 + t (i' = i - round * RT), conflict-free.
  constexpr int RT_FIT = wq2_lds_bytes(TM, NW) / (TN * 16 * NT0 * 4);  // tiles of TM per round that fit
  constexpr int RT = RT_FIT < TM ? RT_FIT : TM;
  static_assert(RT >= 1 && TM % RT == 0, "reduction rounds");
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int rd = 0; rd < TM / RT; ++rd) {
    if (grp == 1) {
#pragma unroll
      for (int ii = 0; ii < RT; ++ii)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            red[((ii * TN + j) * 16 + r) * NT0 + (tid - NT0)] = acc[rd * RT + ii][j][r];
    }
    __syncthreads();
    if (grp == 0) {
#pragma unroll
      for (int ii = 0; ii < RT; ++ii)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[rd * RT + ii][j][r] += red[((ii * TN + j) * 16 + r) * NT0 + tid];
    }
    __syncthreads();
  }

  auto store = [&]() {
    const bool vec = (N & 3) == 0 && ((uintptr_t)C & 7) == 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int gm = m0 + 32 * i + r32;
      if (gm >= M) continue;
      half_t* crow = C + (size_t)gm * N;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int gn = n0 + wn + 32 * j + 8 * q + 4 * kb;
          const half_t h0 = (half_t)acc[i][j][4 * q + 0], h1 = (half_t)acc[i][j][4 * q + 1];
          const half_t h2 = (half_t)acc[i][j][4 * q + 2], h3 = (half_t)acc[i][j][4 * q + 3];
          if (vec && gn + 3 < N) {
            typedef _Float16 half4v __attribute__((ext_vector_type(4)));
            *reinterpret_cast<half4v*>(crow + gn) = half4v{h0, h1, h2, h3};
          } else {
            if (gn + 0 < N) crow[gn + 0] = h0;
            if (gn + 1 < N) crow[gn + 1] = h1;
            if (gn + 2 < N) crow[gn + 2] = h2;
            if (gn + 3 < N) crow[gn + 3] = h3;
          }
        }
    }
  };
  if constexpr (!SPLIT) {
    if (grp == 0) store();
    return;
  }
  // K split across workgroups: group 0 parks its tile and the last
  // workgroup of the tile adds the KG partial tiles in order (the fix-up of
  // gemm_wq_kernel, with group 0's 256 threads).
  const int tile = blockIdx.x;
  const CoherentTile tile_ws(reinterpret_cast<float4v*>(ws_part) + (size_t)tile * KG * (BM * BN / 4),
                             (uint32_t)(KG * BM * BN * 4));
  if (grp == 0) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          tile_ws.store((uint32_t)kg * (BM * BN / 4) + ((i * TN + j) * 4 + q) * NT0 + tid,
                        float4v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ uint32_t is_last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ws_cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == (uint32_t)(KG - 1);
  }
  __syncthreads();
  if (!is_last || grp != 0) return;
  // (Registers: the accumulators already use half of them, so half a tile
  // of loads at a time.)
  splitk_gather<TM, TN, NT0, (TM >= 2 ? TM / 2 : 1)>(acc, tile_ws, BM * BN / 4, KG, tid);
  store();
  if (tid == 0) __hip_atomic_store(&ws_cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// small-tile kernel (any K % 32 == 0)

constexpr int kTile = 64;
constexpr int kLdsPad = 8;  // halves; keeps 16-B alignment of row starts

template <class QF>
__device__ __forceinline__ half8 quarter_f16(const uint8_t* blk, int quarter) {
  float v[8];
  quarter_f32<QF>(blk, quarter, v);
  half8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (half_t)v[i];
  return h;
}

template <class QF>
__global__ __launch_bounds__(256) void gemm_small_kernel(const half_t* __restrict__ A,
                                                         const uint8_t* __restrict__ W,
                                                         half_t* __restrict__ C, int M, int N,
                                                         int K) {
  __shared__ __attribute__((aligned(16))) half_t As[kTile][32 + kLdsPad];
  __shared__ __attribute__((aligned(16))) half_t Ws[kTile][32 + kLdsPad];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int m_base = blockIdx.y * kTile, n_base = blockIdx.x * kTile;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const int nb = K >> 5;
  const int lr = tid >> 2, lq = tid & 3;  // loader: row, quarter
  float4v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};

  for (int b = 0; b < nb; ++b) {
    {
      const int gm = m_base + lr;
      half8 v = {};
      if (gm < M) v = *reinterpret_cast<const half8*>(A + (size_t)gm * K + (size_t)b * 32 + lq * 8);
      *reinterpret_cast<half8*>(&As[lr][lq * 8]) = v;
    }
    {
      const int gn = n_base + lr;
      half8 v = {};
      if (gn < N) v = quarter_f16<QF>(W + ((size_t)gn * nb + b) * QF::kBytes, lq);
      *reinterpret_cast<half8*>(&Ws[lr][lq * 8]) = v;
    }
    __syncthreads();
    const int r = lane & 15, kq = (lane >> 4) * 8;
    half8 af[2], bf[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const half8*>(&As[wm + i * 16 + r][kq]);
#pragma unroll
    for (int j = 0; j < 2; ++j) bf[j] = *reinterpret_cast<const half8*>(&Ws[wn + j * 16 + r][kq]);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    __syncthreads();
  }

  const int col = lane & 15, row4 = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gm = m_base + wm + i * 16 + row4 + r;
        const int gn = n_base + wn + j * 16 + col;
        if (gm < M && gn < N) C[(size_t)gm * N + gn] = (half_t)acc[i][j][r];
      }
}

// NF_HIP_GEMM_TILE for the dense fp16 path: an LDS-staged tile shape 0..6,
// or -1 (automatic choice).
inline int forced_tile() {
  static const int forced = nfhip::gemm_tile_from_name(std::getenv("NF_HIP_GEMM_TILE"));
  return forced;
}

// Tile shape for the LDS-staged tiled MFMA kernel: 0 = 256x256 (8 waves, one
// CTA per CU), 1 = 256x128 (8 waves, one CTA per CU), 2 = 128x128 (4 waves,
// two CTAs per CU).  Score = fraction of CTA slots busy over the whole run
// (the last round is usually partial) x the tile's relative per-CU
// efficiency, which measured on MI355X at about 0.8 for the two smaller
// tiles against 256x256; ties go to 128x128, whose two CTAs per CU hide each
// other's barriers.  NF_HIP_GEMM_TILE overrides the choice.
inline int pick_tile(uint32_t M, uint32_t N, int forced) {
  if (forced >= 0 && forced <= 6) return forced;
  constexpr long kCUs = 256;
  auto fill = [](long tiles, long slots) {
    const long rounds = (tiles + slots - 1) / slots;
    return (double)tiles / (double)(rounds * slots);
  };
  const long mt256 = (M + 255) / 256, mt128 = (M + 127) / 128;
  const long nt256 = (N + 255) / 256, nt128 = (N + 127) / 128;
  const double s0 = fill(mt256 * nt256, kCUs);
  const double s1 = 0.8 * fill(mt256 * nt128, kCUs);
  const double s2 = 0.8 * fill(mt128 * nt128, 2 * kCUs);
  if (s0 > s1 && s0 > s2) return 0;
  return s1 > s2 ? 1 : 2;
}

template <class QF, int BM, int BN, int WGM, int WGN, int NS = 2, typename CT = half_t>
hipError_t gemm_tile_launch(const half_t* a, const uint8_t* w, CT* c, uint32_t M, uint32_t N,
                            uint32_t K, const nfhip::Workspace& ws, hipStream_t s) {
  const long tiles = (long)((N + BN - 1) / BN) * ((M + BM - 1) / BM);
  if (tiles > (1L << 31) - 1) return hipErrorInvalidConfiguration;
  // Split K over 2, 4, ... workgroups per tile while the grid is below one
  // workgroup per CU and every part keeps at least 64 K steps (measured on
  // MI355X: shorter parts lose more to the fix-up than the wider grid gains);
  // bounded by the workspace.
  const int nk = (int)(K / kBK);
  static const int kg_max = [] {
    const char* e = std::getenv("NF_HIP_GEMM_SPLITK_MAX");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 ? v : 8;
  }();
  int kg = 1;
  while (kg < kg_max && tiles * kg < 256 && nk >= 128 * kg && tiles <= (long)ws.cnt_len &&
         (size_t)tiles * 2 * kg * BM * BN <= ws.part_floats)
    kg *= 2;
  const size_t lds = (size_t)NS * (BM + BN) * 64 * sizeof(half_t);
  // More than 64 KB of dynamic LDS must be allowed explicitly, once per kernel.
  if (kg == 1) {
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_tile_kernel<QF, BM, BN, WGM, WGN, NS, false, CT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    gemm_tile_kernel<QF, BM, BN, WGM, WGN, NS, false, CT><<<dim3((unsigned)tiles), dim3(64 * WGM * WGN), lds, s>>>(
        a, w, c, M, N, K, ws.part, ws.cnt);
  } else {
    if constexpr (std::is_same<QF, F16B>::value) return hipErrorInvalidValue;  // dense path never splits
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_tile_kernel<QF, BM, BN, WGM, WGN, NS, true, CT>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    gemm_tile_kernel<QF, BM, BN, WGM, WGN, NS, true, CT><<<dim3((unsigned)tiles, (unsigned)kg), dim3(64 * WGM * WGN), lds, s>>>(
        a, w, c, M, N, K, ws.part, ws.cnt);
  }
  return hipGetLastError();
}

template <class QF, int TM, int TN, int NW, int PF>
hipError_t gemm_wq_launch(const half_t* a, const uint8_t* w, half_t* c, uint32_t M, uint32_t N, uint32_t K,
                          const nfhip::Workspace& ws, hipStream_t s) {
  constexpr int BM = 32 * TM, BN = 32 * TN * NW;
  const long tiles = (long)((N + BN - 1) / BN) * ((M + BM - 1) / BM);
  if (tiles > (1L << 31) - 1) return hipErrorInvalidConfiguration;
  // Split K over kg = 1, 2, 4, ... workgroups per tile: one workgroup per CU
  // (256 CUs), so the run time goes as (rounds of 256 workgroups) x (K steps
  // per workgroup); take the smallest kg that minimizes it, with at least 16
  // K steps per part, bounded by the workspace.
  const int nk = (int)(K / kBK);
  static const int kg_max = [] {
    const char* e = std::getenv("NF_HIP_GEMM_SPLITK_MAX");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 ? v : 8;
  }();
  constexpr long kCUs = 256;
  int kg = 1;
  long best = ((tiles + kCUs - 1) / kCUs) * nk;
  for (int g = 2; g <= kg_max && g <= 8 && nk / g >= 16 && tiles <= (long)ws.cnt_len &&
                  (size_t)tiles * g * BM * BN <= ws.part_floats;
       g *= 2) {
    const long cost = ((tiles * g + kCUs - 1) / kCUs) * ((nk + g - 1) / g);
    if (cost < best) best = cost, kg = g;
  }
  const size_t lds = (size_t)2 * BM * 64 * sizeof(half_t);
  if (kg == 1) {
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_wq_kernel<QF, TM, TN, NW, PF, false>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    gemm_wq_kernel<QF, TM, TN, NW, PF, false><<<dim3((unsigned)tiles), dim3(64 * NW), lds, s>>>(
        a, w, c, M, N, K, ws.part, ws.cnt);
  } else {
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_wq_kernel<QF, TM, TN, NW, PF, true>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    gemm_wq_kernel<QF, TM, TN, NW, PF, true><<<dim3((unsigned)tiles, (unsigned)kg), dim3(64 * NW), lds, s>>>(
        a, w, c, M, N, K, ws.part, ws.cnt);
  }
  return hipGetLastError();
}

// gemm_wq2_kernel: K in whole step pairs (K % 128 == 0).  K is split over
// kg = 1, 2, 4, 8 workgroups per tile like gemm_wq_launch (one workgroup per
// CU; the smallest kg minimizing rounds x step pairs per workgroup, at least
// 8 pairs per part, bounded by the workspace).
template <class QF, int TM, int NW>
hipError_t gemm_wq2_launch(const half_t* a, const uint8_t* w, half_t* c, uint32_t M, uint32_t N, uint32_t K,
                           const nfhip::Workspace& ws, hipStream_t s) {
  constexpr int BM = 32 * TM, BN = 64 * NW;
  const long tiles = (long)((N + BN - 1) / BN) * ((M + BM - 1) / BM);
  if (tiles > (1L << 31) - 1 || K % 128 != 0) return hipErrorInvalidConfiguration;
  const int np = (int)(K / 128);
  static const int kg_max = [] {
    const char* e = std::getenv("NF_HIP_GEMM_SPLITK_MAX");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 ? v : 8;
  }();
  constexpr long kCUs = 256;
  int kg = 1;
  long best = ((tiles + kCUs - 1) / kCUs) * np;
  for (int g = 2; g <= kg_max && g <= 8 && np / g >= 8 && tiles <= (long)ws.cnt_len &&
                  (size_t)tiles * g * BM * BN <= ws.part_floats;
       g *= 2) {
    const long cost = ((tiles * g + kCUs - 1) / kCUs) * ((np + g - 1) / g);
    if (cost < best) best = cost, kg = g;
  }
  const size_t lds = (size_t)wq2_lds_bytes(TM, NW);
  if (kg == 1) {
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_wq2_kernel<QF, TM, NW, false>), hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)lds);
    if (attr != hipSuccess) return attr;
    gemm_wq2_kernel<QF, TM, NW, false><<<dim3((unsigned)tiles), dim3(128 * NW), lds, s>>>(a, w, c, M, N, K, ws.part,
                                                                                        ws.cnt);
  } else {
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_wq2_kernel<QF, TM, NW, true>), hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)lds);
    if (attr != hipSuccess) return attr;
    gemm_wq2_kernel<QF, TM, NW, true><<<dim3((unsigned)tiles, (unsigned)kg), dim3(128 * NW), lds, s>>>(
        a, w, c, M, N, K, ws.part, ws.cnt);
  }
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// f32 activations on bf16 MFMA: gemm_f32a_kernel
//
// C (f32) = A (f32) x deq(W)^T, every weight the exact f32 value d*(q-8)
// (Q4_0) or d*q (Q8_0), for batches too large for the small-batch kernel
// (which takes at most 32 activation rows per launch and so streams the
// weights once per 32 rows).  Here a workgroup streams each weight once per
// 32*TM rows, and the products are formed on v_mfma_f32_32x32x16_bf16 from
// exact bf16 pieces:
//   * each activation x = a1 + a2 + r (split2_rne: round-to-nearest bf16
//     pieces, |a2| <= 2^-8 |x|, |r| <= 2^-16 |x|), split once per workgroup
//     while its 64-column K step is staged into two bf16 planes in LDS;
//   * each weight v (at most 15 significant bits for Q4_0, 18 for Q8_0) =
//     b1 + b2 (+ b3 for Q8_0) exactly (truncated bf16 pieces, |b2| < 2^-7 |v|,
//     |b3| < 2^-14 |v|), formed in registers from the codes and the scale one
//     MFMA slice ahead;
//   * the MFMA terms are a1b1, a2b1, a1b2 (+ a1b3 for Q8_0); the dropped
//     a2b2 < 2^-15 |x v|, r v < 2^-16 |x v| and a2b3 < 2^-22 |x v|.  The
//     products are exact and the MFMA accumulates in fp32, so each x*v
//     enters the sum within 3 * 2^-16 (4.6e-5) of its value, and an output
//     within 4.6e-5 of the sum of |x v| over K plus its fp32 accumulation
//     error: the 1e-3 bar of the reference's f32 loop
//     (metal_provider.mm:1396-1431) with room to spare.  (Three activation
//     pieces and 5 / 6 terms, every piece product above 2^-22 |x v|, took
//     4096x4096 at M = 2048 / 512 / 128 to 249 / 203 / 124 TFLOP/s against
//     351 / 261 / 139 for Q4_0, and Q8_0 M = 2048 to 213 against 282, on
//     MI355X.)
// Tiling as gemm_wq_kernel: 32*TM x 32*TN per wave, NW waves along N, the
// same K permutation (slice kk of a step pairs lane group kb with elements
// 8kk..8kk+7 of block kb) and output layout; A through a two-stage LDS
// buffer (A of step s+1 loaded into registers at the start of step s, split
// and written at its end), weights two steps ahead in two register sets.
// K may be split across workgroups (the fix-up of gemm_wq_kernel).

// Weight pieces of slice kk of the lane's block: 8 values, as NB bf16x8.
template <class QF, int NB>
__device__ __forceinline__ void f32a_weight_slice(const uint32_t (&w)[WBlk<QF>::kDwords], uint32_t sel, float d,
                                                  int kk, u32x4 (&out)[NB]) {
  float v[8];
  if constexpr (std::is_same<QF, Q4_0>::value) {
    const int t0 = 2 * (kk & 1);
    const uint32_t qa = __builtin_amdgcn_perm(w[t0 + 1], w[t0], sel);
    const uint32_t qb = __builtin_amdgcn_perm(w[t0 + 2], w[t0 + 1], sel);
    const uint32_t xa = (kk >> 1) ? (qa >> 4) & 0x0F0F0F0Fu : qa & 0x0F0F0F0Fu;
    const uint32_t xb = (kk >> 1) ? (qb >> 4) & 0x0F0F0F0Fu : qb & 0x0F0F0F0Fu;
    const float m8d = -8.f * d;  // exact
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __builtin_fmaf((float)((xa >> (8 * e)) & 0xFFu), d, m8d);  // d*(q-8), exact
      v[4 + e] = __builtin_fmaf((float)((xb >> (8 * e)) & 0xFFu), d, m8d);
    }
  } else {
    const uint32_t ua = __builtin_amdgcn_perm(w[2 * kk + 1], w[2 * kk], sel) ^ 0x80808080u;  // q + 128
    const uint32_t ub = __builtin_amdgcn_perm(w[2 * kk + 2], w[2 * kk + 1], sel) ^ 0x80808080u;
    const float m128d = -128.f * d;  // exact
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = __builtin_fmaf((float)((ua >> (8 * e)) & 0xFFu), d, m128d);  // d*q, exact
      v[4 + e] = __builtin_fmaf((float)((ub >> (8 * e)) & 0xFFu), d, m128d);
    }
  }
#pragma unroll
  for (int p = 0; p < NB; ++p) {
    out[p] = u32x4{pack_hi16(v[0], v[1]), pack_hi16(v[2], v[3]), pack_hi16(v[4], v[5]), pack_hi16(v[6], v[7])};
    if (p + 1 < NB) {
#pragma unroll
      for (int e = 0; e < 8; ++e)  // residual below the truncated piece: exact
        v[e] -= __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v[e]) & 0xFFFF0000u);
    }
  }
}

template <class QF, int TM, int TN, int NW, bool SPLIT>
__global__ __launch_bounds__(64 * NW, 1) void gemm_f32a_kernel(const float* __restrict__ A,
                                                               const uint8_t* __restrict__ W, float* __restrict__ C,
                                                               int M, int N, int K, float* __restrict__ ws_part,
                                                               uint32_t* __restrict__ ws_cnt) {
  constexpr bool kQ4 = std::is_same<QF, Q4_0>::value;
  constexpr int NB = kQ4 ? 2 : 3;  // bf16 pieces of a weight
  constexpr int NA = 2;            // bf16 pieces of an activation
  constexpr int NTERM = kQ4 ? 3 : 4;
  constexpr int BM = 32 * TM, BN = 32 * TN * NW, NT = 64 * NW;
  constexpr int PLANE = BM * 64;     // bf16 values per piece plane per stage
  constexpr int STAGE = NA * PLANE;  // the activation pieces
  constexpr int A_T = BM / (8 * NW);  // 8-float activation chunks per lane per step
  static_assert(BM % (8 * NW) == 0, "A rows per wave");
  constexpr int WD = WBlk<QF>::kDwords;
  extern __shared__ __attribute__((aligned(16))) uint16_t ldsb[];  // [2][NA][BM][64] bf16

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, kb = lane >> 5;
  int tm, tn;
  xcd_tile(blockIdx.x, (M + BM - 1) / BM, (N + BN - 1) / BN, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN, wn = wave * 32 * TN;
  const int KG = SPLIT ? (int)gridDim.y : 1, kg = SPLIT ? (int)blockIdx.y : 0;
  const int nk_all = K / kBK;
  const int k_first = (int)((long)nk_all * kg / KG);
  const int nk = (int)((long)nk_all * (kg + 1) / KG) - k_first;

  // A: chunk i of a lane is row (wave*A_T + i)*8 + l/8, floats 8*(l%8) ..
  // +7 of the step (eight lanes read one row's 256 B).  Rows past M read row
  // M-1 (their outputs are never stored).
  const float* asrc[A_T];
  int adst[A_T];
#pragma unroll
  for (int i = 0; i < A_T; ++i) {
    const int r = (wave * A_T + i) * 8 + (lane >> 3);
    const int gr = m0 + r < M ? m0 + r : M - 1;
    asrc[i] = A + (size_t)gr * K + (size_t)k_first * kBK + (lane & 7) * 8;
    adst[i] = tile_off(r, lane & 7);
  }
  // W: frag j of this lane is row n0 + wn + 32j + r32, block kb of each pair
  // (rows past N read row 0 with the scale forced to zero).
  const size_t row_bytes = (size_t)(K / 64) * GPair<QF>::kBytes;
  const uint32_t w_sel = kb ? 0x07060504u : 0x05040302u, w_sh = kb ? 16u : 0u;
  const uint8_t* wsrc[TN];
  bool w_valid[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn + 32 * j + r32;
    w_valid[j] = n < N;
    wsrc[j] = W + (size_t)(w_valid[j] ? n : 0) * row_bytes + (size_t)k_first * GPair<QF>::kBytes +
              kb * 4 * WBlk<QF>::kStride;
  }

  float ra[A_T][8];
  auto load_a = [&](int ks) {
#pragma unroll
    for (int i = 0; i < A_T; ++i) {
      const float4v lo = *reinterpret_cast<const float4v*>(asrc[i] + (size_t)ks * kBK);
      const float4v hi = *reinterpret_cast<const float4v*>(asrc[i] + (size_t)ks * kBK + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) ra[i][e] = lo[e], ra[i][4 + e] = hi[e];
    }
  };
  auto write_a = [&](int stage) {
    uint16_t* dst = ldsb + stage * STAGE;
#pragma unroll
    for (int i = 0; i < A_T; ++i) {
      bf16x8 p1, p2;
      split2_rne(ra[i], p1, p2);
      *reinterpret_cast<bf16x8*>(dst + adst[i]) = p1;
      *reinterpret_cast<bf16x8*>(dst + PLANE + adst[i]) = p2;
    }
  };
  uint32_t wr[2][TN][WD];
  auto load_w = [&](int ks, int set) {
#pragma unroll
    for (int j = 0; j < TN; ++j) load_wblk<QF>(wsrc[j] + (size_t)ks * GPair<QF>::kBytes, wr[set][j]);
  };
  float dsc[2][TN];
  auto scales = [&](int set) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint32_t db = (wr[set][j][0] >> w_sh) & 0xFFFFu;
      dsc[set][j] = w_valid[j] ? h2f_bits((uint16_t)db) : 0.f;
    }
  };
  u32x4 bp[2][TN][NB];
  auto weights = [&](int set, int kk, int buf) {
#pragma unroll
    for (int j = 0; j < TN; ++j) f32a_weight_slice<QF, NB>(wr[set][j], w_sel, dsc[set][j], kk, bp[buf][j]);
  };
  bf16x8 ap[2][NA][TM];
  auto read_a = [&](int stage, int kk, int buf) {
    const uint16_t* As = ldsb + stage * STAGE;
#pragma unroll
    for (int p = 0; p < NA; ++p)
#pragma unroll
      for (int i = 0; i < TM; ++i)
        ap[buf][p][i] = *reinterpret_cast<const bf16x8*>(As + p * PLANE + tile_off(32 * i + r32, 4 * kb + kk));
  };
  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};
  // Terms (weight piece, activation piece), most significant first.
  constexpr int kWb[4] = {0, 0, 1, 2}, kAb[4] = {0, 1, 0, 0};
  auto mfma = [&](int buf) {
#pragma unroll
    for (int t = 0; t < NTERM; ++t)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, bp[buf][j][kWb[t]]),
                                                              ap[buf][kAb[t]][i], acc[i][j], 0, 0, 0);
  };
  auto lds_barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  // Prologue: A of step 0 split into stage 0; weights of steps 0 and 1 (past
  // the last step: its loads again, never used) in register sets 0 and 1.
  load_a(0);
  load_w(0, 0);
  load_w(nk > 1 ? 1 : 0, 1);
  write_a(0);
  scales(0);
  lds_barrier();
  read_a(0, 0, 0);
  weights(0, 0, 0);

  // Step s (register set and stage u = s & 1): A of step s+1 loaded at the
  // start; per slice kk the next slice's operands, then this slice's MFMAs;
  // the weights of step s+2 loaded into set u once its last slice is formed;
  // A of step s+1 split into stage u^1; barrier; slice 0 of step s+1.
  auto step = [&](auto uc, int s) {
    constexpr int u = decltype(uc)::value;
    load_a(s + 1 < nk ? s + 1 : nk - 1);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk < 3) {
        read_a(u, kk + 1, (kk + 1) & 1);
        weights(u, kk + 1, (kk + 1) & 1);
      } else {
        load_w(s + 2 < nk ? s + 2 : nk - 1, u);
        if (s + 1 < nk) write_a(u ^ 1);
      }
      mfma(kk & 1);
    }
    lds_barrier();
    if (s + 1 < nk) {
      scales(u ^ 1);
      read_a(u ^ 1, 0, 0);
      weights(u ^ 1, 0, 0);
    }
  };
  int s = 0;
  for (; s + 2 <= nk; s += 2) {
    step(std::integral_constant<int, 0>{}, s);
    step(std::integral_constant<int, 1>{}, s + 1);
  }
  if (s < nk) step(std::integral_constant<int, 0>{}, s);

  // accumulator r of lane l: C[m = 32i + l%32][n = 32j + (r/4)*8 + (l/32)*4 + r%4]
  auto store = [&]() {
    const bool vec = (N & 3) == 0 && ((uintptr_t)C & 15) == 0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int gm = m0 + 32 * i + r32;
      if (gm >= M) continue;
      float* crow = C + (size_t)gm * N;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int gn = n0 + wn + 32 * j + 8 * q + 4 * kb;
          if (vec && gn + 3 < N) {
            *reinterpret_cast<float4v*>(crow + gn) =
                float4v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (gn + e < N) crow[gn + e] = acc[i][j][4 * q + e];
          }
        }
    }
  };
  if constexpr (!SPLIT) {
    store();
    return;
  }
  // K split across workgroups: the fix-up of gemm_wq_kernel.
  const int tile = blockIdx.x;
  const CoherentTile tile_ws(reinterpret_cast<float4v*>(ws_part) + (size_t)tile * KG * (BM * BN / 4),
                             (uint32_t)(KG * BM * BN * 4));
  {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          tile_ws.store((uint32_t)kg * (BM * BN / 4) + ((i * TN + j) * 4 + q) * NT + tid,
                        float4v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]});
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ uint32_t is_last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ws_cnt[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == (uint32_t)(KG - 1);
  }
  __syncthreads();
  if (!is_last) return;
  splitk_gather<TM, TN, NT, (TM % 2 == 0) ? TM / 2 : TM>(acc, tile_ws, BM * BN / 4, KG, tid);
  store();
  if (tid == 0) __hip_atomic_store(&ws_cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// K % 64 == 0.  K split over kg = 1, 2, 4, 8 workgroups per tile as in
// gemm_wq_launch, with at least 8 K steps per part.
template <class QF, int TM, int TN, int NW>
hipError_t gemm_f32a_launch(const float* a, const uint8_t* w, float* c, uint32_t M, uint32_t N, uint32_t K,
                            const nfhip::Workspace& ws, hipStream_t s) {
  constexpr int BM = 32 * TM, BN = 32 * TN * NW;
  const long tiles = (long)((N + BN - 1) / BN) * ((M + BM - 1) / BM);
  if (tiles > (1L << 31) - 1 || K % kBK != 0) return hipErrorInvalidConfiguration;
  const int nk = (int)(K / kBK);
  static const int kg_max = [] {
    const char* e = std::getenv("NF_HIP_GEMM_SPLITK_MAX");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 ? v : 8;
  }();
  constexpr long kCUs = 256;
  int kg = 1;
  long best = ((tiles + kCUs - 1) / kCUs) * nk;
  for (int g = 2; g <= kg_max && g <= 8 && nk / g >= 8 && tiles <= (long)ws.cnt_len &&
                  (size_t)tiles * g * BM * BN <= ws.part_floats;
       g *= 2) {
    const long cost = ((tiles * g + kCUs - 1) / kCUs) * ((nk + g - 1) / g);
    if (cost < best) best = cost, kg = g;
  }
  const size_t lds = (size_t)2 * 2 * BM * 64 * sizeof(uint16_t);  // two stages of two activation planes
  if (kg == 1) {
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_f32a_kernel<QF, TM, TN, NW, false>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    gemm_f32a_kernel<QF, TM, TN, NW, false><<<dim3((unsigned)tiles), dim3(64 * NW), lds, s>>>(a, w, c, M, N, K,
                                                                                             ws.part, ws.cnt);
  } else {
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_f32a_kernel<QF, TM, TN, NW, true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    gemm_f32a_kernel<QF, TM, TN, NW, true><<<dim3((unsigned)tiles, (unsigned)kg), dim3(64 * NW), lds, s>>>(
        a, w, c, M, N, K, ws.part, ws.cnt);
  }
  return hipGetLastError();
}

}  // namespace nfk

namespace nfhip {

// Dense fp16 x fp16 linear on the tiled MFMA kernel (B stored [N,K]), fp16
// or fp32 output.
template <typename CT>
hipError_t dense_mfma_f16(const nfk::half_t* a, const uint8_t* b, CT* c, uint32_t M, uint32_t N, uint32_t K,
                          hipStream_t s) {
  switch (nfk::pick_tile(M, N, nfk::forced_tile())) {
    case 0: return nfk::gemm_tile_launch<nfk::F16B, 256, 256, 2, 4, 2, CT>(a, b, c, M, N, K, nfhip::Workspace{}, s);
    case 1: return nfk::gemm_tile_launch<nfk::F16B, 256, 128, 4, 2, 2, CT>(a, b, c, M, N, K, nfhip::Workspace{}, s);
    case 3: return nfk::gemm_tile_launch<nfk::F16B, 256, 128, 2, 2, 2, CT>(a, b, c, M, N, K, nfhip::Workspace{}, s);
    case 4: return nfk::gemm_tile_launch<nfk::F16B, 256, 128, 2, 2, 3, CT>(a, b, c, M, N, K, nfhip::Workspace{}, s);
    case 5: return nfk::gemm_tile_launch<nfk::F16B, 128, 128, 2, 2, 3, CT>(a, b, c, M, N, K, nfhip::Workspace{}, s);
    case 6: return nfk::gemm_tile_launch<nfk::F16B, 128, 256, 2, 4, 2, CT>(a, b, c, M, N, K, nfhip::Workspace{}, s);
    default: return nfk::gemm_tile_launch<nfk::F16B, 128, 128, 2, 2, 2, CT>(a, b, c, M, N, K, nfhip::Workspace{}, s);
  }
}

hipError_t launch_dense_mfma_f16(const void* A, const void* B, void* C, uint32_t M, uint32_t N, uint32_t K,
                                 bool out_f32, hipStream_t s) {
  const nfk::half_t* a = static_cast<const nfk::half_t*>(A);
  const uint8_t* b = static_cast<const uint8_t*>(B);
  if (K % 64 != 0 || (uintptr_t)A % 16 != 0 || (uintptr_t)B % 16 != 0) return hipErrorInvalidValue;
  return out_f32 ? dense_mfma_f16<float>(a, b, static_cast<float*>(C), M, N, K, s)
                 : dense_mfma_f16<nfk::half_t>(a, b, static_cast<nfk::half_t*>(C), M, N, K, s);
}

hipError_t launch_gemm_mfma(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                            uint32_t N, uint32_t K, int tile, const Workspace& ws, hipStream_t s) {
  if (t == EType::F32) {  // f32 activations and output: bf16-piece MFMA kernel
    // Operands at addresses the kernel's 16-byte activation loads and dword
    // weight loads cannot take (imported buffers at odd offsets, raw
    // pointers of the no-allocation entry point): the GEMV, whose block
    // kernel reads any alignment and any M.
    const bool aligned = ((uintptr_t)A % 16 == 0) && ((uintptr_t)W % 4 == 0);
    if (K % 64 != 0 || !aligned) return launch_gemv(q, t, A, W, C, M, N, K, s);
    const float* a = static_cast<const float*>(A);
    const uint8_t* w = static_cast<const uint8_t*>(W);
    float* c = static_cast<float*>(C);
    // 64-row waves up to M = 64, and while the batch makes few 64x256
    // tiles (at most 32, or 64 with K <= 8192): measured on MI355X, Q4_0
    // 4096x4096 M = 128 39.0 against 56.6 us with 128-row waves, 4096x14336
    // M = 128 100.0 against 139.6; 128-row waves win from 86 tiles on
    // (11008x4096 M = 65: 85.0 against 96.0).  Tile 9 / 8 force them.
    const long tiles64 = (long)((M + 63) / 64) * (long)((N + 255) / 256);
    if (tile == 9 || (tile != 8 && (M <= 64 || tiles64 <= 32 || (tiles64 <= 64 && K <= 8192))))
      return q == QFmt::Q4_0 ? nfk::gemm_f32a_launch<nfk::Q4_0, 2, 2, 4>(a, w, c, M, N, K, ws, s)
                             : nfk::gemm_f32a_launch<nfk::Q8_0, 2, 2, 4>(a, w, c, M, N, K, ws, s);
    return q == QFmt::Q4_0 ? nfk::gemm_f32a_launch<nfk::Q4_0, 4, 2, 4>(a, w, c, M, N, K, ws, s)
                           : nfk::gemm_f32a_launch<nfk::Q8_0, 4, 2, 4>(a, w, c, M, N, K, ws, s);
  }
  if (t != EType::F16) return hipErrorInvalidValue;
  const nfk::half_t* a = static_cast<const nfk::half_t*>(A);
  const uint8_t* w = static_cast<const uint8_t*>(W);
  nfk::half_t* c = static_cast<nfk::half_t*>(C);
  const bool aligned = ((uintptr_t)A % 16 == 0) && ((uintptr_t)W % 4 == 0);
  if (K % 64 == 0 && aligned) {
    // Default: the register-dequantizing kernels (measured faster than the
    // LDS-staged tiles at every prefill shape with M > 64), picked by M
    // (bench sweeps on MI355X, f16 activations, graph replay over 4 weight
    // copies):
    //   * M <= 32: two waves per SIMD with 32-row waves (gemm_wq2_kernel,
    //     TM = 1): 71 against 96-102 us at 28672x8192 / 8192x28672 M = 32;
    //   * M <= 64: the same with 64-row waves (TM = 2): 81 / 84 against
    //     102 / 110 us at M = 64;
    //   * M > 64 with few 64-row tiles (ceil(M/64) x ceil(N/256) <= 80 for
    //     Q4_0, <= 64 for Q8_0) and K <= 16384: 64-row waves again, which
    //     spread a short batch over more workgroups (4096x4096 Q4_0 M = 128:
    //     24.6 against 38.1 us, 4096x11008 M = 256: 45.9 against 62.6; Q8_0
    //     4096x4096 M = 128: 31.2 against 41.5; not at K = 28672, where
    //     8192x28672 M = 128 took 122.0 against 104.1 us with 128-row waves);
    //   * other Q4_0 batches: 128-row waves (TM = 4): at M = 2048 816 / 747
    //     / 859 against 785 / 735 / 804 TFLOP/s on the three Llama-2-7B
    //     projection shapes, at M = 512 41.9 / 77.4 / 69.9 against 45.6 /
    //     78.6 / 76.4 us (within 2 % either way on the 28672-row FFN
    //     shapes);
    //     but Q4_0 batches whose 128 x 256 grid holds little work
    //     (ceil(M/128) x ceil(N/256) x K/128 <= 4096 step pairs) take
    //     128 x 128 tiles (two waves per K group), which double the
    //     workgroups and halve each split-K partial: 4096x4096 M = 384 /
    //     512 / 1024 34.5 / 36.4 / 50.6 against 37.0 / 40.5 / 55.6 us,
    //     2048x4096 M = 1024 35.5 against 40.3, 1024x4096 M = 2048 34.5
    //     against 38.9, 4096x8192 M = 512 55.1 against 57.7; above that
    //     bound they lost (8192x8192 M = 512 95.0 against 92.2, 11008x4096
    //     M = 512 91.8 against 72.7, 4096x11008 M = 512 73.4 against 70.8,
    //     4096x4096 M = 2048 91.4 against 79.8 us);
    //   * otherwise one wave per SIMD (gemm_wq_kernel; also Q8_0 at larger
    //     M, where the two-wave kernel measured 5-12 % slower);
    // all of them need K % 128 == 0 but gemm_wq_kernel.  Tile 7 forces the
    // one-wave kernel, tiles 8 / 9 / 10 the two-wave kernel with 128 / 64 /
    // 32-row waves (8: Q4_0 only), tile 11 the 128-row waves on 128 x 128
    // tiles (Q4_0 only); 0..6 select one of the LDS-staged tile shapes.
    const bool k128 = K % 128 == 0;
    const bool q4 = q == QFmt::Q4_0;
    const long tiles64 = (long)((M + 63) / 64) * (long)((N + 255) / 256);
    if ((tile == 10 || (tile < 0 && M <= 32)) && k128)
      return q4 ? nfk::gemm_wq2_launch<nfk::Q4_0, 1, 4>(a, w, c, M, N, K, ws, s)
                : nfk::gemm_wq2_launch<nfk::Q8_0, 1, 4>(a, w, c, M, N, K, ws, s);
    if ((tile == 9 || (tile < 0 && (M <= 64 || (tiles64 <= (q4 ? 80 : 64) && K <= 16384)))) && k128)
      return q4 ? nfk::gemm_wq2_launch<nfk::Q4_0, 2, 4>(a, w, c, M, N, K, ws, s)
                : nfk::gemm_wq2_launch<nfk::Q8_0, 2, 4>(a, w, c, M, N, K, ws, s);
    const long pairs128 = (long)((M + 127) / 128) * (long)((N + 255) / 256) * (long)(K / 128);
    if ((tile == 11 || (tile < 0 && pairs128 <= 4096)) && k128 && q4)
      return nfk::gemm_wq2_launch<nfk::Q4_0, 4, 2>(a, w, c, M, N, K, ws, s);
    if ((tile == 8 || tile < 0) && k128 && q4)
      return nfk::gemm_wq2_launch<nfk::Q4_0, 4, 4>(a, w, c, M, N, K, ws, s);
    if (tile < 0 || tile > 6)
      return (q == QFmt::Q4_0) ? nfk::gemm_wq_launch<nfk::Q4_0, 4, 2, 4, 4>(a, w, c, M, N, K, ws, s)
                               : nfk::gemm_wq_launch<nfk::Q8_0, 4, 2, 4, 4>(a, w, c, M, N, K, ws, s);
    switch (tile) {
      case 0:
        return (q == QFmt::Q4_0) ? nfk::gemm_tile_launch<nfk::Q4_0, 256, 256, 2, 4>(a, w, c, M, N, K, ws, s)
                                 : nfk::gemm_tile_launch<nfk::Q8_0, 256, 256, 2, 4>(a, w, c, M, N, K, ws, s);
      case 1:
        return (q == QFmt::Q4_0) ? nfk::gemm_tile_launch<nfk::Q4_0, 256, 128, 4, 2>(a, w, c, M, N, K, ws, s)
                                 : nfk::gemm_tile_launch<nfk::Q8_0, 256, 128, 4, 2>(a, w, c, M, N, K, ws, s);
      case 3:
        return (q == QFmt::Q4_0) ? nfk::gemm_tile_launch<nfk::Q4_0, 256, 128, 2, 2>(a, w, c, M, N, K, ws, s)
                                 : nfk::gemm_tile_launch<nfk::Q8_0, 256, 128, 2, 2>(a, w, c, M, N, K, ws, s);
      case 4:
        return (q == QFmt::Q4_0) ? nfk::gemm_tile_launch<nfk::Q4_0, 256, 128, 2, 2, 3>(a, w, c, M, N, K, ws, s)
                                 : nfk::gemm_tile_launch<nfk::Q8_0, 256, 128, 2, 2, 3>(a, w, c, M, N, K, ws, s);
      case 5:
        return (q == QFmt::Q4_0) ? nfk::gemm_tile_launch<nfk::Q4_0, 128, 128, 2, 2, 3>(a, w, c, M, N, K, ws, s)
                                 : nfk::gemm_tile_launch<nfk::Q8_0, 128, 128, 2, 2, 3>(a, w, c, M, N, K, ws, s);
      case 6:
        return (q == QFmt::Q4_0) ? nfk::gemm_tile_launch<nfk::Q4_0, 128, 256, 2, 4>(a, w, c, M, N, K, ws, s)
                                 : nfk::gemm_tile_launch<nfk::Q8_0, 128, 256, 2, 4>(a, w, c, M, N, K, ws, s);
      default:
        return (q == QFmt::Q4_0) ? nfk::gemm_tile_launch<nfk::Q4_0, 128, 128, 2, 2>(a, w, c, M, N, K, ws, s)
                                 : nfk::gemm_tile_launch<nfk::Q8_0, 128, 128, 2, 2>(a, w, c, M, N, K, ws, s);
    }
  }
  const dim3 grid((N + nfk::kTile - 1) / nfk::kTile, (M + nfk::kTile - 1) / nfk::kTile);
  if (grid.y > 65535) return hipErrorInvalidConfiguration;
  if (q == QFmt::Q4_0)
    nfk::gemm_small_kernel<nfk::Q4_0><<<grid, dim3(256), 0, s>>>(a, w, c, M, N, K);
  else
    nfk::gemm_small_kernel<nfk::Q8_0><<<grid, dim3(256), 0, s>>>(a, w, c, M, N, K);
  return hipGetLastError();
}

}  // namespace nfhip
