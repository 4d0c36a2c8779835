// skinny.hip — fused dequant + matmul for small batches (M up to 64) on MFMA.
//
// C[m, n] = sum_k A[m, k] * deq(W)[n, k] with fp32 accumulation, for the
// batch sizes between the decode GEMV (M = 1..2) and the prefill GEMM.  The
// weight stream is read once; MFMA absorbs the per-row multiply so the cost
// per weight stays flat in M.
//
// MFMA v_mfma_f32_16x16x32 (f16 or bf16 operands): A = activations (16 rows
// of M), B = weights (16 rows of N), D[m][n] = sum over 32 k.  Lane l:
//   A: row l%16, eight k values of slot s = l/16;
//   B: weight row l%16, the same eight k values;
//   D: weight row l%16, activation rows 4s..4s+3.
// One instruction covers exactly one 32-element block.  Slot s holds the k
// values a lane can unpack from one code word: Q4_0 slot s = qs[4s..4s+3],
// i.e. k = 4s..4s+3 (low nibbles) and 16+4s..16+4s+3 (high nibbles); Q8_0
// slot s = codes 8s..8s+7.  A is gathered in the same order.
//
// f16 activations (the _f16 op): B = RNE(d*q) in fp16 (the bits of
// dequant_*_f16), one MFMA per block and tile, accumulated across blocks.
//
// f32 activations: each activation x is split into two bf16 parts (x ~ b1 +
// b2: b1 the upper half of x, b2 the remainder rounded, within 2^-16 |x|;
// bf16 has f32's exponent range), B = the integer codes, exact in bf16
// (Q4_0: 128 + n, the nibble placed under bf16 exponent bits 0x43 by one
// byte permute per two codes; Q8_0: the signed code), two chained MFMAs give
// sum_k code*x with exact products and fp32 accumulation, and the block
// scale is applied per block: acc += d * D.  The Q4_0 offset of -136 (128 of
// the bf16 placement and the code's own 8) starts each block's chain from
// sum_k (-136)*x, one extra chain per activation tile that all weight tiles
// share.  Each product code * x is within 2^-16 of exact, a few parts in
// 10^5 of the output at most, against the 1e-3 bar.
//
// Work split: a wave owns 64 weight rows (4 tiles of 16) and a contiguous
// range of K, in chunks of CHP pairs (64 elements each); the waves of a
// workgroup split K, park their partial sums in LDS and the workgroup adds
// them in a fixed order before storing C.  A chunk of weights is fetched with contiguous 4/8/16-byte
// loads (4 bytes per pair of the chunk, so consecutive lanes read consecutive
// bytes of a row) into a wave-private LDS area, from which each lane gathers
// its slot dwords; the activations are gathered straight from global memory
// (they are L2-resident).  Both go through range-checked buffer loads.  Per
// chunk the loads are issued as activations, then weights, so chunk c
// computes while both of chunk c+1 are in flight.
// At most 32 activation rows per launch keep the two activation register sets
// and the accumulators in registers; more rows take more launches.
//
// f32 activations go to skinny_ring_kernel (below) instead: the same MFMA
// chain, with the weights streamed through a four-stage LDS ring by buffer
// loads to LDS (three chunks in flight at no register cost), the activations
// split into bf16 pieces once per workgroup of 8 waves rather than once per
// wave, and up to 64 rows in one pass (one read of the weights).  Measured
// on MI355X: Llama-3-8B Q8_0 decode step at M = 64 10.7 -> 5.95 ms, M = 16
// 3.39 -> 3.26 ms; TinyLlama Q4_0 M = 16 1042 -> 971 us.  skinny_kernel
// remains the f32 path with NF_HIP_SKINNY_RING=0.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "../launch.hpp"
#include "common.hpp"

namespace nfk {


template <class QF> struct SkW;
template <> struct SkW<Q4_0> {
  static constexpr int kPairBytes = 36, kLoads = 5;
};
template <> struct SkW<Q8_0> {
  static constexpr int kPairBytes = 68, kLoads = 7;
};

// The dwords of pair `p` of weight row `row` that slot s needs.
template <class QF>
__device__ __forceinline__ void sk_load_w(const uint32_t* __restrict__ pr, int s, uint32_t (&w)[SkW<QF>::kLoads]) {
  if constexpr (SkW<QF>::kLoads == 5) {
    w[0] = pr[s];      // block 0 codes, realigned with w[1]
    w[1] = pr[s + 1];
    w[2] = pr[5 + s];  // block 1 codes
    w[3] = pr[0];      // block 0 scale (low half)
    w[4] = pr[4];      // block 1 scale (high half)
  } else {
    w[0] = pr[2 * s];  // block 0 codes: bytes 2+8s .. 9+8s across three dwords
    w[1] = pr[2 * s + 1];
    w[2] = pr[2 * s + 2];
    w[3] = pr[9 + 2 * s];   // block 1 codes
    w[4] = pr[10 + 2 * s];
    w[5] = pr[0];      // block 0 scale (low half)
    w[6] = pr[8];      // block 1 scale (high half)
  }
}

template <class QF>
__device__ __forceinline__ uint32_t sk_scale_bits(const uint32_t (&w)[SkW<QF>::kLoads], int h) {
  if constexpr (SkW<QF>::kLoads == 5) return h == 0 ? (w[3] & 0xFFFFu) : (w[4] >> 16);
  else return h == 0 ? (w[5] & 0xFFFFu) : (w[6] >> 16);
}

__device__ __forceinline__ half2v h2u(uint32_t u) { return __builtin_bit_cast(half2v, u); }
__device__ __forceinline__ uint32_t u2h(half2v h) { return __builtin_bit_cast(uint32_t, h); }

// B operand, f16 path: RNE(d*q) for the 8 k values of the lane's slot.
template <class QF>
__device__ __forceinline__ half8 sk_b_f16(const uint32_t (&w)[SkW<QF>::kLoads], int h) {
  const uint32_t db = sk_scale_bits<QF>(w, h);
  const half2v d2 = h2u(db | (db << 16));
  u32x4 o;
  if constexpr (SkW<QF>::kLoads == 5) {
    const uint32_t q = h == 0 ? __builtin_amdgcn_alignbyte(w[1], w[0], 2) : w[2];
    const uint32_t l = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
    const half2v off = {(half_t)-1032.f, (half_t)-1032.f};
    o.x = u2h((h2u(__builtin_amdgcn_perm(0x64646464u, l, 0x04010400u)) + off) * d2);
    o.y = u2h((h2u(__builtin_amdgcn_perm(0x64646464u, l, 0x04030402u)) + off) * d2);
    o.z = u2h((h2u(__builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u)) + off) * d2);
    o.w = u2h((h2u(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)) + off) * d2);
  } else {
    const uint32_t qa = h == 0 ? __builtin_amdgcn_alignbyte(w[1], w[0], 2) : w[3];
    const uint32_t qb = h == 0 ? __builtin_amdgcn_alignbyte(w[2], w[1], 2) : w[4];
    const half2v off = {(half_t)-1152.f, (half_t)-1152.f};
    const uint32_t ua = qa ^ 0x80808080u, ub = qb ^ 0x80808080u;
    o.x = u2h((h2u(__builtin_amdgcn_perm(0x64646464u, ua, 0x04010400u)) + off) * d2);
    o.y = u2h((h2u(__builtin_amdgcn_perm(0x64646464u, ua, 0x04030402u)) + off) * d2);
    o.z = u2h((h2u(__builtin_amdgcn_perm(0x64646464u, ub, 0x04010400u)) + off) * d2);
    o.w = u2h((h2u(__builtin_amdgcn_perm(0x64646464u, ub, 0x04030402u)) + off) * d2);
  }
  return __builtin_bit_cast(half8, o);
}

// B operand, f32 path: the codes of the lane's slot as exact bf16 (Q4_0:
// 128 + n with n the unsigned nibble, bf16 0x43nn; Q8_0: the signed code).
template <class QF>
__device__ __forceinline__ bf16x8 sk_b_codes(const uint32_t (&w)[SkW<QF>::kLoads], int h) {
  u32x4 o;
  if constexpr (SkW<QF>::kLoads == 5) {
    const uint32_t q = h == 0 ? __builtin_amdgcn_alignbyte(w[1], w[0], 2) : w[2];
    const uint32_t l = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
    o.x = __builtin_amdgcn_perm(0x43434343u, l, 0x04010400u);   // k = 4s, 4s+1
    o.y = __builtin_amdgcn_perm(0x43434343u, l, 0x04030402u);   // 4s+2, 4s+3
    o.z = __builtin_amdgcn_perm(0x43434343u, hi, 0x04010400u);  // 16+4s, 16+4s+1
    o.w = __builtin_amdgcn_perm(0x43434343u, hi, 0x04030402u);  // 16+4s+2, 16+4s+3
  } else {
    const uint32_t qa = h == 0 ? __builtin_amdgcn_alignbyte(w[1], w[0], 2) : w[3];
    const uint32_t qb = h == 0 ? __builtin_amdgcn_alignbyte(w[2], w[1], 2) : w[4];
    o.x = pack_hi16((float)(int8_t)qa, (float)(int8_t)(qa >> 8));
    o.y = pack_hi16((float)(int8_t)(qa >> 16), (float)((int32_t)qa >> 24));
    o.z = pack_hi16((float)(int8_t)qb, (float)(int8_t)(qb >> 8));
    o.w = pack_hi16((float)(int8_t)(qb >> 16), (float)((int32_t)qb >> 24));
  }
  return __builtin_bit_cast(bf16x8, o);
}

// Activation slot values: the 8 k values of slot s in block h of pair p.
template <class QF> struct SkK;
template <> struct SkK<Q4_0> {  // k = 4s..4s+3 and 16+4s..16+4s+3
  __device__ static int off0(int s) { return 4 * s; }
  __device__ static int off1(int s) { return 16 + 4 * s; }
};
template <> struct SkK<Q8_0> {  // k = 8s..8s+7
  __device__ static int off0(int s) { return 8 * s; }
  __device__ static int off1(int s) { return 8 * s + 4; }
};


// Staging piece of a weight chunk: 4 B per pair of the chunk (16 B for
// 4-pair chunks, 8 B for 2-pair, 4 B for 1-pair), so a row of a chunk is
// always 9 (Q4_0) or 17 (Q8_0) pieces.
template <int PS> struct Piece;
template <> struct Piece<16> { typedef u32x4 T; };
template <> struct Piece<8> { typedef uint2 T; };
template <> struct Piece<4> { typedef uint32_t T; };

// Range-checked buffer loads (gfx9 raw buffer resource: base, no stride,
// num_records bytes).  A load through a resource with num_records = 0
// returns zeros without touching memory and still counts as an outstanding
// load, which lets a loop issue the same loads on every pass (so the
// compiler's wait counts stay exact) while loads past a wave's range cost
// nothing.
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
template <int PS>
__device__ __forceinline__ typename Piece<PS>::T sk_buf_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  if constexpr (PS == 16) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  } else if constexpr (PS == 8) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
  } else {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  }
}

// Up to kGroupMax small-batch linears over the same activations in one
// launch: job j owns row tiles (grid x) begin[j] .. begin[j+1]-1 and runs on
// its own weights, output and N with the launch's shared K split, exactly as
// a launch of its own with that split would.
constexpr int kSkGroupMax = nfhip::kGemvGroupMax;
struct SkinnyGroup {
  const uint8_t* W[kSkGroupMax];
  void* C[kSkGroupMax];
  int N[kSkGroupMax];
  int begin[kSkGroupMax + 1];
};
static_assert(kSkGroupMax == 4, "the small-batch kernels pass begin[1..3] as scalar arguments");

// Arguments of the small-batch kernels: job 0's fields and the job
// boundaries begin[1..3] come first as plain scalars (W0 = grp.W[0], ...),
// so they are among the arguments preloaded into SGPRs at wave launch and a
// workgroup of job 0 (every workgroup of a single launch) issues its first
// loads without a scalar load from the argument block; other jobs read
// their entries of `grp`.  begin[] is non-decreasing and its unused entries
// equal the number of workgroups (tiles) along x.
__device__ __forceinline__ int group_job(int b1, int b2, int b3) {
  const int bx = (int)blockIdx.x;
  return (bx >= b1) + (bx >= b2) + (bx >= b3);
}

template <class QF, typename XT, int MT, int CHP>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 4))) void skinny_kernel(
    const XT* __restrict__ A, const uint8_t* __restrict__ W0, int N0, int b1, int b2, int b3, int M, int K,
    void* C0, float* __restrict__ ws_part, uint32_t* __restrict__ ws_cnt, const SkinnyGroup grp) {
  // This workgroup's job (uniform).
  const int job = group_job(b1, b2, b3);
  const uint8_t* __restrict__ W = W0;
  void* Cv = C0;
  int N = N0, tile0 = 0;
  if (job > 0) {
    W = grp.W[job];
    Cv = grp.C[job];
    N = grp.N[job];
    tile0 = grp.begin[job];
  }
  XT* __restrict__ C = static_cast<XT*>(Cv);
  constexpr bool kF32 = sizeof(XT) == 4;
  constexpr bool kQ4 = SkW<QF>::kLoads == 5;
  constexpr int WL = SkW<QF>::kLoads;
  constexpr int PB = SkW<QF>::kPairBytes;
  constexpr int T = 4;                      // 16-row weight tiles per wave
  constexpr int RW = 16 * T;                // weight rows per wave
  constexpr int PS = 4 * CHP;               // staging piece bytes
  constexpr int CB = CHP * PB / PS;         // pieces per row per chunk (9 / 17)
  constexpr int J = RW * CB / 64;           // pieces per lane per chunk
  constexpr int PITCH = CHP * PB / 4;       // dwords per staged row
  static_assert(RW * CB % 64 == 0, "chunk pieces per lane");
  typedef typename Piece<PS>::T PieceT;
  constexpr int NV = MT * T * 4;            // accumulator values per lane
  // Per wave, one LDS area holds the staged weight rows during the K loop
  // and the wave's partial sums afterwards.
  constexpr int AREA = RW * PITCH > NV * 64 ? RW * PITCH : NV * 64;  // dwords
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar loop control
  const int KS = blockDim.x >> 6;
  const int r16 = lane & 15, s = lane >> 4;
  const int P = K >> 6;
  const int NC = P / CHP;  // chunks along K
  const int n0 = ((int)blockIdx.x - tile0) * RW;
  uint32_t* wst = smem + (size_t)wave * AREA;

  // K range of this wave (whole chunks): the KG = gridDim.y workgroups of a
  // row tile and their KS waves split the chunks evenly.
  const int KG = gridDim.y, kg = blockIdx.y;
  const int gw = kg * KS + wave, nw = KG * KS;
  const int c_begin = (int)((long)NC * gw / nw), c_end = (int)((long)NC * (gw + 1) / nw);

  // Weight staging: piece f = lane + 64*j of the wave's RW x CB chunk is row
  // f / CB, piece f % CB; consecutive lanes read consecutive bytes of a row,
  // and piece f lands at LDS dword f * PS/4 (= row * PITCH + piece * PS/4).
  // Rows past N read row N-1 (their B operands are zeroed below).  Offsets
  // are 32-bit (the host keeps a weight matrix below 4 GB on this path).
  const uint32_t row_bytes = (uint32_t)P * PB;
  uint32_t wsrc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int f = lane + 64 * j;
    const int row = f / CB, pc = f % CB;
    const int n = n0 + row < N ? n0 + row : N - 1;
    wsrc[j] = (uint32_t)n * row_bytes + (uint32_t)(pc * PS);
  }
  bool wvalid[T];
#pragma unroll
  for (int t = 0; t < T; ++t) wvalid[t] = n0 + 16 * t + r16 < N;
  // Loads of chunks past the wave's range go through a resource of zero
  // bytes.  (Sizes and offsets pass through readfirstlane so the resources
  // stay in scalar registers.)
  const uint32_t w_bytes = (uint32_t)N * row_bytes;
  const uint32_t x_bytes = (uint32_t)M * (uint32_t)K * (uint32_t)sizeof(XT);

  // Activation rows past M read row 0: an activation row only feeds its own
  // output row, and output rows past M are never stored, so no masking.
  uint32_t xrow[MT];  // element offset of the lane's activation row
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r16;
    xrow[mt] = (uint32_t)(m < M ? m : 0) * (uint32_t)K;
  }

  // Activation registers of one chunk: per pair, per tile, per block half,
  // the 8 k values of the lane's slot (f32: 8 floats, f16: 4 dwords).
  typedef float XC32[CHP][MT][2][8];
  typedef uint32_t XC16[CHP][MT][2][4];
  typedef typename std::conditional<kF32, XC32, XC16>::type XChunkT;
  // Chunk c's loads: activations, then weights (chunks at or past c_end
  // through the empty resource).
  auto load_x = [&](int c, XChunkT& xb) {
    const __amdgpu_buffer_rsrc_t r = sk_rsrc(A, __builtin_amdgcn_readfirstlane(c < c_end ? x_bytes : 0u));
    const uint32_t cbase = __builtin_amdgcn_readfirstlane((uint32_t)(c * CHP * 64) * (uint32_t)sizeof(XT));
#pragma unroll
    for (int pi = 0; pi < CHP; ++pi)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t o = (xrow[mt] + pi * 64 + h * 32) * (uint32_t)sizeof(XT);
          if constexpr (kF32) {
            const float4v v0 = __builtin_bit_cast(float4v, sk_buf_load<16>(r, o + 4 * SkK<QF>::off0(s), cbase));
            const float4v v1 = __builtin_bit_cast(float4v, sk_buf_load<16>(r, o + 4 * SkK<QF>::off1(s), cbase));
            xb[pi][mt][h][0] = v0.x; xb[pi][mt][h][1] = v0.y; xb[pi][mt][h][2] = v0.z; xb[pi][mt][h][3] = v0.w;
            xb[pi][mt][h][4] = v1.x; xb[pi][mt][h][5] = v1.y; xb[pi][mt][h][6] = v1.z; xb[pi][mt][h][7] = v1.w;
          } else {
            const uint2 v0 = sk_buf_load<8>(r, o + 2 * SkK<QF>::off0(s), cbase);
            const uint2 v1 = sk_buf_load<8>(r, o + 2 * SkK<QF>::off1(s), cbase);
            xb[pi][mt][h][0] = v0.x; xb[pi][mt][h][1] = v0.y; xb[pi][mt][h][2] = v1.x; xb[pi][mt][h][3] = v1.y;
          }
        }
  };
  auto fetch_w = [&](int c, PieceT (&wr)[J]) {
    const __amdgpu_buffer_rsrc_t r = sk_rsrc(W, __builtin_amdgcn_readfirstlane(c < c_end ? w_bytes : 0u));
    const uint32_t cbase = __builtin_amdgcn_readfirstlane((uint32_t)c * CHP * PB);
#pragma unroll
    for (int j = 0; j < J; ++j) wr[j] = sk_buf_load<PS>(r, wsrc[j], cbase);
  };
  auto write_w = [&](const PieceT (&wr)[J]) {
#pragma unroll
    for (int j = 0; j < J; ++j) *reinterpret_cast<PieceT*>(wst + (lane + 64 * j) * (PS / 4)) = wr[j];
  };
  // The slot dwords of staged pair pi (of the chunk) of tile t's row r16.
  auto read_w = [&](int pi, int t, uint32_t (&w)[WL]) {
    const uint32_t* pr = wst + (16 * t + r16) * PITCH + pi * (PB / 4);
    if constexpr (WL == 5) {
      w[0] = pr[s]; w[1] = pr[s + 1]; w[2] = pr[5 + s]; w[3] = pr[0]; w[4] = pr[4];
    } else {
      w[0] = pr[2 * s]; w[1] = pr[2 * s + 1]; w[2] = pr[2 * s + 2];
      w[3] = pr[9 + 2 * s]; w[4] = pr[10 + 2 * s]; w[5] = pr[0]; w[6] = pr[8];
    }
  };

  float4v acc[MT][T];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[mt][t] = float4v{0.f, 0.f, 0.f, 0.f};


  // One staged chunk: CHP pairs x 2 blocks x T tiles x MT activation tiles.
  auto compute = [&](const XChunkT& xc) {
#pragma unroll
    for (int pi = 0; pi < CHP; ++pi)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (kF32) {
          bf16x8 a1[MT], a2[MT];
          float4v base[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            split2(xc[pi][mt][h], a1[mt], a2[mt]);
            base[mt] = float4v{0.f, 0.f, 0.f, 0.f};
            if constexpr (kQ4) {
              // sum_k (-136) * x, the offset of the 128 + n codes, shared by
              // all weight tiles
              const __bf16 c8 = (__bf16)(-136.0f);
              const bf16x8 bc = {c8, c8, c8, c8, c8, c8, c8, c8};
              base[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[mt], bc, base[mt], 0, 0, 0);
              base[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[mt], bc, base[mt], 0, 0, 0);
            }
          }
#pragma unroll
          for (int t = 0; t < T; ++t) {
            uint32_t w[WL];
            read_w(pi, t, w);
            const bf16x8 b = sk_b_codes<QF>(w, h);
            float d = h2f_bits((uint16_t)sk_scale_bits<QF>(w, h));
            if (!wvalid[t]) d = 0.f;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              float4v dd = base[mt];
              dd = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[mt], b, dd, 0, 0, 0);
              dd = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[mt], b, dd, 0, 0, 0);
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[mt][t][i] = __builtin_fmaf(d, dd[i], acc[mt][t][i]);
            }
          }
        } else {
#pragma unroll
          for (int t = 0; t < T; ++t) {
            uint32_t w[WL];
            read_w(pi, t, w);
            half8 b = sk_b_f16<QF>(w, h);
            if (!wvalid[t]) b = half8{};
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const u32x4 av = {xc[pi][mt][h][0], xc[pi][mt][h][1], xc[pi][mt][h][2], xc[pi][mt][h][3]};
              acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, av), b, acc[mt][t], 0, 0, 0);
            }
          }
        }
      }
  };

  // Chunk pipeline.  Loads complete in issue order; per chunk the issue
  // order is x(c), W(c).  Chunk c computes while x(c+1) and W(c+1) are in
  // flight; the wait is the LDS write of W(c+1) at the top of the next
  // chunk.  Two activation and two weight register sets alternate: the loop
  // body takes two chunks with no branch inside (so the compiler neither
  // moves loads behind a branch nor loses its wait counts), and an odd last
  // chunk, whose loads the last pass already issued, is computed after the
  // loop.  Loads past the wave's range go through the empty resource (zeros,
  // no memory traffic).  (Measured and not kept: weights two chunks ahead,
  // +/- 5 % by shape at 24-34 more registers.)
  if (c_begin < c_end) {
    XChunkT xa, xb;
    PieceT wA[J], wB[J];
    load_x(c_begin, xa);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order x, W
    fetch_w(c_begin, wA);
    int c = c_begin;
    for (; c + 1 < c_end; c += 2) {
      __builtin_amdgcn_sched_barrier(0);
      write_w(wA);
      __builtin_amdgcn_sched_barrier(0);
      load_x(c + 1, xb);
      __builtin_amdgcn_sched_barrier(0);
      fetch_w(c + 1, wB);
      __builtin_amdgcn_sched_barrier(0);
      compute(xa);
      __builtin_amdgcn_sched_barrier(0);
      write_w(wB);
      __builtin_amdgcn_sched_barrier(0);
      load_x(c + 2, xa);
      __builtin_amdgcn_sched_barrier(0);
      fetch_w(c + 2, wA);
      __builtin_amdgcn_sched_barrier(0);
      compute(xb);
    }
    if (c < c_end) {
      __builtin_amdgcn_sched_barrier(0);
      write_w(wA);
      __builtin_amdgcn_sched_barrier(0);
      compute(xa);
    }
  }

  // Combine the KS partial sums: each wave writes its accumulators into its
  // own LDS area (value v = ((mt * T + t) * 4 + i) * 64 + lane), then every
  // thread sums values v = tid, tid + 64*KS, ... over the waves in a fixed
  // order (deterministic) and stores them.
  float* part = reinterpret_cast<float*>(wst);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[((mt * T + t) * 4 + i) * 64 + lane] = acc[mt][t][i];
  __syncthreads();
  const float* parts = reinterpret_cast<const float*>(smem);
  auto store = [&](int v, float sum) {
    const int l = v & 63, q = v >> 6;  // q = (mt * T + t) * 4 + i
    const int i = q & 3, t = (q >> 2) % T, mt = (q >> 2) / T;
    const int n = n0 + 16 * t + (l & 15), m = 16 * mt + 4 * (l >> 4) + i;
    if (n < N && m < M) C[(size_t)m * N + n] = (XT)sum;
  };
  if (KG == 1) {
    for (int v = tid; v < NV * 64; v += blockDim.x) {
      float sum = 0.f;
      for (int w = 0; w < KS; ++w) sum += parts[(size_t)w * AREA + v];
      store(v, sum);
    }
    return;
  }
  // Split K across workgroups: each workgroup parks its tile sum in the
  // workspace; the last one to arrive (per-tile counter) adds the KG partial
  // tiles in order kg = 0..KG-1 and stores C, then resets the counter for
  // the next launch.
  float* mine = ws_part + ((size_t)blockIdx.x * KG + kg) * (NV * 64);
  for (int v = tid; v < NV * 64; v += blockDim.x) {
    float sum = 0.f;
    for (int w = 0; w < KS; ++w) sum += parts[(size_t)w * AREA + v];
    // agent-scope atomic store: an sc1 store, written through to the level
    // all XCDs share (the exchange protocol of CoherentTile)
    __hip_atomic_store(&mine[v], sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // Every wave waits for its stores to complete (the workgroup barrier alone
  // does not); one thread then bumps the tile counter (relaxed: the partials
  // never sit in an XCD's L2, so no writeback or invalidate is needed), and
  // the last workgroup reads them back with agent-scope atomic (sc1) loads.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ uint32_t is_last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ws_cnt[blockIdx.x], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == (uint32_t)(KG - 1);
  }
  __syncthreads();
  if (!is_last) return;
  const float* tile = ws_part + (size_t)blockIdx.x * KG * (NV * 64);
  for (int v = tid; v < NV * 64; v += blockDim.x) {
    float sum = 0.f;
    for (int g = 0; g < KG; ++g)
      sum += __hip_atomic_load(&tile[(size_t)g * (NV * 64) + v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    store(v, sum);
  }
  if (tid == 0) __hip_atomic_store(&ws_cnt[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// skinny_ring_kernel: f32 activations, up to 64 rows in one pass, weights
// streamed into an LDS ring by buffer loads to LDS.
//
// A workgroup is 8 waves (two per SIMD) over 128*T weight rows (wave w: rows
// 16T*w .. 16T*w + 16T-1 as T 16-row tiles), and all waves walk the same K
// range chunk by chunk; a chunk is CHP pairs (64*CHP elements).  The weight
// ring has S stages; chunk i+S-1 is requested while chunk i is computed, by
// buffer_load ... lds, which writes LDS without passing through registers
// (so S-1 chunks in flight cost no registers), range-checked: chunks past
// the workgroup's range read through a resource of zero bytes (zeros, no
// memory traffic).  A weight row's staged pairs are 9 (17) dwords apart, an
// odd stride, so the 16 rows of a tile read 16 different banks.
//
// The activations (16*MT rows, rows past M repeating row M-1, whose outputs
// are never stored) are L2-resident: each thread loads the 8 values of its
// A operand(s) of chunk i+1 into registers while chunk i computes, and after
// chunk i splits them once for the whole workgroup into the two bf16 pieces
// of the MFMA operand (x ~ b1 + b2, split2), stored in operand order in one
// of two LDS buffers, so a wave reads each piece with one conflict-free
// ds_read_b128.  Every wave then runs skinny_kernel's f32 MFMA chain on its
// tiles (exact bf16 codes, two chained MFMAs, the block scale applied per
// block in fp32).
//
// With K split over KG workgroups (grid y), each parks its partial tile and
// the last to arrive adds the KG tiles in order kg = 0..KG-1 (deterministic)
// and stores C.
template <class QF, int MT, int T, int CHP>
struct RingGeom {
  static constexpr int kWaves = 8;
  static constexpr int kPB = SkW<QF>::kPairBytes, kPD = kPB / 4;
  static constexpr int kRW = 16 * T;                   // weight rows per wave
  static constexpr int kWRow = CHP * kPD;              // dwords per staged weight row
  static constexpr int kWDw = kRW * kWRow;             // weight dwords of a wave per chunk
  static constexpr int kJW = (kWDw + 63) / 64;         // dword loads per lane per chunk
  // A wave's area in a stage is padded to whole loads: every lane issues all
  // kJW loads (lanes past kWDw reload the last dword into the padding), so
  // no load sits behind a lane-dependent branch, which made the compiler's
  // wait analysis drop count and wait for loads issued an iteration later.
  static constexpr int kWArea = kJW * 64;
  static constexpr int kStage = kWaves * kWArea;       // dwords of a stage
  static constexpr int kUnits = CHP * 2 * MT * 64;     // A operands (lane slots) per chunk
  static constexpr int kUPT = (kUnits + 511) / 512;    // A operands per thread
  static constexpr int kXB = kUnits * 8;               // dwords of one split buffer (two bf16x8 each)
};

// s_waitcnt immediate: vmcnt(v) (6 bits, split), expcnt and lgkmcnt not waited on.
constexpr int sk_vmcnt_imm(int v) { return (v & 15) | ((v >> 4) << 14) | 0x0070 | 0x0F00; }

// Buffer load to LDS: lane i writes lds + 4*i; the builtin exists only in
// the device pass.
__device__ __forceinline__ void sk_dma4(__amdgpu_buffer_rsrc_t r, uint32_t* lds, uint32_t voff, uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, (int)voff,
                                           (int)soff, 0, 0);
#endif
}

// Workgroup barrier without a memory fence (the compiler's fence would wait
// for every outstanding load, including the ring's younger chunks).
__device__ __forceinline__ void sk_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Jobs of one ring launch: job j owns workgroups begin[j] .. begin[j+1]-1,
// tiles[j] row tiles with its own K split kg[j] (tile-major: the kg[j]
// workgroups of a tile are consecutive), and arrival counters
// ctr[j] .. ctr[j] + tiles[j] - 1; a workgroup's partial tile sits at its
// own index in the workspace.
struct RingGroup {
  const uint8_t* W[kSkGroupMax];
  void* C[kSkGroupMax];
  int N[kSkGroupMax];
  int begin[kSkGroupMax + 1];
  int kg[kSkGroupMax];
  int ctr[kSkGroupMax];
};

// Partial-tile loads (float4 per thread) the split-K fix-up keeps in flight.
constexpr int kRingGatherF4 = 16;

// Arguments as skinny_kernel's (job 0's fields first: W0 = grp.W[0], N0,
// KG0 = grp.kg[0], C0, CTR0 = grp.ctr[0]).
template <class QF, int MT, int T, int CHP, int S>
__global__ __launch_bounds__(512) void skinny_ring_kernel(const float* __restrict__ A,
                                                         const uint8_t* __restrict__ W0, int N0, int KG0, int b1,
                                                         int b2, int b3, int M, int K, void* C0, int CTR0,
                                                         float* __restrict__ ws_part,
                                                         uint32_t* __restrict__ ws_cnt, const RingGroup grp) {
  const int job = group_job(b1, b2, b3);
  const uint8_t* __restrict__ W = W0;
  void* Cv = C0;
  int N = N0, wg0 = 0, KG = KG0, ctr0 = CTR0;
  if (job > 0) {
    W = grp.W[job];
    Cv = grp.C[job];
    N = grp.N[job];
    wg0 = grp.begin[job];
    KG = grp.kg[job];
    ctr0 = grp.ctr[job];
  }
  float* __restrict__ C = static_cast<float*>(Cv);
  const int local = (int)blockIdx.x - wg0, tile = local / KG, kg = local - tile * KG;
  typedef RingGeom<QF, MT, T, CHP> G;
  constexpr bool kQ4 = SkW<QF>::kLoads == 5;
  constexpr int WL = SkW<QF>::kLoads;
  constexpr int RW = G::kRW, NW = G::kWaves, UPT = G::kUPT;
  static_assert(S >= 3 && (S - 2) * G::kJW <= 63, "ring depth and the vmcnt field");
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  uint32_t* const xb0 = smem + S * G::kStage;  // split operands, two buffers of kXB dwords

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, s = lane >> 4;
  const int NC = (K >> 6) / CHP;
  const int n0 = tile * (NW * RW) + wave * RW;  // this wave's first row
  const int c_begin = (int)((long)NC * kg / KG), c_end = (int)((long)NC * (kg + 1) / KG);

  // Weight loads: dword f = lane + 64j of the wave's RW x kWRow chunk is row
  // f / kWRow, dword f % kWRow (pairs of a row are contiguous, so the byte
  // offset within the row is 4 * (f % kWRow)); it lands at LDS dword f.
  const uint32_t row_bytes = (uint32_t)(K >> 6) * G::kPB;
  uint32_t wsrc[G::kJW];
#pragma unroll
  for (int j = 0; j < G::kJW; ++j) {
    const int f = lane + 64 * j < G::kWDw ? lane + 64 * j : G::kWDw - 1;
    const int row = f / G::kWRow, dw = f % G::kWRow;
    const int n = n0 + row < N ? n0 + row : N - 1;
    wsrc[j] = (uint32_t)n * row_bytes + (uint32_t)(4 * dw);
  }
  const uint32_t w_bytes = (uint32_t)N * row_bytes;
  auto fetch_w = [&](int c, int st) {
    const bool live = c < c_end;
    const __amdgpu_buffer_rsrc_t rw = sk_rsrc(W, __builtin_amdgcn_readfirstlane(live ? w_bytes : 0u));
    const uint32_t wo = __builtin_amdgcn_readfirstlane(live ? (uint32_t)c * (uint32_t)(CHP * G::kPB) : 0u);
    uint32_t* wsb = smem + st * G::kStage + wave * G::kWArea;
#pragma unroll
    for (int j = 0; j < G::kJW; ++j) sk_dma4(rw, wsb + 64 * j, wsrc[j], wo);
  };

  // A operands: unit u = ((pi * 2 + h) * MT + mt) * 64 + l is the operand of
  // lane l (row 16mt + l%16, slot l/16) for block h of pair pi of a chunk:
  // activations k = 64pi + 32h + {off0 .. off0+3, off1 .. off1+3} of its row
  // (the k order of the lane's weight codes).  Thread tid takes units tid,
  // tid + 512, ...; piece k (0: hi, 1: lo) of unit u goes to 16-byte slot
  // ((u / 64) * 2 + k) * 64 + l of a split buffer, so a wave's read of one
  // piece covers 1 KB contiguously.
  uint32_t xoff[UPT];
  bool xlive[UPT];
#pragma unroll
  for (int k = 0; k < UPT; ++k) {
    const int u = tid + 512 * k;
    xlive[k] = G::kUnits % 512 == 0 || u < G::kUnits;
    const int uu = xlive[k] ? u : 0;
    const int l = uu & 63, mt = (uu >> 6) % MT, ph = (uu >> 6) / MT, h = ph & 1, pi = ph >> 1;
    const int m = 16 * mt + (l & 15);
    const int mm = m < M ? m : M - 1;
    xoff[k] = ((uint32_t)mm * (uint32_t)K + (uint32_t)(64 * pi + 32 * h + (kQ4 ? 4 : 8) * (l >> 4))) * 4u;
  }
  const uint32_t x_bytes = (uint32_t)M * (uint32_t)K * 4u;
  typedef float4v XSet[UPT][2];
  XSet xr[2];  // activations of two chunks in registers (two chunks ahead)
  auto load_x = [&](int c, XSet& x) {
    const bool live = c < c_end;
    const __amdgpu_buffer_rsrc_t rx = sk_rsrc(A, __builtin_amdgcn_readfirstlane(live ? x_bytes : 0u));
    const uint32_t xo = __builtin_amdgcn_readfirstlane(live ? (uint32_t)c * (CHP * 256u) : 0u);
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      x[k][0] = __builtin_bit_cast(float4v, sk_buf_load<16>(rx, xoff[k], xo));
      x[k][1] = __builtin_bit_cast(float4v, sk_buf_load<16>(rx, xoff[k] + (kQ4 ? 64u : 16u), xo));
    }
  };
  auto split_x = [&](uint32_t* xb, const XSet& x) {
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      if (xlive[k]) {
        const int u = tid + 512 * k;
        const float xv[8] = {x[k][0].x, x[k][0].y, x[k][0].z, x[k][0].w,
                             x[k][1].x, x[k][1].y, x[k][1].z, x[k][1].w};
        bf16x8 a1, a2;
        split2(xv, a1, a2);
        uint32_t* dst = xb + (((u >> 6) * 2) * 64 + (u & 63)) * 4;
        *reinterpret_cast<bf16x8*>(dst) = a1;
        *reinterpret_cast<bf16x8*>(dst + 256) = a2;
      }
    }
  };

  bool wvalid[T];
#pragma unroll
  for (int t = 0; t < T; ++t) wvalid[t] = n0 + 16 * t + r16 < N;

  float4v acc[MT][T];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < T; ++t) acc[mt][t] = float4v{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int st, const uint32_t* xb) {
    const uint32_t* wsb = smem + st * G::kStage + wave * G::kWArea;
#pragma unroll
    for (int pi = 0; pi < CHP; ++pi)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        bf16x8 a1[MT], a2[MT];
        float4v base[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint32_t* up = xb + ((((pi * 2 + h) * MT + mt) * 2) * 64 + lane) * 4;
          a1[mt] = *reinterpret_cast<const bf16x8*>(up);
          a2[mt] = *reinterpret_cast<const bf16x8*>(up + 256);
          base[mt] = float4v{0.f, 0.f, 0.f, 0.f};
          if constexpr (kQ4) {
            // sum_k (-136) * x, the offset of the 128 + n codes, shared by
            // all weight tiles
            const __bf16 c8 = (__bf16)(-136.0f);
            const bf16x8 bc = {c8, c8, c8, c8, c8, c8, c8, c8};
            base[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[mt], bc, base[mt], 0, 0, 0);
            base[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[mt], bc, base[mt], 0, 0, 0);
          }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint32_t* pr = wsb + (16 * t + r16) * G::kWRow + pi * G::kPD;
          uint32_t w[WL];
          if constexpr (WL == 5) {
            w[0] = pr[s]; w[1] = pr[s + 1]; w[2] = pr[5 + s]; w[3] = pr[0]; w[4] = pr[4];
          } else {
            w[0] = pr[2 * s]; w[1] = pr[2 * s + 1]; w[2] = pr[2 * s + 2];
            w[3] = pr[9 + 2 * s]; w[4] = pr[10 + 2 * s]; w[5] = pr[0]; w[6] = pr[8];
          }
          const bf16x8 b = sk_b_codes<QF>(w, h);
          float d = h2f_bits((uint16_t)sk_scale_bits<QF>(w, h));
          if (!wvalid[t]) d = 0.f;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            float4v dd = base[mt];
            dd = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[mt], b, dd, 0, 0, 0);
            dd = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[mt], b, dd, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mt][t][i] = __builtin_fmaf(d, dd[i], acc[mt][t][i]);
          }
        }
      }
  };

  // Pipeline.  Before the loop: chunk 0's activations, the weights of
  // chunks c_begin .. c_begin+S-3, chunk 1's activations and chunk S-2's
  // weights go out, in that order (the order of the loop's own issue, so the
  // loads pending at the loop entry match those pending around the loop and
  // the compiler's waits stay exact), and chunk 0 is split.  Iteration i
  // (activation register set p = i & 1):
  //   wait for chunk i's weights and for its own split stores, then one
  //   barrier makes chunk i's weights and split operands visible and retires
  //   chunk i-1 (its stage receives chunk i+S-1, its split buffer the split
  //   of chunk i+1);
  //   chunk i+2's activations are requested into set p (chunk i's, split in
  //   iteration i-1), then chunk i+S-1's weights;
  //   chunk i computes, and chunk i+1 (set p^1, requested one iteration
  //   earlier) is split.
  // Loads complete in issue order, so the activations are requested two
  // chunks ahead: the split's wait then covers only loads issued an
  // iteration earlier (with them one chunk ahead, it also waited for the
  // weight loads issued just before them).  Measured on MI355X with the
  // batched fix-up below (same box, against the previous kernel): Llama-3-8B
  // Q8_0 decode step 5.31 -> 5.17 ms at M = 64, 3.32 -> 3.11 ms at M = 16,
  // TinyLlama Q4_0 M = 16 961 -> 940 us; 14336 x 4096 at M = 64 stays at
  // about 1.4 us per chunk, which the load order therefore does not set.  Every thread issues the same loads per
  // chunk (2 * UPT activation, kJW weight), so the counts below are exact:
  // after chunk i's weights come at most S-2 chunks of weight loads and one
  // of activation loads.
  static_assert((S - 2) * G::kJW + 2 * UPT <= 63, "vmcnt field");
  const int nch = c_end - c_begin;
  load_x(c_begin, xr[0]);
#pragma unroll
  for (int i = 0; i < S - 2; ++i) fetch_w(c_begin + i, i);
  load_x(c_begin + 1, xr[1]);
  fetch_w(c_begin + S - 2, S - 2);
  split_x(xb0, xr[0]);
  auto iteration = [&](auto pc, int i) {
    constexpr int p = decltype(pc)::value;
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(sk_vmcnt_imm((S - 2) * G::kJW + 2 * UPT) & ~0x0F00);
    sk_barrier();
    load_x(c_begin + i + 2, xr[p]);
    __builtin_amdgcn_sched_barrier(0);
    fetch_w(c_begin + i + S - 1, (i + S - 1) % S);
    __builtin_amdgcn_sched_barrier(0);
    compute(i % S, xb0 + p * G::kXB);
    __builtin_amdgcn_sched_barrier(0);
    split_x(xb0 + (p ^ 1) * G::kXB, xr[p ^ 1]);
  };
  int i = 0;
  for (; i + 2 <= nch; i += 2) {
    iteration(std::integral_constant<int, 0>{}, i);
    iteration(std::integral_constant<int, 1>{}, i + 1);
  }
  if (i < nch) iteration(std::integral_constant<int, 0>{}, i);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  auto store = [&](int mt, int t, int i, float v) {
    const int n = n0 + 16 * t + r16, m = 16 * mt + 4 * s + i;
    if (n < N && m < M) C[(size_t)m * N + n] = v;
  };
  if (KG == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) store(mt, t, i, acc[mt][t][i]);
    return;
  }
  // K split across workgroups: park this tile (float4 (mt*T + t) of thread
  // tid at index (mt*T + t) * 512 + tid, sc1 stores), count arrivals; the
  // last workgroup reads the KG tiles back and adds them in order kg =
  // 0..KG-1.  The loads of up to GB tiles are issued before any of them is
  // added: each load is a round trip to the level all XCDs share, so one
  // tile per round trip made the fix-up of a 16-way split take about 16 of
  // them.
  constexpr int NQ = MT * T;
  const CoherentTile tile_ws(reinterpret_cast<float4v*>(ws_part) + (size_t)(wg0 + tile * KG) * (NQ * 512),
                             (uint32_t)(KG * NQ * 512 * 16));
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < T; ++t) tile_ws.store((uint32_t)kg * (NQ * 512) + (mt * T + t) * 512 + tid, acc[mt][t]);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ uint32_t is_last;
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(&ws_cnt[ctr0 + tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == (uint32_t)(KG - 1);
  }
  __syncthreads();
  if (!is_last) return;
  constexpr int GB = NQ >= kRingGatherF4 ? 1 : kRingGatherF4 / NQ;
  for (int g0 = 0; g0 < KG; g0 += GB) {
    float4v p[GB][MT][T];
#pragma unroll
    for (int gb = 0; gb < GB; ++gb) {
      const int g = g0 + gb;
      if (g < KG) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < T; ++t) p[gb][mt][t] = tile_ws.load((uint32_t)g * (NQ * 512) + (mt * T + t) * 512 + tid);
      }
    }
#pragma unroll
    for (int gb = 0; gb < GB; ++gb) {
      const int g = g0 + gb;
      if (g < KG) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < T; ++t) acc[mt][t] = g == 0 ? p[gb][mt][t] : acc[mt][t] + p[gb][mt][t];
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) store(mt, t, i, acc[mt][t][i]);
  if (tid == 0) __hip_atomic_store(&ws_cnt[ctr0 + tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Ring geometry per format, activation tiles (MT) and weight tiles per wave
// (T): two pairs per chunk with one activation tile, else one; as many
// stages as fit in 160 KB of LDS beside the two split buffers, at most 4, at
// least 3.
template <class QF, int MT, int T>
struct RingCfg {
  static constexpr int kCHP = MT == 1 ? 2 : 1;
  typedef RingGeom<QF, MT, T, kCHP> G;
  static constexpr int kFree = 160 * 1024 / 4 - 2 * G::kXB - 64;  // dwords (64 for the static LDS)
  static constexpr int kSLds = kFree / G::kStage, kSVm = 2 + (63 - 2 * G::kUPT) / G::kJW;  // LDS, vmcnt field
  static constexpr int kSMax = 4;  // deeper rings measured slower (fewer workgroups per CU)
  static constexpr int kS = kSLds < kSVm ? (kSLds < kSMax ? kSLds : kSMax) : (kSVm < kSMax ? kSVm : kSMax);
  static constexpr bool kOk = kS >= 3;
  static constexpr int kLds = (kS * G::kStage + 2 * G::kXB) * 4;
};

// Weight tiles per wave: the largest of 4, 2, 1 whose ring fits with at
// least 128 row groups (so a matrix spreads over the CUs with few K splits),
// else 1.
template <class QF, int MT>
int ring_t(uint32_t N) {
  static const int forced = [] {
    const char* e = std::getenv("NF_HIP_RING_T");  // tuning override: 1, 2 or 4
    const int v = e ? std::atoi(e) : 0;
    return (v == 1 || v == 2 || v == 4) ? v : 0;
  }();
  if (forced == 4 && RingCfg<QF, MT, 4>::kOk) return 4;
  if (forced == 2 && RingCfg<QF, MT, 2>::kOk) return 2;
  if (forced == 1) return 1;
  if (RingCfg<QF, MT, 4>::kOk && N >= 128u * 512u) return 4;
  if (RingCfg<QF, MT, 2>::kOk && N >= 128u * 256u) return 2;
  return 1;
}

// Workgroups per row group (kg): up to about 256 workgroups in all, at
// least `min_chunks` chunks each (2 where a row's whole K is at most 16
// chunks, else 4), within the workspace.  The short-K rows are the
// latency-bound ones, and two chunks per workgroup halve each workgroup's
// chain: TinyLlama decode step at M = 16 884 -> 854 us (2048-row linears at
// K = 2048: 8 splits instead of 4, the q+k+v launch 160 workgroups).  At
// K = 4096 two chunks measured slower (Llama-3-8B Q8_0 step at M = 16: 2.94
// -> 3.05 ms, its k / v rows taking 16 splits and the q+k+v launch 384
// workgroups).  The choice depends on the job alone, so a grouped launch
// splits every job as its own launch would.
template <class QF, int MT, int T>
int ring_split(long tiles, uint32_t K, const nfhip::Workspace& ws) {
  typedef RingCfg<QF, MT, T> Cfg;
  constexpr int NQ = MT * T;
  const int NC = (int)(K / (64 * Cfg::kCHP));
  static const long target = [] {
    const char* e = std::getenv("NF_HIP_RING_WGS");  // tuning override
    const long v = e ? std::atol(e) : 0;
    return v > 0 ? v : 256L;
  }();
  static const int forced_min = [] {
    const char* e = std::getenv("NF_HIP_RING_MIN_CHUNKS");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 ? v : 0;
  }();
  const int min_chunks = forced_min ? forced_min : (NC <= 16 ? 2 : 4);
  int kg = 1;
  while (tiles * kg * 2 <= target && NC >= min_chunks * kg * 2 && tiles <= (long)ws.cnt_len &&
         (size_t)tiles * kg * 2 * NQ * 512 * 4 <= ws.part_floats)
    kg *= 2;
  // Longer K ranges (at least 8 chunks) where the launch keeps at least 128
  // workgroups: each split adds a partial tile written and read back.
  // Measured on MI355X: Llama-3-8B Q8_0 decode step at M = 16 3.11 ->
  // 3.01 ms (4096-row linears at K = 4096: 4 splits of 8 chunks instead of 8
  // of 4); TinyLlama at M = 16 keeps its splits (fewer workgroups there
  // took the step from 0.94 to 1.12 ms).
  while (kg > 1 && NC / kg < 8 && tiles * (kg / 2) >= 128) kg /= 2;
  return kg;
}

template <class QF, int MT, int T>
hipError_t ring_launch_group(const float* A, const RingGroup& grp, long wgs, uint32_t M, uint32_t K,
                             const nfhip::Workspace& ws, hipStream_t s) {
  typedef RingCfg<QF, MT, T> Cfg;
  if constexpr (!Cfg::kOk) {
    return hipErrorNotSupported;
  } else {
    constexpr int CHP = Cfg::kCHP, S = Cfg::kS;
    if ((K / 64) % CHP != 0) return hipErrorNotSupported;
    static const hipError_t attr =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&skinny_ring_kernel<QF, MT, T, CHP, S>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::kLds);
    if (attr != hipSuccess) return attr;
    skinny_ring_kernel<QF, MT, T, CHP, S><<<dim3((unsigned)wgs), dim3(512), Cfg::kLds, s>>>(
        A, grp.W[0], grp.N[0], grp.kg[0], grp.begin[1], grp.begin[2], grp.begin[3], (int)M, (int)K, grp.C[0],
        grp.ctr[0], ws.part, ws.cnt, grp);
    return hipGetLastError();
  }
}

// One launch for n jobs (n = 1: a single linear) over the same activations,
// each with the geometry and K split a launch of its own would get (so its
// output is bit-identical to that launch); hipErrorNotSupported if the
// jobs need different row tiles per wave or exceed the workspace.
template <class QF, int MT, int T>
hipError_t ring_group_t(const float* A, const nfhip::GemvJob* jobs, uint32_t n, uint32_t M, uint32_t K,
                        const nfhip::Workspace& ws, hipStream_t s) {
  RingGroup grp{};
  long wgs = 0, tiles = 0;
  bool split = false;
  for (uint32_t j = 0; j < n; ++j) {
    if (ring_t<QF, MT>(jobs[j].N) != T) return hipErrorNotSupported;
    const long t = ((long)jobs[j].N + 128 * T - 1) / (128 * T);
    const int kg = ring_split<QF, MT, T>(t, K, ws);
    split = split || kg > 1;
    grp.W[j] = static_cast<const uint8_t*>(jobs[j].W);
    grp.C[j] = jobs[j].C;
    grp.N[j] = (int)jobs[j].N;
    grp.begin[j] = (int)wgs;
    grp.kg[j] = kg;
    grp.ctr[j] = (int)tiles;
    wgs += t * kg;
    tiles += t;
  }
  if (split && (tiles > (long)ws.cnt_len || (size_t)wgs * MT * T * 512 * 4 > ws.part_floats))
    return hipErrorNotSupported;
  for (int q = (int)n; q <= kSkGroupMax; ++q) grp.begin[q] = (int)wgs;
  return ring_launch_group<QF, MT, T>(A, grp, wgs, M, K, ws, s);
}

template <class QF, int MT>
hipError_t ring_group(const float* A, const nfhip::GemvJob* jobs, uint32_t n, uint32_t M, uint32_t K,
                      const nfhip::Workspace& ws, hipStream_t s) {
  switch (ring_t<QF, MT>(jobs[0].N)) {
    case 1: return ring_group_t<QF, MT, 1>(A, jobs, n, M, K, ws, s);
    case 2: return ring_group_t<QF, MT, 2>(A, jobs, n, M, K, ws, s);
    default: return ring_group_t<QF, MT, 4>(A, jobs, n, M, K, ws, s);
  }
}

template <class QF>
hipError_t ring_dispatch(const float* A, const nfhip::GemvJob* jobs, uint32_t n, uint32_t M, uint32_t K,
                         const nfhip::Workspace& ws, hipStream_t s) {
  if (M <= 16) return ring_group<QF, 1>(A, jobs, n, M, K, ws, s);
  if (M <= 32) return ring_group<QF, 2>(A, jobs, n, M, K, ws, s);
  return ring_group<QF, 4>(A, jobs, n, M, K, ws, s);
}

// The ring kernel serves f32 activations unless turned off for comparison
// (NF_HIP_SKINNY_RING=0).
inline bool ring_on() {
  static const bool on = [] {
    const char* e = std::getenv("NF_HIP_SKINNY_RING");
    return !(e && e[0] == '0');
  }();
  return on;
}

// Waves per workgroup (ks) and workgroups per row tile (kg) for a launch of
// `wgs` row tiles, bounded by the kernel's launch bound of 512 threads, by
// at least one chunk per wave and by the workspace: 8 waves per workgroup up
// to 256 row tiles, else 4; then up to 4 workgroups per row tile while the
// launch stays within 2048 waves.  Measured on MI355X at M = 8 and 16 (waves
// x kg sweep): with a few chunks per wave each wave pays about one memory
// round trip per chunk, so spreading K over more waves pays for the fix-up:
// Llama-3-8B Q8_0 4096x14336 f32 72 -> 33 us, 4096x4096 25 -> 15 us;
// Llama-7B Q4_0 4096x11008 f16 45 -> 22 us; 8192x28672 f16 92 -> 60 us;
// TinyLlama 2048x5632 f32 18 -> 13 us.  Row-rich shapes (11264 rows and up)
// stay at kg = 1, with 4 waves once past 256 row tiles (28672x4096 f32: 47
// against 53 us with 8).
template <int MT, int CHP>
void skinny_split(long wgs, uint32_t K, const nfhip::Workspace& ws, int& ks, int& kg) {
  constexpr int NV = MT * 4 * 4;
  const int NC = (int)(K / (64 * CHP));
  static const int ks_max = [] {
    const char* e = std::getenv("NF_HIP_SKINNY_KS_MAX");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 && v <= 8 ? v : 8;
  }();
  static const int kg_max = [] {
    const char* e = std::getenv("NF_HIP_SKINNY_KG_MAX");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 && v <= 64 ? v : 4;
  }();
  static const int min_chunks = [] {
    const char* e = std::getenv("NF_HIP_SKINNY_MIN_CHUNKS");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 && v <= 8 ? v : 2;
  }();
  static const int max_waves = [] {
    const char* e = std::getenv("NF_HIP_SKINNY_MAX_WAVES");  // tuning override
    const int v = e ? std::atoi(e) : 0;
    return v > 0 ? v : 2048;
  }();
  ks = std::min(ks_max, wgs <= 256 ? 8 : 4);
  while (ks > 1 && NC < ks) ks >>= 1;
  kg = 1;
  while (kg < kg_max && wgs * ks * kg * 2 <= max_waves && NC >= min_chunks * ks * kg && wgs <= (long)ws.cnt_len &&
         (size_t)wgs * 2 * kg * NV * 64 <= ws.part_floats)
    kg *= 2;
}

template <class QF, typename XT, int MT, int CHP>
hipError_t skinny_launch_group(const void* A, const SkinnyGroup& grp, long tiles, uint32_t M, uint32_t K, int ks,
                               int kg, const nfhip::Workspace& ws, hipStream_t s) {
  constexpr int RW = 64, PITCH = CHP * SkW<QF>::kPairBytes / 4, NV = MT * 4 * 4;
  constexpr int AREA = RW * PITCH > NV * 64 ? RW * PITCH : NV * 64;  // dwords per wave
  if (kg > 1 && (tiles > (long)ws.cnt_len || (size_t)tiles * kg * NV * 64 > ws.part_floats))
    return hipErrorNotSupported;
  const size_t lds = (size_t)ks * AREA * 4;
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&skinny_kernel<QF, XT, MT, CHP>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024);
  if (attr != hipSuccess) return attr;
  skinny_kernel<QF, XT, MT, CHP><<<dim3((unsigned)tiles, (unsigned)kg), dim3(64 * ks), lds, s>>>(
      static_cast<const XT*>(A), grp.W[0], grp.N[0], grp.begin[1], grp.begin[2], grp.begin[3], (int)M, (int)K,
      grp.C[0], ws.part, ws.cnt, grp);
  return hipGetLastError();
}

template <class QF, typename XT, int MT, int CHP>
hipError_t skinny_launch(const void* A, const void* W, void* C, uint32_t M, uint32_t N, uint32_t K,
                         const nfhip::Workspace& ws, hipStream_t s) {
  const long wgs = ((long)N + 63) / 64;
  int ks, kg;
  skinny_split<MT, CHP>(wgs, K, ws, ks, kg);
  SkinnyGroup grp{};
  grp.W[0] = static_cast<const uint8_t*>(W);
  grp.C[0] = C;
  grp.N[0] = (int)N;
  for (int q = 1; q <= kSkGroupMax; ++q) grp.begin[q] = (int)wgs;
  return skinny_launch_group<QF, XT, MT, CHP>(A, grp, wgs, M, K, ks, kg, ws, s);
}

// A group of jobs goes out as one launch when every job would get the same
// kernel variant and K split on its own (so each output is bit-identical to
// its own launch); otherwise hipErrorNotSupported.
template <class QF, typename XT, int MT, int CHP>
hipError_t skinny_group_same_split(const void* A, const nfhip::GemvJob* jobs, uint32_t n, uint32_t M, uint32_t K,
                                   const nfhip::Workspace& ws, hipStream_t s) {
  SkinnyGroup grp{};
  long tiles = 0;
  int ks0 = 0, kg0 = 0;
  for (uint32_t j = 0; j < n; ++j) {
    const long wgs = ((long)jobs[j].N + 63) / 64;
    int ks, kg;
    skinny_split<MT, CHP>(wgs, K, ws, ks, kg);
    if (j == 0) {
      ks0 = ks;
      kg0 = kg;
    } else if (ks != ks0 || kg != kg0) {
      return hipErrorNotSupported;
    }
    grp.W[j] = static_cast<const uint8_t*>(jobs[j].W);
    grp.C[j] = jobs[j].C;
    grp.N[j] = (int)jobs[j].N;
    grp.begin[j] = (int)tiles;
    tiles += wgs;
  }
  for (int q = (int)n; q <= kSkGroupMax; ++q) grp.begin[q] = (int)tiles;
  return skinny_launch_group<QF, XT, MT, CHP>(A, grp, tiles, M, K, ks0, kg0, ws, s);
}

// Activation tiles per launch (16 rows each) and pairs per staged chunk,
// sized so the two activation register sets and the staged weight pieces
// stay within the register file.
template <class QF, typename XT>
hipError_t skinny_dispatch(const void* A, const void* W, void* C, uint32_t M, uint32_t N, uint32_t K,
                           const nfhip::Workspace& ws, hipStream_t s) {
  constexpr bool kQ4 = SkW<QF>::kLoads == 5;
  // Up to 16 rows: two-pair chunks at every N (4-12 % faster than one-pair
  // chunks at M = 16, and as fast as four-pair ones); 17..32 rows: one-pair
  // chunks for f32 and for f16 with few row tiles, so two activation tiles'
  // registers fit.
  const bool small = N < 64u * 128u;
  if (M <= 16) return skinny_launch<QF, XT, 1, 2>(A, W, C, M, N, K, ws, s);
  if constexpr (sizeof(XT) == 4) {
    return skinny_launch<QF, XT, 2, 1>(A, W, C, M, N, K, ws, s);
  } else {
    if (small) return skinny_launch<QF, XT, 2, 1>(A, W, C, M, N, K, ws, s);
    return skinny_launch<QF, XT, 2, kQ4 ? 2 : 1>(A, W, C, M, N, K, ws, s);
  }
}

// The variant a job gets on its own (skinny_dispatch's choice); a group
// launch needs the same for every job.
template <class QF, typename XT>
int skinny_variant(uint32_t M, uint32_t N) {
  const bool small = N < 64u * 128u;
  if (M <= 16) return 1;
  if constexpr (sizeof(XT) == 4) return 2;
  return small ? 2 : 4;
}

template <class QF, typename XT>
hipError_t skinny_group_dispatch(const void* A, const nfhip::GemvJob* jobs, uint32_t n, uint32_t M, uint32_t K,
                                 const nfhip::Workspace& ws, hipStream_t s) {
  constexpr bool kQ4 = SkW<QF>::kLoads == 5;
  if (n < 1 || n > (uint32_t)kSkGroupMax || M < 1 || M > 32) return hipErrorNotSupported;
  const int v = skinny_variant<QF, XT>(M, jobs[0].N);
  for (uint32_t j = 1; j < n; ++j)
    if (skinny_variant<QF, XT>(M, jobs[j].N) != v) return hipErrorNotSupported;
  if (v == 1) return skinny_group_same_split<QF, XT, 1, 2>(A, jobs, n, M, K, ws, s);
  if (v == 2) return skinny_group_same_split<QF, XT, 2, 1>(A, jobs, n, M, K, ws, s);
  return skinny_group_same_split<QF, XT, 2, kQ4 ? 2 : 1>(A, jobs, n, M, K, ws, s);
}

}  // namespace nfk

namespace nfhip {

hipError_t launch_skinny_group(QFmt q, EType t, const void* A, const GemvJob* jobs, uint32_t n, uint32_t M,
                               uint32_t K, const Workspace& ws, hipStream_t s) {
  for (uint32_t j = 0; j < n; ++j)
    if (!skinny_fits(M, jobs[j].N, K, A, jobs[j].W)) return hipErrorNotSupported;
  if (t == EType::F32 && nfk::ring_on()) {
    const float* a = static_cast<const float*>(A);
    return q == QFmt::Q4_0 ? nfk::ring_dispatch<nfk::Q4_0>(a, jobs, n, M, K, ws, s)
                           : nfk::ring_dispatch<nfk::Q8_0>(a, jobs, n, M, K, ws, s);
  }
  if (q == QFmt::Q4_0)
    return t == EType::F32 ? nfk::skinny_group_dispatch<nfk::Q4_0, float>(A, jobs, n, M, K, ws, s)
                           : nfk::skinny_group_dispatch<nfk::Q4_0, nfk::half_t>(A, jobs, n, M, K, ws, s);
  return t == EType::F32 ? nfk::skinny_group_dispatch<nfk::Q8_0, float>(A, jobs, n, M, K, ws, s)
                         : nfk::skinny_group_dispatch<nfk::Q8_0, nfk::half_t>(A, jobs, n, M, K, ws, s);
}

bool skinny_fits(uint32_t M, uint32_t N, uint32_t K, const void* A, const void* W) {
  // 32-bit in-kernel offsets: weight matrix and activation tile below 4 GB
  const uint64_t wbytes = (uint64_t)N * (K / 32) * 34, abytes = (uint64_t)64 * K * 4;
  return M >= 1 && M <= 64 && K % 256 == 0 && (uintptr_t)A % 16 == 0 && (uintptr_t)W % 16 == 0 &&
         wbytes < (1ull << 32) && abytes < (1ull << 32);
}

// f32 activations: all 64 rows in one pass with the ring kernel (32 with
// skinny_kernel, whose activation registers limit it to two 16-row tiles).
uint32_t skinny_max_rows(EType t) { return (t == EType::F32 && nfk::ring_on()) ? 64u : 32u; }

hipError_t launch_skinny(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M, uint32_t N,
                         uint32_t K, const Workspace& ws, hipStream_t s) {
  if (t == EType::F32 && nfk::ring_on()) {
    const GemvJob job{W, C, N};
    const float* a = static_cast<const float*>(A);
    const hipError_t e = q == QFmt::Q4_0 ? nfk::ring_dispatch<nfk::Q4_0>(a, &job, 1, M, K, ws, s)
                                         : nfk::ring_dispatch<nfk::Q8_0>(a, &job, 1, M, K, ws, s);
    if (e != hipErrorNotSupported) return e;
    // declined (workspace): skinny_kernel, 32 rows per launch
    for (uint32_t m0 = 0; m0 < M; m0 += 32) {
      const uint32_t mc = M - m0 < 32 ? M - m0 : 32;
      const float* am = a + (size_t)m0 * K;
      float* cm = static_cast<float*>(C) + (size_t)m0 * N;
      const hipError_t e2 = q == QFmt::Q4_0 ? nfk::skinny_dispatch<nfk::Q4_0, float>(am, W, cm, mc, N, K, ws, s)
                                            : nfk::skinny_dispatch<nfk::Q8_0, float>(am, W, cm, mc, N, K, ws, s);
      if (e2 != hipSuccess) return e2;
    }
    return hipSuccess;
  }
  if (q == QFmt::Q4_0)
    return t == EType::F32 ? nfk::skinny_dispatch<nfk::Q4_0, float>(A, W, C, M, N, K, ws, s)
                           : nfk::skinny_dispatch<nfk::Q4_0, nfk::half_t>(A, W, C, M, N, K, ws, s);
  return t == EType::F32 ? nfk::skinny_dispatch<nfk::Q8_0, float>(A, W, C, M, N, K, ws, s)
                         : nfk::skinny_dispatch<nfk::Q8_0, nfk::half_t>(A, W, C, M, N, K, ws, s);
}

}  // namespace nfhip
