// dense.hip — dense `linear` / `linear_tiled` with an fp32 operand on the
// fp32 MFMA (metal_provider.mm:150-164, 899-935; host dispatch_linear
// :2544-2613): C[m, n] = sum_k A[m, k] * B[n, k], B stored [N, K], fp32
// products and accumulation (v_mfma_f32_32x32x2_f32), C rounded to its dtype.
// fp16 operands are widened to fp32 exactly when staged, so every dtype mix
// with at least one fp32 input runs here; fp16 x fp16 goes to the fp16 MFMA
// kernel instead.
//
// Workgroup tile 128 x 128, K step 32, 4 waves in a 2 x 2 arrangement, each
// owning 64 x 64 = 2 x 2 tiles of 32 x 32 (64 fp32 accumulators per lane).
// Both operand tiles are staged in LDS as fp32 rows of 32 (128 B, 16-B
// chunks XOR-swizzled by row pair), double buffered: the next step's tiles
// are loaded into registers while the MFMAs of this step run, then written
// to the other stage; one barrier per step.
//
// K order of a step: the MFMA sums over its two k slots, so any permutation
// of the step's 32 k values that A and B share gives the same sum.
// Instruction s (0..15) pairs slot kb (lane group l/32) with k = 16*kb + s,
// so a lane's operands for the whole step are 16 consecutive floats of its
// row (four ds_read_b128).
#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

typedef float float16v __attribute__((ext_vector_type(16)));

namespace {

constexpr int kDBK = 32;

// float offset of 16-B chunk c (0..7) of row r in an operand tile
__device__ __forceinline__ int dslot(int r, int c) { return r * kDBK + ((c ^ ((r >> 1) & 7)) << 2); }

// One operand tile (ROWS rows x 32 elements) per step, register-staged by
// the 256 threads: fp32 rows are 8 chunks of 4 floats, fp16 rows 4 chunks of
// 8 halves (each widened to two fp32 chunks when stored).  Rows past the
// matrix re-read its last valid row (their outputs are never stored).
template <typename T, int ROWS> struct DTile;
template <int ROWS> struct DTile<float, ROWS> {
  static constexpr int kChunks = ROWS * 8;
  static constexpr int kLoads = (kChunks + 255) / 256;
  __device__ static void load(const float* base, size_t ld, int rows_valid, int tid, int ks, u32x4 (&r)[kLoads]) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = (tid + 256 * i) % kChunks, row = id >> 3, c = id & 7;
      const int rr = row < rows_valid ? row : rows_valid - 1;
      r[i] = *reinterpret_cast<const u32x4*>(base + (size_t)rr * ld + (size_t)ks * kDBK + c * 4);
    }
  }
  __device__ static void store(float* tile, int tid, const u32x4 (&r)[kLoads]) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = tid + 256 * i, row = id >> 3, c = id & 7;
      if (kChunks % 256 == 0 || id < kChunks) *reinterpret_cast<u32x4*>(tile + dslot(row, c)) = r[i];
    }
  }
};
template <int ROWS> struct DTile<half_t, ROWS> {
  static constexpr int kChunks = ROWS * 4;
  static constexpr int kLoads = (kChunks + 255) / 256;
  __device__ static void load(const half_t* base, size_t ld, int rows_valid, int tid, int ks, u32x4 (&r)[kLoads]) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = (tid + 256 * i) % kChunks, row = id >> 2, c = id & 3;
      const int rr = row < rows_valid ? row : rows_valid - 1;
      r[i] = *reinterpret_cast<const u32x4*>(base + (size_t)rr * ld + (size_t)ks * kDBK + c * 8);
    }
  }
  __device__ static void store(float* tile, int tid, const u32x4 (&r)[kLoads]) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = tid + 256 * i, row = id >> 2, c = id & 3;
      if (kChunks % 256 == 0 || id < kChunks) {
        const half8 h = __builtin_bit_cast(half8, r[i]);
        const float4v lo = {(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
        const float4v hi = {(float)h[4], (float)h[5], (float)h[6], (float)h[7]};
        *reinterpret_cast<float4v*>(tile + dslot(row, 2 * c)) = lo;
        *reinterpret_cast<float4v*>(tile + dslot(row, 2 * c + 1)) = hi;
      }
    }
  }
};

// Workgroup tile BM x BN = (32*TM*WGM) x (64*(4/WGM)): 4 waves, WGM along
// M, each owning TM x 2 tiles of 32 x 32.  SPLIT: K is split over gridDim.y
// workgroups per tile, which park fp32 partial tiles in the workspace; the
// last to arrive adds them in order and stores C (as in the fused kernels).
template <typename AT, typename BT, typename CT, int TM, int WGM, bool SPLIT>
__global__ __launch_bounds__(256, 2) void dense_f32_mfma_kernel(const AT* __restrict__ A, const BT* __restrict__ B,
                                                                CT* __restrict__ C, int M, int N, int K,
                                                                float* __restrict__ ws_part,
                                                                uint32_t* __restrict__ ws_cnt) {
  constexpr int WGN = 4 / WGM, TN = 2;
  constexpr int BM = 32 * TM * WGM, BN = 64 * WGN, STAGE = (BM + BN) * kDBK;
  __shared__ __attribute__((aligned(16))) float lds[2 * STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, kb = lane >> 5;
  const int wm = (wave / WGN) * 32 * TM, wn = (wave % WGN) * 64;
  const int n_tiles = (N + BN - 1) / BN;
  const int m0 = (int)(blockIdx.x / n_tiles) * BM, n0 = (int)(blockIdx.x % n_tiles) * BN;
  const int KG = SPLIT ? (int)gridDim.y : 1, kg = SPLIT ? (int)blockIdx.y : 0;
  const int nk_all = K / kDBK;
  const int k_first = (int)((long)nk_all * kg / KG);
  const int nk = (int)((long)nk_all * (kg + 1) / KG) - k_first;
  const AT* a_base = A + (size_t)m0 * K + (size_t)k_first * kDBK;
  const BT* b_base = B + (size_t)n0 * K + (size_t)k_first * kDBK;
  const int a_rows = M - m0 < BM ? M - m0 : BM;
  const int b_rows = N - n0 < BN ? N - n0 : BN;

  u32x4 ra[DTile<AT, BM>::kLoads], rb[DTile<BT, BN>::kLoads];
  float16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float16v{};

  DTile<AT, BM>::load(a_base, (size_t)K, a_rows, tid, 0, ra);
  DTile<BT, BN>::load(b_base, (size_t)K, b_rows, tid, 0, rb);
  DTile<AT, BM>::store(lds, tid, ra);
  DTile<BT, BN>::store(lds + BM * kDBK, tid, rb);
  __syncthreads();

  for (int ks = 0; ks < nk; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < nk) {
      DTile<AT, BM>::load(a_base, (size_t)K, a_rows, tid, ks + 1, ra);
      DTile<BT, BN>::load(b_base, (size_t)K, b_rows, tid, ks + 1, rb);
    }
    const float* As = lds + cur * STAGE;
    const float* Bs = As + BM * kDBK;
    float16v av[TM], bv[TN];  // 16 consecutive k of the lane's row
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = wm + 32 * i + r32;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4v t = *reinterpret_cast<const float4v*>(As + dslot(row, 4 * kb + q));
        av[i][4 * q + 0] = t[0];
        av[i][4 * q + 1] = t[1];
        av[i][4 * q + 2] = t[2];
        av[i][4 * q + 3] = t[3];
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int row = wn + 32 * j + r32;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4v t = *reinterpret_cast<const float4v*>(Bs + dslot(row, 4 * kb + q));
        bv[j][4 * q + 0] = t[0];
        bv[j][4 * q + 1] = t[1];
        bv[j][4 * q + 2] = t[2];
        bv[j][4 * q + 3] = t[3];
      }
    }
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], bv[j][s], acc[i][j], 0, 0, 0);
    if (ks + 1 < nk) {
      float* nxt = lds + (cur ^ 1) * STAGE;
      DTile<AT, BM>::store(nxt, tid, ra);
      DTile<BT, BN>::store(nxt + BM * kDBK, tid, rb);
    }
    __syncthreads();
  }

  // accumulator r of lane l in tile (i, j): row (r/4)*8 + (l/32)*4 + r%4, col l%32
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int gn = n0 + wn + 32 * j + r32;
        if (gn >= N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int gm = m0 + wm + 32 * i + (r >> 2) * 8 + kb * 4 + (r & 3);
          if (gm < M) C[(size_t)gm * N + gn] = (CT)acc[i][j][r];
        }
      }
  };
  if constexpr (!SPLIT) {
    store();
    return;
  }
  // Split K: partial tile of this workgroup as 16-B groups (values 4q..4q+3
  // of tile (i, j) of thread tid at float4 index ((i*TN + j)*4 + q)*256 +
  // tid, through sc1 accesses: CoherentTile); the last arrival at the
  // tile counter loads every partial of a 32x32 tile before adding them in
  // order kg = 0..KG-1, stores C and resets the counter.
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
          tile_ws.store((uint32_t)kg * (BM * BN / 4) + ((i * TN + j) * 4 + q) * 256 + tid,
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
  constexpr int kMaxKG = 16;  // the launcher splits K at most 16 ways
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      float4v part[kMaxKG][4];
#pragma unroll
      for (int g = 0; g < kMaxKG; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (g < KG && g != kg) part[g][q] = tile_ws.load((uint32_t)g * (BM * BN / 4) + ((i * TN + j) * 4 + q) * 256 + tid);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float4v sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < kMaxKG; ++g) {
          if (g >= KG) break;
          sum += g == kg ? float4v{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]}
                         : part[g][q];
        }
        acc[i][j][4 * q + 0] = sum[0];
        acc[i][j][4 * q + 1] = sum[1];
        acc[i][j][4 * q + 2] = sum[2];
        acc[i][j][4 * q + 3] = sum[3];
      }
    }
  store();
  if (tid == 0) __hip_atomic_store(&ws_cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tile shape by M (32-row tiles while M <= 64, so small batches do not pay
// for empty rows), then split K over kg = 1, 2, 4, ... 16 workgroups per
// tile: two workgroups per CU (512 slots), time ~ (rounds of 512
// workgroups) x (K steps per workgroup); the smallest kg that minimizes it
// with at least 8 K steps per part, bounded by the workspace.
template <typename AT, typename BT, typename CT, int TM, int WGM>
hipError_t dense_f32_launch_t(const void* A, const void* B, void* C, uint32_t M, uint32_t N, uint32_t K,
                              const nfhip::Workspace& ws, hipStream_t s) {
  constexpr int BM = 32 * TM * WGM, BN = 64 * (4 / WGM);
  const long tiles = (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  if (tiles > (1L << 31) - 1) return hipErrorInvalidConfiguration;
  const int nk = (int)(K / kDBK);
  constexpr long kSlots = 512;
  int kg = 1;
  long best = ((tiles + kSlots - 1) / kSlots) * nk;
  for (int g = 2; g <= 16 && nk / g >= 8 && tiles <= (long)ws.cnt_len && (size_t)tiles * g * BM * BN <= ws.part_floats;
       g *= 2) {
    const long cost = ((tiles * g + kSlots - 1) / kSlots) * ((nk + g - 1) / g);
    if (cost < best) best = cost, kg = g;
  }
  const AT* a = static_cast<const AT*>(A);
  const BT* b = static_cast<const BT*>(B);
  CT* c = static_cast<CT*>(C);
  if (kg == 1)
    dense_f32_mfma_kernel<AT, BT, CT, TM, WGM, false><<<dim3((unsigned)tiles), dim3(256), 0, s>>>(
        a, b, c, (int)M, (int)N, (int)K, ws.part, ws.cnt);
  else
    dense_f32_mfma_kernel<AT, BT, CT, TM, WGM, true><<<dim3((unsigned)tiles, (unsigned)kg), dim3(256), 0, s>>>(
        a, b, c, (int)M, (int)N, (int)K, ws.part, ws.cnt);
  return hipGetLastError();
}

template <typename AT, typename BT, typename CT>
hipError_t dense_f32_launch(const void* A, const void* B, void* C, uint32_t M, uint32_t N, uint32_t K,
                            const nfhip::Workspace& ws, hipStream_t s) {
  if (M <= 64) return dense_f32_launch_t<AT, BT, CT, 1, 1>(A, B, C, M, N, K, ws, s);
  return dense_f32_launch_t<AT, BT, CT, 2, 2>(A, B, C, M, N, K, ws, s);
}

}  // namespace

}  // namespace nfk

namespace nfhip {

hipError_t launch_dense_mfma_f32(EType a, EType b, EType c, const void* A, const void* B, void* C, uint32_t M,
                                 uint32_t N, uint32_t K, const Workspace& ws, hipStream_t s) {
  if (K % nfk::kDBK != 0 || (uintptr_t)A % 16 != 0 || (uintptr_t)B % 16 != 0 || M == 0 || N == 0)
    return hipErrorNotSupported;
  using nfk::half_t;
  if (c == EType::F32) {
    if (a == EType::F32)
      return b == EType::F32 ? nfk::dense_f32_launch<float, float, float>(A, B, C, M, N, K, ws, s)
                             : nfk::dense_f32_launch<float, half_t, float>(A, B, C, M, N, K, ws, s);
    return b == EType::F32 ? nfk::dense_f32_launch<half_t, float, float>(A, B, C, M, N, K, ws, s)
                           : nfk::dense_f32_launch<half_t, half_t, float>(A, B, C, M, N, K, ws, s);
  }
  if (a == EType::F32)
    return b == EType::F32 ? nfk::dense_f32_launch<float, float, half_t>(A, B, C, M, N, K, ws, s)
                           : nfk::dense_f32_launch<float, half_t, half_t>(A, B, C, M, N, K, ws, s);
  return b == EType::F32 ? nfk::dense_f32_launch<half_t, float, half_t>(A, B, C, M, N, K, ws, s)
                         : nfk::dense_f32_launch<half_t, half_t, half_t>(A, B, C, M, N, K, ws, s);
}

}  // namespace nfhip
