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

constexpr int kDBM = 128, kDBN = 128, kDBK = 32;
constexpr int kDStage = (kDBM + kDBN) * kDBK;  // floats per LDS stage

// float offset of 16-B chunk c (0..7) of row r in a stage
__device__ __forceinline__ int dslot(int r, int c) { return r * kDBK + ((c ^ ((r >> 1) & 7)) << 2); }

// One operand tile (128 rows x 32 elements) per step, register-staged: for
// fp32 8 chunks of 4 floats per row (4 per thread), for fp16 4 chunks of 8
// halves per row (2 per thread, each widened to two fp32 chunks).
template <typename T> struct DTile;
template <> struct DTile<float> {
  static constexpr int kLoads = 4;  // 16-B loads per thread per step
  __device__ static void load(const float* base, size_t ld, int rows_valid, int tid, int ks, u32x4 (&r)[kLoads]) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = tid + 256 * i, row = id >> 3, c = id & 7;
      const int rr = row < rows_valid ? row : rows_valid - 1;
      r[i] = *reinterpret_cast<const u32x4*>(base + (size_t)rr * ld + (size_t)ks * kDBK + c * 4);
    }
  }
  __device__ static void store(float* tile, int tid, const u32x4 (&r)[kLoads]) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = tid + 256 * i, row = id >> 3, c = id & 7;
      *reinterpret_cast<u32x4*>(tile + dslot(row, c)) = r[i];
    }
  }
};
template <> struct DTile<half_t> {
  static constexpr int kLoads = 2;
  __device__ static void load(const half_t* base, size_t ld, int rows_valid, int tid, int ks, u32x4 (&r)[kLoads]) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = tid + 256 * i, row = id >> 2, c = id & 3;
      const int rr = row < rows_valid ? row : rows_valid - 1;
      r[i] = *reinterpret_cast<const u32x4*>(base + (size_t)rr * ld + (size_t)ks * kDBK + c * 8);
    }
  }
  __device__ static void store(float* tile, int tid, const u32x4 (&r)[kLoads]) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int id = tid + 256 * i, row = id >> 2, c = id & 3;
      const half8 h = __builtin_bit_cast(half8, r[i]);
      const float4v lo = {(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
      const float4v hi = {(float)h[4], (float)h[5], (float)h[6], (float)h[7]};
      *reinterpret_cast<float4v*>(tile + dslot(row, 2 * c)) = lo;
      *reinterpret_cast<float4v*>(tile + dslot(row, 2 * c + 1)) = hi;
    }
  }
};

template <typename AT, typename BT, typename CT>
__global__ __launch_bounds__(256, 2) void dense_f32_mfma_kernel(const AT* __restrict__ A, const BT* __restrict__ B,
                                                                CT* __restrict__ C, int M, int N, int K) {
  __shared__ __attribute__((aligned(16))) float lds[2 * kDStage];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r32 = lane & 31, kb = lane >> 5;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int n_tiles = (N + kDBN - 1) / kDBN;
  const int m0 = (int)(blockIdx.x / n_tiles) * kDBM, n0 = (int)(blockIdx.x % n_tiles) * kDBN;
  const AT* a_base = A + (size_t)m0 * K;
  const BT* b_base = B + (size_t)n0 * K;
  const int a_rows = M - m0 < kDBM ? M - m0 : kDBM;  // rows past M / N re-read the last valid row
  const int b_rows = N - n0 < kDBN ? N - n0 : kDBN;
  const int nk = K / kDBK;

  u32x4 ra[DTile<AT>::kLoads], rb[DTile<BT>::kLoads];
  float16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = float16v{};

  DTile<AT>::load(a_base, (size_t)K, a_rows, tid, 0, ra);
  DTile<BT>::load(b_base, (size_t)K, b_rows, tid, 0, rb);
  DTile<AT>::store(lds, tid, ra);
  DTile<BT>::store(lds + kDBM * kDBK, tid, rb);
  __syncthreads();

  for (int ks = 0; ks < nk; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < nk) {
      DTile<AT>::load(a_base, (size_t)K, a_rows, tid, ks + 1, ra);
      DTile<BT>::load(b_base, (size_t)K, b_rows, tid, ks + 1, rb);
    }
    const float* As = lds + cur * kDStage;
    const float* Bs = As + kDBM * kDBK;
    float16v av[2], bv[2];  // 16 consecutive k of the lane's row
#pragma unroll
    for (int i = 0; i < 2; ++i) {
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
    for (int j = 0; j < 2; ++j) {
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
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], bv[j][s], acc[i][j], 0, 0, 0);
    if (ks + 1 < nk) {
      float* nxt = lds + (cur ^ 1) * kDStage;
      DTile<AT>::store(nxt, tid, ra);
      DTile<BT>::store(nxt + kDBM * kDBK, tid, rb);
    }
    __syncthreads();
  }

  // accumulator r of lane l in tile (i, j): row (r/4)*8 + (l/32)*4 + r%4, col l%32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int gn = n0 + wn + 32 * j + r32;
      if (gn >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = m0 + wm + 32 * i + (r >> 2) * 8 + kb * 4 + (r & 3);
        if (gm < M) C[(size_t)gm * N + gn] = (CT)acc[i][j][r];
      }
    }
}

template <typename AT, typename BT>
hipError_t dense_f32_launch(nfhip::EType c, const void* A, const void* B, void* C, uint32_t M, uint32_t N,
                            uint32_t K, hipStream_t s) {
  const long tiles = (long)((M + kDBM - 1) / kDBM) * ((N + kDBN - 1) / kDBN);
  if (tiles > (1L << 31) - 1) return hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)tiles), block(256);
  if (c == nfhip::EType::F32)
    dense_f32_mfma_kernel<AT, BT, float><<<grid, block, 0, s>>>(static_cast<const AT*>(A), static_cast<const BT*>(B),
                                                                static_cast<float*>(C), (int)M, (int)N, (int)K);
  else
    dense_f32_mfma_kernel<AT, BT, half_t><<<grid, block, 0, s>>>(static_cast<const AT*>(A), static_cast<const BT*>(B),
                                                                 static_cast<half_t*>(C), (int)M, (int)N, (int)K);
  return hipGetLastError();
}

}  // namespace

}  // namespace nfk

namespace nfhip {

hipError_t launch_dense_mfma_f32(EType a, EType b, EType c, const void* A, const void* B, void* C, uint32_t M,
                                 uint32_t N, uint32_t K, hipStream_t s) {
  if (K % nfk::kDBK != 0 || (uintptr_t)A % 16 != 0 || (uintptr_t)B % 16 != 0 || M == 0 || N == 0)
    return hipErrorNotSupported;
  if (a == EType::F32)
    return b == EType::F32 ? nfk::dense_f32_launch<float, float>(c, A, B, C, M, N, K, s)
                           : nfk::dense_f32_launch<float, nfk::half_t>(c, A, B, C, M, N, K, s);
  return b == EType::F32 ? nfk::dense_f32_launch<nfk::half_t, float>(c, A, B, C, M, N, K, s)
                         : nfk::dense_f32_launch<nfk::half_t, nfk::half_t>(c, A, B, C, M, N, K, s);
}

}  // namespace nfhip
