// generic.hip — fallback kernels that are correct for any shape.
//
//  * generic fused dequant+linear for K % 32 != 0: the reference indexes
//    weight element (n, k) by its flat position n*K + k, so rows may straddle
//    blocks (metal_provider.mm:1413-1420).  One thread per output element.
//  * dense linear C = A * B^T with B stored [N, K]
//    (metal_provider.mm:150-164, 899-935, 1152-1178), any mix of f32/f16
//    operands, fp32 accumulation: an HBM-bound GEMV for M <= 8, the tiled
//    MFMA kernel for f16 x f16 -> f16 (gemm.hip), else 16x16 LDS tiles.
#include <type_traits>

#include "../launch.hpp"
#include "common.hpp"

namespace nfk {

template <class QF, typename AT>
__global__ __launch_bounds__(256) void generic_fused_kernel(const AT* __restrict__ A,
                                                            const uint8_t* __restrict__ W,
                                                            AT* __restrict__ C, int M, int N,
                                                            int K) {
  constexpr bool kHalfW = sizeof(AT) == 2;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y;
  if (n >= N || m >= M) return;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) {
    const uint64_t e = (uint64_t)n * K + k;
    const uint8_t* blk = W + (e >> 5) * QF::kBytes;
    float w = h2f_bits(*reinterpret_cast<const uint16_t*>(blk)) * (float)code_of<QF>(blk, (int)(e & 31));
    if constexpr (kHalfW) w = (float)(half_t)w;
    acc = __builtin_fmaf((float)A[(size_t)m * K + k], w, acc);
  }
  C[(size_t)m * N + n] = (AT)acc;
}

template <typename AT, typename BT, typename CT>
__global__ __launch_bounds__(256) void dense_kernel(const AT* __restrict__ A,
                                                    const BT* __restrict__ B,
                                                    CT* __restrict__ C, int M, int N, int K) {
  __shared__ float As[16][17];
  __shared__ float Bs[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int row = blockIdx.y * 16 + ty;
  const int col = blockIdx.x * 16 + tx;
  const int bn = blockIdx.x * 16 + ty;  // B row loaded by this thread
  float acc = 0.f;
  for (int t = 0; t < K; t += 16) {
    As[ty][tx] = (row < M && t + tx < K) ? (float)A[(size_t)row * K + t + tx] : 0.f;
    Bs[ty][tx] = (bn < N && t + tx < K) ? (float)B[(size_t)bn * K + t + tx] : 0.f;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) acc = __builtin_fmaf(As[ty][k], Bs[tx][k], acc);
    __syncthreads();
  }
  if (row < M && col < N) C[(size_t)row * N + col] = (CT)acc;
}

// ---- dense decode GEMV (M <= 8): C[m, n] = sum_k A[m, k] * B[n, k] -------
//
// HBM-bound on B.  A wave owns RW consecutive rows of B and sweeps K with
// contiguous 16-byte loads (64 lanes x 16 B = one 1 KB stretch of a row per
// instruction); the activation chunk at the same k is loaded once per wave
// and used for all RW rows and M activation rows.  Partial sums are kept
// per lane in fp32 and reduced across the wave with DPP at the end.  Four
// chunks per lane are in flight per step.

template <typename T> struct Vec16;
template <> struct Vec16<float> {
  typedef float4v V;
  static constexpr int kN = 4;
};
template <> struct Vec16<half_t> {
  typedef half8 V;
  static constexpr int kN = 8;
};

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dense_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xF, false));
}

// Sum over the 64 lanes with DPP; the total lands in lane 63.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dense_dpp<0xB1>(v);           // quad_perm [1,0,3,2]
  v += dense_dpp<0x4E>(v);           // quad_perm [2,3,0,1]
  v += dense_dpp<0x141>(v);          // row_half_mirror
  v += dense_dpp<0x140>(v);          // row_mirror
  v += dense_dpp<0x142, 0xA>(v);     // row_bcast15
  v += dense_dpp<0x143, 0xC>(v);     // row_bcast31
  return v;
}

template <typename T>
__device__ __forceinline__ float lane_dot(const typename Vec16<T>::V& a, const typename Vec16<T>::V& b, float acc) {
  if constexpr (sizeof(T) == 4) {
    acc = __builtin_fmaf(a[0], b[0], acc);
    acc = __builtin_fmaf(a[1], b[1], acc);
    acc = __builtin_fmaf(a[2], b[2], acc);
    acc = __builtin_fmaf(a[3], b[3], acc);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i += 2)
      acc = __builtin_amdgcn_fdot2(half2v{a[i], a[i + 1]}, half2v{b[i], b[i + 1]}, acc, false);
  }
  return acc;
}

// Element type of the K sweep: both operands are converted to it before
// the multiply-add (f32 if either operand is f32).
template <typename AT, typename BT, typename CT, int MM, int RW>
__global__ __launch_bounds__(256) void dense_gemv_kernel(const AT* __restrict__ A, const BT* __restrict__ B,
                                                         CT* __restrict__ C, int M, int N, int K) {
  constexpr bool kF16 = sizeof(AT) == 2 && sizeof(BT) == 2;
  typedef typename std::conditional<kF16, half_t, float>::type ET;
  constexpr int EN = Vec16<ET>::kN;       // elements per 16-byte chunk of the sweep type
  typedef typename Vec16<ET>::V EV;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r0 = (blockIdx.x * 4 + wave) * RW;
  if (r0 >= N) return;
  float acc[RW][MM];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;
  const BT* brow[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) brow[r] = B + (size_t)(r0 + r < N ? r0 + r : N - 1) * K;

  auto load = [&](const auto* p, int k) -> EV {
    typedef typename std::remove_cv<typename std::remove_pointer<decltype(p)>::type>::type ST;
    EV v;
    if constexpr (sizeof(ST) == sizeof(ET)) {
      v = *reinterpret_cast<const EV*>(p + k);
    } else {
#pragma unroll
      for (int i = 0; i < EN; ++i) v[i] = (ET)p[k + i];
    }
    return v;
  };
  const int step = 64 * EN;
  int k = lane * EN;
  // main sweep: four chunks per lane per iteration
  for (; k + 3 * step < K - (K % EN); k += 4 * step) {
    EV bv[4][RW], av[4][MM];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int r = 0; r < RW; ++r) bv[u][r] = load(brow[r], k + u * step);
#pragma unroll
      for (int m = 0; m < MM; ++m) av[u][m] = load(A + (size_t)(m < M ? m : 0) * K, k + u * step);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m) acc[r][m] = lane_dot<ET>(av[u][m], bv[u][r], acc[r][m]);
  }
  for (; k + EN <= K; k += step) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const EV bv = load(brow[r], k);
#pragma unroll
      for (int m = 0; m < MM; ++m) acc[r][m] = lane_dot<ET>(load(A + (size_t)(m < M ? m : 0) * K, k), bv, acc[r][m]);
    }
  }
  // ragged tail (K % EN != 0): lane 0 takes the last elements one by one
  if (lane == 0) {
    for (int kk = K - (K % EN); kk < K; ++kk)
#pragma unroll
      for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m)
          acc[r][m] = __builtin_fmaf((float)A[(size_t)(m < M ? m : 0) * K + kk], (float)brow[r][kk], acc[r][m]);
  }
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float v = wave_sum_dpp(acc[r][m]);
      if (lane == 63 && r0 + r < N && m < M) C[(size_t)m * N + r0 + r] = (CT)v;
    }
}

template <typename AT, typename BT, typename CT>
hipError_t dense_gemv(const void* A, const void* B, void* C, uint32_t M, uint32_t N, uint32_t K, hipStream_t s) {
  constexpr int RW = 2;
  const dim3 grid((N + 4 * RW - 1) / (4 * RW));
  const AT* a = static_cast<const AT*>(A);
  const BT* b = static_cast<const BT*>(B);
  CT* c = static_cast<CT*>(C);
  if (M == 1) dense_gemv_kernel<AT, BT, CT, 1, RW><<<grid, dim3(256), 0, s>>>(a, b, c, M, N, K);
  else if (M == 2) dense_gemv_kernel<AT, BT, CT, 2, RW><<<grid, dim3(256), 0, s>>>(a, b, c, M, N, K);
  else if (M <= 4) dense_gemv_kernel<AT, BT, CT, 4, RW><<<grid, dim3(256), 0, s>>>(a, b, c, M, N, K);
  else dense_gemv_kernel<AT, BT, CT, 8, RW><<<grid, dim3(256), 0, s>>>(a, b, c, M, N, K);
  return hipGetLastError();
}

template <typename AT, typename BT>
hipError_t dense_gemv_c(nfhip::EType c, const void* A, const void* B, void* C, uint32_t M, uint32_t N, uint32_t K,
                        hipStream_t s) {
  return c == nfhip::EType::F32 ? dense_gemv<AT, BT, float>(A, B, C, M, N, K, s)
                                : dense_gemv<AT, BT, half_t>(A, B, C, M, N, K, s);
}

template <typename AT, typename BT>
hipError_t dense_c(nfhip::EType c, const void* A, const void* B, void* C, uint32_t M, uint32_t N,
                   uint32_t K, hipStream_t s) {
  const dim3 block(256);
  const dim3 grid((N + 15) / 16, (M + 15) / 16);
  if (grid.y > 65535) return hipErrorInvalidConfiguration;
  if (c == nfhip::EType::F32)
    dense_kernel<AT, BT, float><<<grid, block, 0, s>>>((const AT*)A, (const BT*)B, (float*)C, M, N, K);
  else
    dense_kernel<AT, BT, half_t><<<grid, block, 0, s>>>((const AT*)A, (const BT*)B, (half_t*)C, M, N, K);
  return hipGetLastError();
}

}  // namespace nfk

namespace nfhip {

hipError_t launch_generic(QFmt q, EType t, const void* A, const void* W, void* C, uint32_t M,
                          uint32_t N, uint32_t K, hipStream_t s) {
  const dim3 block(256);
  const dim3 grid((N + 255) / 256, M);
  if (M > 65535) return hipErrorInvalidConfiguration;
  const uint8_t* w = static_cast<const uint8_t*>(W);
  if (q == QFmt::Q4_0) {
    if (t == EType::F32)
      nfk::generic_fused_kernel<nfk::Q4_0, float><<<grid, block, 0, s>>>((const float*)A, w, (float*)C, M, N, K);
    else
      nfk::generic_fused_kernel<nfk::Q4_0, nfk::half_t><<<grid, block, 0, s>>>((const nfk::half_t*)A, w, (nfk::half_t*)C, M, N, K);
  } else {
    if (t == EType::F32)
      nfk::generic_fused_kernel<nfk::Q8_0, float><<<grid, block, 0, s>>>((const float*)A, w, (float*)C, M, N, K);
    else
      nfk::generic_fused_kernel<nfk::Q8_0, nfk::half_t><<<grid, block, 0, s>>>((const nfk::half_t*)A, w, (nfk::half_t*)C, M, N, K);
  }
  return hipGetLastError();
}

hipError_t launch_dense(EType a, EType b, EType c, const void* A, const void* B, void* C,
                        uint32_t M, uint32_t N, uint32_t K, const Workspace& ws, hipStream_t s) {
  // Decode-sized batches: the HBM-bound dense GEMV (16-byte aligned rows).
  const size_t ea = a == EType::F16 ? 2 : 4, eb = b == EType::F16 ? 2 : 4;
  if (M <= 8 && (uintptr_t)A % 16 == 0 && (uintptr_t)B % 16 == 0 && (K * ea) % 16 == 0 && (K * eb) % 16 == 0) {
    if (a == EType::F32)
      return b == EType::F32 ? nfk::dense_gemv_c<float, float>(c, A, B, C, M, N, K, s)
                             : nfk::dense_gemv_c<float, nfk::half_t>(c, A, B, C, M, N, K, s);
    return b == EType::F32 ? nfk::dense_gemv_c<nfk::half_t, float>(c, A, B, C, M, N, K, s)
                           : nfk::dense_gemv_c<nfk::half_t, nfk::half_t>(c, A, B, C, M, N, K, s);
  }
  // fp16 x fp16 with enough rows for MFMA tiles: the tiled fp16 MFMA kernel
  // (fp32 accumulation; fp16 or fp32 output).
  if (a == EType::F16 && b == EType::F16 && M >= 32 && K % 64 == 0 && (uintptr_t)A % 16 == 0 &&
      (uintptr_t)B % 16 == 0)
    return launch_dense_mfma_f16(A, B, C, M, N, K, c == EType::F32, s);
  // Every other dtype mix (fp32 operands, or an fp32 output) on the fp32
  // MFMA, fp16 operands widened exactly; the VALU tile kernel below takes
  // K % 32 != 0 and misaligned buffers.
  {
    const hipError_t e = launch_dense_mfma_f32(a, b, c, A, B, C, M, N, K, ws, s);
    if (e != hipErrorNotSupported) return e;
  }
  if (a == EType::F32) {
    return b == EType::F32 ? nfk::dense_c<float, float>(c, A, B, C, M, N, K, s)
                           : nfk::dense_c<float, nfk::half_t>(c, A, B, C, M, N, K, s);
  }
  return b == EType::F32 ? nfk::dense_c<nfk::half_t, float>(c, A, B, C, M, N, K, s)
                         : nfk::dense_c<nfk::half_t, nfk::half_t>(c, A, B, C, M, N, K, s);
}

}  // namespace nfhip
